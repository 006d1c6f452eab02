"""Writes tests/golden/reference_vectors.npz: the reference's own CPU references
evaluated on seeded inputs, for the oracle and the GPU path to be checked against.

Functions evaluated (all from the reference checkout, imported from its tests/
directory with bytecode writing off; nothing of it is copied or kept):
  tests/paged_attention_reference.py:6-22       direct_bf16_pv
  tests/paged_attention_reference.py:25-59      tiled_bf16_pv
  tests/paged_attention_reference_test.py:8-28  direct_tiled
  tests/fp64_reference.py:7-29                  direct_bf16 (fp64 -> bf16, round to nearest even)

Cases:
  reftest  the inputs of tests/paged_attention_reference_test.py:39-50 (torch seed 771,
           4 q / 2 kv heads, d 4, positions 1, 7, 11), tiles 2, 3, 5, 16; the inputs are
           stored with the outputs.
  c1       tests/paged_cases.c1_case() (workload C1: 4 decode rows, 8 q / 2 kv heads, d 128,
           block 128); kv tiles 512 (the reference harness's tile) and 64.
  prefill  tests/paged_cases.PrefillCase(31, 14, 2, 64, 16, prefixes=[300, 0], chunks=[9, 7])
           (the reference's multi-tile geometry, 14 q / 2 kv heads, d 64), kv tiles 512 and 64.
  long     the reference's multi-tile geometry at its first long case
           (tests/multitile_paged_attention_unit_test.cpp:1642-1655: 3840 + 263): 14 q / 2 kv heads,
           d 64, block 16, inputs from tests/paged_cases.PrefillCase(47, ...); outputs of the rows
           at every 32-row boundary (long_rows) only, to keep the file small.
  decode_long  decode rows at C5's group (16 q / 2 kv heads, d 128, block 128) with contexts
           32768, 20000 and 777: tests/paged_cases.decode_case(53, ...); kv tile 512.
  round    direct_bf16 on edge values (ties, the bf16 subnormal range, overflow) and on
           seeded random doubles over the whole exponent range.
The c1, prefill, long and decode_long inputs are regenerated from their seeds by the tests; a SHA-256
of their bits is stored to catch a generator that drifts.

Run from the repository root, in a container that holds the reference checkout:
    python tests/golden/make_reference_vectors.py /root/reference
"""

import hashlib
import pathlib
import sys

sys.dont_write_bytecode = True

import numpy as np  # noqa: E402
import torch  # noqa: E402

ROOT = pathlib.Path(__file__).resolve().parents[2]
# Rows of the long case kept: both sides of every 32-row boundary, and the last row.
LONG_ROWS = np.array(sorted({r for k in range(0, 263, 32) for r in (k - 1, k) if 0 <= r < 263} | {262}),
                     dtype=np.int64)
OUT = pathlib.Path(__file__).resolve().parent / "reference_vectors.npz"


def bits(t):
    """bf16-valued tensor (any float dtype) -> uint16 bits."""
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_tensor(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def reference_args(case, requests, positions):
    """The reference functions' arguments: slot-major pools [S, Hkv, d], mapping [requests, context]."""
    from oracle import oracle as orc
    context = int(np.max(positions)) + 1
    mapping = orc.mapping_from_block_table(case.block_tables, case.block_size, context)
    return (bf16_tensor(case.query), bf16_tensor(case.pool[0].transpose(1, 0, 2)),
            bf16_tensor(case.pool[1].transpose(1, 0, 2)), torch.as_tensor(np.asarray(requests, dtype=np.int64)),
            torch.as_tensor(np.asarray(positions, dtype=np.int64)), torch.as_tensor(mapping.astype(np.int64)),
            case.heads, case.kv_heads, case.head_dim, case.scale)


def rounding_inputs():
    edge = [0.0, 1.0, -1.0, 1 + 2.0**-8, 1 + 3 * 2.0**-8, 1 + 2.0**-8 + 2.0**-32, 1 + 2.0**-8 - 2.0**-40,
            -(1 + 2.0**-8), 2.0**-126, 2.0**-127, 2.0**-130 * 1.5, 2.0**-133, 2.0**-134, 2.0**-133 * 0.5,
            2.0**-133 * 1.5, 2.0**-133 * 2.5, 2.0**-126 * (1 - 2.0**-9), 3.3895313892515355e38,
            3.3895313892515355e38 * (1 + 2.0**-9), 3.3961e38, 2.0**127, -(2.0**127) * 1.999, 1e-45, -1e-40]
    rng = np.random.default_rng(20261203)
    mant = rng.uniform(1.0, 2.0, 2000)
    expo = rng.integers(-140, 128, 2000)
    sign = rng.choice([-1.0, 1.0], 2000)
    rand = sign * np.ldexp(mant, expo)
    # exact ties between neighbouring bf16 values, with both parities
    ties = np.ldexp(1.0 + (2 * rng.integers(0, 128, 200) + 1) * 2.0**-8, rng.integers(-120, 120, 200))
    return np.concatenate([np.asarray(edge, dtype=np.float64), rand, ties])


def main():
    ref = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference").resolve() / "tests"
    sys.path.insert(0, str(ref))
    sys.path.insert(0, str(ROOT))
    from paged_attention_reference import direct_bf16_pv, tiled_bf16_pv
    from paged_attention_reference_test import direct_tiled
    from fp64_reference import direct_bf16
    from tests import paged_cases as cases

    out = {}
    # reftest: the reference test's own inputs and settings
    torch.set_num_threads(2)
    torch.manual_seed(771)
    heads, kv_heads, d = 4, 2, 4
    query = torch.randn(3, heads * d).bfloat16()
    keys = torch.randn(13, kv_heads, d).bfloat16()
    values = torch.randn_like(keys).bfloat16()
    mapping = torch.tensor([[9, 2, 11, 5, 3, 10, 6, 1, 12, 4, 8, 7]], dtype=torch.int64)
    requests = torch.tensor([0, 0, 0])
    positions = torch.tensor([1, 7, 11])
    args = (query, keys, values, requests, positions, mapping, heads, kv_heads, d, 0.5)
    out["reftest_query"], out["reftest_keys"], out["reftest_values"] = bits(query), bits(keys), bits(values)
    out["reftest_mapping"], out["reftest_positions"] = mapping.numpy().astype(np.int32), positions.numpy()
    out["reftest_direct"] = bits(direct_bf16_pv(*args))
    for tile in (2, 3, 5, 16):
        out[f"reftest_tiled_{tile}"] = bits(tiled_bf16_pv(*args, tile))
        out[f"reftest_direct_tiled_{tile}"] = bits(direct_tiled(*args, tile))

    # c1: decode rows (position = length - 1)
    c1 = cases.c1_case()
    out["c1_input_sha256"] = np.array(digest(c1.query, c1.pool, c1.block_tables, c1.lens))
    a = reference_args(c1, np.arange(c1.batch), c1.lens.astype(np.int64) - 1)
    out["c1_direct"] = bits(direct_bf16_pv(*a))
    for tile in (512, 64):
        out[f"c1_tiled_{tile}"] = bits(tiled_bf16_pv(*a, tile))

    # prefill: chunk rows after a cached prefix, causal
    pf = cases.PrefillCase(31, 14, 2, 64, 16, prefixes=[300, 0], chunks=[9, 7])
    out["prefill_input_sha256"] = np.array(digest(pf.query, pf.pool, pf.block_tables))
    a = reference_args(pf, pf.requests, pf.positions)
    out["prefill_direct"] = bits(direct_bf16_pv(*a))
    for tile in (512, 64):
        out[f"prefill_tiled_{tile}"] = bits(tiled_bf16_pv(*a, tile))

    # long: 3840-token prefix + 263 rows, rows at the 32-row boundaries
    lc = cases.PrefillCase(47, 14, 2, 64, 16, prefixes=[3840], chunks=[263])
    out["long_input_sha256"] = np.array(digest(lc.query, lc.pool, lc.block_tables))
    rows = LONG_ROWS
    out["long_rows"] = rows
    a = reference_args(lc, lc.requests, lc.positions)
    a = (a[0][rows],) + a[1:3] + (a[3][rows], a[4][rows]) + a[5:]
    out["long_direct"] = bits(direct_bf16_pv(*a))
    out["long_tiled_512"] = bits(tiled_bf16_pv(*a, 512))

    # decode_long: one row at 32768 keys, split over many workgroups by the balanced decode
    dl = cases.decode_case(53, 3, 16, 2, 128, 128, 420, [32768, 20000, 777])
    out["decode_long_input_sha256"] = np.array(digest(dl.query, dl.pool, dl.block_tables, dl.lens))
    a = reference_args(dl, np.arange(dl.batch), dl.lens.astype(np.int64) - 1)
    out["decode_long_direct"] = bits(direct_bf16_pv(*a))
    out["decode_long_tiled_512"] = bits(tiled_bf16_pv(*a, 512))

    # round: direct fp64 -> bf16
    values64 = rounding_inputs()
    out["round_inputs"] = values64
    out["round_bits"] = bits(direct_bf16(torch.from_numpy(values64)))

    out["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, sum(v.nbytes for v in out.values()), "bytes uncompressed")


if __name__ == "__main__":
    main()
