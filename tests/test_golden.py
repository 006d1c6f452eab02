"""The oracle against vectors of the reference's own CPU references.

tests/golden/reference_vectors.npz holds outputs of the reference's
direct_bf16_pv and tiled_bf16_pv (tests/paged_attention_reference.py:6-59),
direct_tiled (tests/paged_attention_reference_test.py:8-28) and direct_bf16
(tests/fp64_reference.py:7-29), written by tests/golden/make_reference_vectors.py.
Where the oracle's fp32 arithmetic and torch's (its vectorised exp, its
reduction order) round one probability, or an output's fp32 sum, to a
different value, an output moves by about one bf16 step of a probability
times |v|: such elements are counted and bounded (max-abs 2e-3, mean-abs 2e-6
over the output, a thousandth of the parity gate's mean); the cases the
reference's own tests use match bit for bit.
"""

import hashlib
import pathlib

import numpy as np
import pytest

from oracle import oracle as orc
from tests import paged_cases as cases

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"
# A probability rounding flip moves an output by about 2^-9 * p * |v| <= ~1e-3 at these sizes.
FLIP_ABS, FLIP_MEAN = 2e-3, 2e-6


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as g:
        return {k: g[k] for k in g.files}


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def compare(name, mine, ref, exact=False):
    assert mine.shape == ref.shape and mine.dtype == ref.dtype == np.uint16
    diff = np.abs(orc.bf16_to_f32(mine).astype(np.float64) - orc.bf16_to_f32(ref).astype(np.float64))
    flips = int((mine != ref).sum())
    print(f"{name}: {flips} of {mine.size} elements differ, max_abs={diff.max():.3e} mean_abs={diff.mean():.2e}",
          flush=True)
    if exact:
        assert flips == 0, name
    else:
        assert diff.max() <= FLIP_ABS and diff.mean() <= FLIP_MEAN, name


def reftest_problem(g):
    pool = np.stack([g["reftest_keys"].transpose(1, 0, 2), g["reftest_values"].transpose(1, 0, 2)])
    positions = g["reftest_positions"].astype(np.int64)
    return orc.Problem(g["reftest_query"], pool, np.zeros(len(positions), dtype=np.int64), positions,
                       g["reftest_mapping"], 4, 2, 4, 0.5)


def test_reference_test_inputs_bit_exact(golden):
    p = reftest_problem(golden)
    compare("direct_bf16_pv", orc.direct_bf16_pv(p), golden["reftest_direct"], exact=True)
    for tile in (2, 3, 5, 16):
        compare(f"tiled_bf16_pv tile {tile}", orc.tiled_bf16_pv(p, tile), golden[f"reftest_tiled_{tile}"],
                exact=True)
        compare(f"direct_tiled tile {tile}", orc.direct_tiled(p, tile), golden[f"reftest_direct_tiled_{tile}"],
                exact=True)


def test_reference_tiled_forms_agree_only_to_the_tiled_gate(golden):
    # tests/paged_attention_reference_test.py:48-50 asserts tiled_bf16_pv == direct_tiled
    # bitwise. The reference's own functions, under the torch that wrote the vectors,
    # differ by a few bf16 ulp (probabilities normalised before vs after the bf16
    # rounding); both stay within the reference's tiled gate of 5e-3 relative L2
    # (tests/paged_attention_reference.py:68), the bound the oracle tests use.
    worst = 0.0
    for tile in (2, 3, 5, 16):
        a = orc.bf16_to_f32(golden[f"reftest_tiled_{tile}"]).astype(np.float64)
        b = orc.bf16_to_f32(golden[f"reftest_direct_tiled_{tile}"]).astype(np.float64)
        rel = np.linalg.norm(a - b, axis=-1) / np.linalg.norm(b, axis=-1)
        worst = max(worst, float(rel.max()))
    print(f"torch {golden['torch_version']}: tiled vs direct_tiled worst relative L2 {worst:.2e}")
    assert worst <= 5e-3


def test_c1_decode(golden):
    c1 = cases.c1_case()
    assert digest(c1.query, c1.pool, c1.block_tables, c1.lens) == str(golden["c1_input_sha256"])
    p = c1.oracle_problem()
    compare("c1 direct_bf16_pv", orc.direct_bf16_pv(p), golden["c1_direct"], exact=True)
    compare("c1 tiled_bf16_pv 512", orc.tiled_bf16_pv(p, 512), golden["c1_tiled_512"], exact=True)
    compare("c1 tiled_bf16_pv 64", orc.tiled_bf16_pv(p, 64), golden["c1_tiled_64"])


def test_prefill_chunk(golden):
    pf = golden_prefill_case()
    assert digest(pf.query, pf.pool, pf.block_tables) == str(golden["prefill_input_sha256"])
    p = pf.oracle_problem()
    compare("prefill direct_bf16_pv", orc.direct_bf16_pv(p), golden["prefill_direct"])
    compare("prefill tiled_bf16_pv 512", orc.tiled_bf16_pv(p, 512), golden["prefill_tiled_512"])
    compare("prefill tiled_bf16_pv 64", orc.tiled_bf16_pv(p, 64), golden["prefill_tiled_64"])


def test_long_prefill_rows(golden):
    # A 3840-token prefix and 263 chunk rows: many 512-key tiles per row, the rows
    # on both sides of every 32-row boundary.
    lc = golden_long_case()
    assert digest(lc.query, lc.pool, lc.block_tables) == str(golden["long_input_sha256"])
    p = lc.oracle_problem(rows=golden["long_rows"])
    compare("long direct_bf16_pv", orc.direct_bf16_pv(p), golden["long_direct"])
    compare("long tiled_bf16_pv 512", orc.tiled_bf16_pv(p, 512), golden["long_tiled_512"])


def test_long_decode(golden):
    # C5's group at contexts up to 32768 keys.
    dl = golden_long_decode_case()
    assert digest(dl.query, dl.pool, dl.block_tables, dl.lens) == str(golden["decode_long_input_sha256"])
    p = dl.oracle_problem()
    compare("long decode direct_bf16_pv", orc.direct_bf16_pv(p), golden["decode_long_direct"])
    compare("long decode tiled_bf16_pv 512", orc.tiled_bf16_pv(p, 512), golden["decode_long_tiled_512"])


def test_fp64_to_bf16_rounding_bit_exact(golden):
    mine = orc.bf16_from_f64(golden["round_inputs"])
    assert np.array_equal(mine, golden["round_bits"])


def golden_long_decode_case():
    """The long decode case of the vectors: 16 q / 2 kv heads, d 128, block 128, contexts 32768, 20000, 777."""
    return cases.decode_case(53, 3, 16, 2, 128, 128, 420, [32768, 20000, 777])


def golden_long_case():
    """The long case of the vectors: 14 q / 2 kv heads, d 64, block 16, a 3840-token prefix + 263 rows."""
    return cases.PrefillCase(47, 14, 2, 64, 16, prefixes=[3840], chunks=[263])


def golden_prefill_case():
    """The prefill case of the vectors: 14 q / 2 kv heads, d 64, block 16, a 300-token prefix + 9 rows, 7 rows."""
    return cases.PrefillCase(31, 14, 2, 64, 16, prefixes=[300, 0], chunks=[9, 7])
