"""GPU ports of the reference's standalone device tests of the path, through the C ABI.

- tests/fixed_kv_descriptor_device_test.cpp: the KV store of a 256-row bucket
  (head_dim 128, 8 kv heads) whose 137 valid rows target slots slots-1, 1, 3,
  5, ... and whose tail points one past the pool, stored with 1, 7 and 137
  valid rows; every pool byte, guards around the pool, and a gather of six pool
  rows after the write are checked;
- tests/fused_paged_decode_device_test.cpp: decode with the new rows' K/V
  stored by the same call (gk_paged_decode's fused store) over one request's
  slot sequence, including the last physical page; padded query rows (here:
  rows with no keys and a negative slot) come back as +0;
- tests/fixed_tile_paged_attention_device_test.cpp: a chunk of query rows
  (one or several query blocks) over several key tiles: the store, then
  gk_paged_prefill.

Each case audits the whole pool bit for bit and its guards, and gates the
output three ways: the flat gate against the oracle's direct_bf16_pv (max-abs
2e-2, mean-abs 2e-3), and the relative-L2 gates: 1e-2 against the fp64 truth
rounded once to bf16, as in the device tests
(tests/fused_paged_decode_device_test.cpp:458,
fixed_tile_paged_attention_device_test.cpp:686), and 5e-3 against the tiled
emulation with bf16 probabilities, the gate of
tests/paged_attention_reference.py:60-69. The device tests hold the tiled
error to 1e-3, which pins the Gaudi kernels' own rounding order (each tile's
probabilities normalised, then rounded to bf16): on these inputs the oracle's
direct_bf16_pv, the reference's own single-pass form, is 2.6e-3 to 3.9e-3 from
that emulation, and an fp32-softmax form 2.5e-3 to 3.2e-3. The HIP kernels
measure 2.4e-3 to 3.3e-3 against the fp64 truth and 3.1e-3 to 3.8e-3 against
the tiled emulation on these cases. The inputs follow the
reference's construction (slot formulas, N(0, 0.6) bf16 values, sentinels
0x3e80 / 0x3f00, guard 0x4110); the random values come from torch's generator,
not from the reference's mt19937. Recipe-cache counters and device timing have
no counterpart here.
"""

import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GUARD, KEY_SENTINEL, VALUE_SENTINEL = 0x4110, 0x3E80, 0x3F00


@pytest.fixture(scope="module")
def runner():
    import torch
    assert torch.cuda.is_available()
    from tests import gk_runner
    return gk_runner


def normal_bits(gen, shape):
    import torch
    return (torch.randn(shape, generator=gen) * 0.6).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def slot_sequence(n, slots, page):
    """Slot of key i: tests/fused_paged_decode_device_test.cpp:159-163."""
    i = np.arange(n, dtype=np.int64)
    if page == 1:
        return (1 + (i * 5) % (slots - 1)).astype(np.int32)
    return ((1 + ((i // page) * 5) % (slots // page - 1)) * page + i % page).astype(np.int32)


def block_table(keys, page):
    """Block table of a page-contiguous slot sequence (block_size = page)."""
    n = len(keys)
    table = keys[::page] // page
    assert np.array_equal(table.repeat(page)[:n] * page + np.arange(n) % page, keys), "not page contiguous"
    return table.astype(np.int32).reshape(1, -1)


def guarded_pool(runner, kv_heads, slots, head_dim, fill=None):
    """A pool inside one buffer with 128 guard elements either side; returns (flat, pool view, initial bits)."""
    half = kv_heads * slots * head_dim
    bits = np.empty(2 * half + 256, dtype=np.uint16)
    bits[:128] = bits[-128:] = GUARD
    bits[128:128 + half] = KEY_SENTINEL
    bits[128 + half:-128] = VALUE_SENTINEL
    if fill is not None:
        bits[128:-128] = fill.reshape(-1)
    flat = runner.bf16_device(bits)
    return flat, flat[128:-128].view(2, kv_heads, slots, head_dim), bits


def check_pool(runner, flat, expected_pool):
    got = runner.bits_of(flat)
    assert (got[:128] == GUARD).all() and (got[-128:] == GUARD).all(), "a guard around the pool changed"
    assert np.array_equal(got[128:-128], expected_pool.reshape(-1)), "KV write corrupted a target or untouched slot"


def gate(actual, problem, kv_tile):
    """Flat gate against direct_bf16_pv, then the device tests' relative-L2 gates."""
    assert np.isfinite(orc.bf16_to_f32(actual)).all(), "nonfinite attention output"
    flat = orc.check_flat_gate(actual, orc.direct_bf16_pv(problem))
    tiled = orc.tiled_bf16_pv(problem, kv_tile)
    rel = orc.isolated_errors(orc.bf16_to_f32(actual), orc.fp64_bf16(problem), orc.bf16_to_f32(tiled))
    return flat, rel


@pytest.mark.parametrize("slots", [512, 8192])
def test_fixed_kv_descriptor(runner, slots):
    # tests/fixed_kv_descriptor_device_test.cpp:76-197
    import torch
    head_dim, kv_heads, bucket, rows = 128, 8, 256, 137
    width = head_dim * kv_heads
    i = np.arange(width * bucket)
    key = (0x3F80 + i % 127).astype(np.uint16).reshape(bucket, width)
    value = (0x4000 + (i * 7) % 127).astype(np.uint16).reshape(bucket, width)
    loc = np.full(bucket, slots, dtype=np.int32)  # the tail points one row past the pool
    loc[0] = slots - 1
    loc[1:rows] = 1 + 2 * np.arange(rows - 1)
    d_key, d_value, d_loc = runner.bf16_device(key), runner.bf16_device(value), runner.to_device(loc)
    gather = np.array([slots - 1, 3 * slots, 7 * slots + 3, kv_heads * slots + slots - 1,
                       (kv_heads + 3) * slots + 3, (kv_heads + 7) * slots + 1], dtype=np.int64)
    for valid in (1, 7, rows):
        flat, pool, initial = guarded_pool(runner, kv_heads, slots, head_dim)
        runner.kv_store(d_key[:valid], d_value[:valid], d_loc[:valid], pool, kv_heads, head_dim)
        gathered = pool.view(-1, head_dim)[torch.from_numpy(gather).cuda()]  # same stream, after the store
        torch.cuda.synchronize()
        expected = initial[128:-128].reshape(2, kv_heads, slots, head_dim).copy()
        expected[0][:, loc[:valid]] = key[:valid].reshape(valid, kv_heads, head_dim).transpose(1, 0, 2)
        expected[1][:, loc[:valid]] = value[:valid].reshape(valid, kv_heads, head_dim).transpose(1, 0, 2)
        check_pool(runner, flat, expected)
        assert np.array_equal(runner.bits_of(gathered), expected.reshape(-1, head_dim)[gather]), \
            "post-write gather mismatch"
        print(f"slots {slots} valid rows {valid}: targets, untouched slots, guards and gather exact", flush=True)


# (head_dim, kv_bucket, q_heads, kv_heads, slots, page, effective_kv, rows, valid)
FUSED_DECODE = [
    (128, 8192, 32, 8, 16384, 16, 8192, 1, 1),
    (64, 512, 14, 2, 2048, 1, 300, 7, 5),
    (128, 4096, 56, 8, 131072, 16, 4000, 1, 1),
    (128, 512, 8, 8, 4096, 16, 512, 256, 200),
    (64, 1024, 16, 4, 2048, 1, 1024, 3, 3),
]


@pytest.mark.parametrize("d,kv,heads,kvh,slots,page,eff,rows,valid", FUSED_DECODE)
def test_fused_paged_decode(runner, d, kv, heads, kvh, slots, page, eff, rows, valid):
    # tests/fused_paged_decode_device_test.cpp:126-212 (construction), :373-458 (gates)
    import torch
    gen = torch.Generator().manual_seed(20261106 + eff + rows)
    width = kvh * d
    q = normal_bits(gen, (rows, heads * d))
    key_new, value_new = normal_bits(gen, (rows, width)), normal_bits(gen, (rows, width))
    keys = np.zeros(kv, dtype=np.int32)
    keys[:eff] = slot_sequence(eff, slots, page)
    target = (eff - 1) // page * page  # include the final physical page, page-contiguous
    hits = np.flatnonzero(keys == slots - page)
    if hits.size == 0:
        keys[target:target + page] = slots - page + np.arange(page)
    else:
        old = int(hits[0])
        moved = keys[target:target + page].copy()
        keys[target:target + page] = keys[old:old + page]
        keys[old:old + page] = moved
    keys = keys[:eff]
    assert len(np.unique(keys)) == eff and (keys == slots - page).any()
    pool = np.empty((2, kvh, slots, d), dtype=np.uint16)
    pool[0], pool[1] = KEY_SENTINEL, VALUE_SENTINEL
    pool[0][:, keys] = normal_bits(gen, (eff, kvh, d)).transpose(1, 0, 2)
    pool[1][:, keys] = normal_bits(gen, (eff, kvh, d)).transpose(1, 0, 2)
    positions = np.arange(rows, dtype=np.int64) + (eff - valid)
    loc = np.full(rows, -1, dtype=np.int32)
    loc[:valid] = keys[positions[:valid]]
    expected = pool.copy()
    expected[0][:, loc[:valid]] = key_new[:valid].reshape(valid, kvh, d).transpose(1, 0, 2)
    expected[1][:, loc[:valid]] = value_new[:valid].reshape(valid, kvh, d).transpose(1, 0, 2)

    flat, d_pool, _ = guarded_pool(runner, kvh, slots, d, fill=pool)
    tables = block_table(keys, page)
    lens = np.where(np.arange(rows) < valid, positions + 1, 0).astype(np.int32)
    scale = float(np.float32(1 / math.sqrt(d)))
    out = torch.full((rows, heads * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    d_q, d_kn, d_vn = runner.bf16_device(q), runner.bf16_device(key_new), runner.bf16_device(value_new)
    # every device input stays referenced until the call has finished
    d_tables, d_lens, d_loc = runner.to_device(tables), runner.to_device(lens), runner.to_device(loc)
    d_req = runner.to_device(np.zeros(rows, np.int32))
    params = runner.decode_params(d_q, d_pool, d_tables, d_lens, heads, kvh, d, page, scale, out, row_request=d_req,
                                  max_context=eff, new_key=d_kn, new_value=d_vn, slot_mapping=d_loc)
    print(f"fused decode d {d} kv {kv} heads {heads}/{kvh} slots {slots} page {page} eff {eff} rows {rows}/{valid}",
          flush=True)
    ws = runner.paged_decode(params)
    torch.cuda.synchronize()
    del ws
    check_pool(runner, flat, expected)
    actual = runner.bits_of(out)
    assert (actual[valid:] == 0).all(), "invalid query row was not zeroed"
    problem = orc.Problem(q[:valid], expected, np.zeros(valid, np.int64), positions[:valid], keys.reshape(1, -1),
                          heads, kvh, d, scale)
    flat_err, rel = gate(actual[:valid], problem, kv)
    print(f"  max/mean abs {flat_err}, relative l2 fp64/tiled {rel}", flush=True)


# (head_dim, q_bucket, valid, kv_tile, q_heads, kv_heads, slots, page, tiles, query_blocks)
FIXED_TILE = [
    (128, 256, 200, 512, 32, 8, 8192, 16, 4, 1),
    (64, 1, 1, 512, 14, 2, 2048, 1, 3, 1),
    (128, 128, 128, 512, 8, 2, 8192, 64, 8, 4),
    (128, 37, 30, 256, 56, 8, 4096, 1, 2, 1),
    (64, 64, 64, 128, 4, 4, 2048, 16, 5, 3),
]


@pytest.mark.parametrize("d,rows,valid,kv,heads,kvh,slots,page,tiles,blocks", FIXED_TILE)
def test_fixed_tile_paged_attention(runner, d, rows, valid, kv, heads, kvh, slots, page, tiles, blocks):
    # tests/fixed_tile_paged_attention_device_test.cpp:146-231 (construction), :592-686 (gates)
    import torch
    from gaudirt_amd import capi
    gen = torch.Generator().manual_seed(20261106 + rows * tiles + blocks)
    width, total_rows = kvh * d, rows * blocks
    q = normal_bits(gen, (total_rows, heads * d))
    key_new, value_new = normal_bits(gen, (total_rows, width)), normal_bits(gen, (total_rows, width))
    keys = slot_sequence(tiles * kv, slots, page)
    assert len(np.unique(keys)) == len(keys)
    pool = np.empty((2, kvh, slots, d), dtype=np.uint16)
    pool[0], pool[1] = KEY_SENTINEL, VALUE_SENTINEL
    pool[0][:, keys] = normal_bits(gen, (len(keys), kvh, d)).transpose(1, 0, 2)
    pool[1][:, keys] = normal_bits(gen, (len(keys), kvh, d)).transpose(1, 0, 2)
    prefix = tiles * kv - total_rows if blocks > 1 else (tiles - 1) * kv + (kv - 1 if rows == 1 else 0)
    total_valid = total_rows if blocks > 1 else valid
    positions = np.arange(total_valid, dtype=np.int64) + prefix
    loc = keys[positions].astype(np.int32)
    expected = pool.copy()
    expected[0][:, loc] = key_new[:total_valid].reshape(total_valid, kvh, d).transpose(1, 0, 2)
    expected[1][:, loc] = value_new[:total_valid].reshape(total_valid, kvh, d).transpose(1, 0, 2)

    flat, d_pool, _ = guarded_pool(runner, kvh, slots, d, fill=pool)
    # every device input stays referenced until the calls have finished
    d_q, d_kn, d_vn = (runner.bf16_device(x[:total_valid]) for x in (q, key_new, value_new))
    d_loc, d_tables = runner.to_device(loc), runner.to_device(block_table(keys, page))
    d_seq = [runner.to_device(np.array([v], dtype=np.int32)) for v in (0, 0, total_valid, prefix)]
    runner.kv_store(d_kn, d_vn, d_loc, d_pool, kvh, d)
    scale = float(np.float32(1 / math.sqrt(d)))
    out = torch.full((total_valid, heads * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.prefill_params(d_q, d_pool, d_tables, *d_seq, heads, kvh, d, page, scale, out, total_valid)
    print(f"fixed tile d {d} rows {rows}/{valid} kv {kv} heads {heads}/{kvh} slots {slots} page {page} "
          f"tiles {tiles} blocks {blocks}", flush=True)
    capi.check(capi.load().gk_paged_prefill(ctypes.byref(params), capi.current_stream()))
    torch.cuda.synchronize()
    check_pool(runner, flat, expected)
    problem = orc.Problem(q[:total_valid], expected, np.zeros(total_valid, np.int64), positions, keys.reshape(1, -1),
                          heads, kvh, d, scale)
    flat_err, rel = gate(runner.bits_of(out), problem, kv)
    print(f"  max/mean abs {flat_err}, relative l2 fp64/tiled {rel}", flush=True)
