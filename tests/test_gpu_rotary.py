"""GPU parity of the rotary embedding and the fused rotary + KV store.

Follows the reference's rotary smokes: tests/rotary_runtime_smoke.py (56/8 and
4/2 heads, head_dim 128 / 96, rotary_dim 128 / 62, both pair layouts, rows 1,
7, 33, 137 with sliced inputs, 1025; bucketed outputs; "cache" and "rotary
dimension" rejections) and tests/rotary_metadata_tensors_smoke.py (the
validated entry point equals the metadata one). Outputs are compared bit for bit
with the oracle's fp32 form (bf16 x bf16 products are exact in fp32, so the
rounding is fixed) and pass the reference's fp64 relative-L2 gate. The fused
path (rotary_paged_attn, gk_rotary_kv_store) must equal rotary_embedding
followed by paged_attn bit for bit: same pool, same output.
"""

import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

REQUESTS, CONTEXT = 64, 64
SLOTS = REQUESTS * CONTEXT + 1


@pytest.fixture(scope="module")
def torch():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def device_bf16(torch, array_bits, sliced=False):
    t = torch.from_numpy(np.ascontiguousarray(array_bits).view(np.int16)).view(torch.bfloat16)
    if not sliced:
        return t.cuda()
    storage = torch.empty(t.shape[0], t.shape[1] + 1, dtype=torch.bfloat16, device="cuda")
    view = storage[:, 1:]
    view.copy_(t)
    return view


def metadata(torch, rows):
    """tests/rotary_runtime_smoke.py:23-28: rows spread over 64 requests, positions row // 64 + 3."""
    mapping = torch.arange(1, SLOTS, dtype=torch.int32).reshape(REQUESTS, CONTEXT)
    requests = torch.arange(rows, dtype=torch.int64) % REQUESTS
    positions = torch.arange(rows, dtype=torch.int64) // REQUESTS + 3
    locations = mapping[requests, positions].to(torch.int64)
    meta = torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, SLOTS)
    return meta, positions.numpy()


def bf16_normal(rng, shape):
    return orc.bf16_from_f32(rng.standard_normal(shape).astype(np.float32))


CASES = [(56, 8, 128, 128, neox, rows) for neox in (True, False) for rows in (1, 7, 33, 137, 1025)]
CASES += [(4, 2, 96, 62, neox, 7) for neox in (True, False)]


@pytest.mark.parametrize("q_heads,k_heads,d,rot,neox,rows", CASES)
def test_rotary_embedding_matches_oracle(torch, q_heads, k_heads, d, rot, neox, rows):
    rng = np.random.default_rng(rows * 7 + d + neox)
    meta, pos = metadata(torch, rows)
    cache = bf16_normal(rng, (CONTEXT, rot))
    q, k = bf16_normal(rng, (rows, q_heads * d)), bf16_normal(rng, (rows, k_heads * d))
    sliced = rows == 137
    print("rotary", q_heads, k_heads, d, rot, neox, rows, "sliced" if sliced else "", flush=True)
    q_out, k_out = torch.ops.gaudirt.rotary_embedding.default(device_bf16(torch, q, sliced),
                                                              device_bf16(torch, k, sliced),
                                                              device_bf16(torch, cache), meta, d, rot, neox)
    torch.cuda.synchronize()
    bucket = 1 << (rows - 1).bit_length()
    for out, src in ((q_out, q), (k_out, k)):
        assert tuple(out.shape) == src.shape and out.is_contiguous()
        assert out.untyped_storage().nbytes() >= bucket * src.shape[1] * 2
        assert out.untyped_storage().nbytes() % 256 == 0
        got = bits(out)
        assert np.array_equal(got, orc.rotary_bf16(src, cache, pos, d, rot, neox))
        orc.rotary_gate(got, src, cache, pos, d, rot, neox)
    # The validated entry point on the metadata's own tensors gives the same bits
    # (tests/rotary_metadata_tensors_smoke.py:27-36).
    q2, k2 = torch.ops.gaudirt._rotary_embedding_validated.default(
        device_bf16(torch, q), device_bf16(torch, k), device_bf16(torch, cache), meta.rotary_positions(),
        meta.rotary_header(), meta.context(), d, rot, neox)
    assert np.array_equal(bits(q2), bits(q_out)) and np.array_equal(bits(k2), bits(k_out))


@pytest.mark.parametrize("dtype", ["int32", "int64"])
@pytest.mark.parametrize("neox", [True, False])
def test_rotary_embedding_positions(torch, dtype, neox):
    # Positions given directly; 3-D [rows, heads, d] inputs keep their shape.
    rng = np.random.default_rng(11 + neox)
    rows, q_heads, k_heads, d, rot, ctx = 300, 8, 2, 128, 64, 4096
    cache = bf16_normal(rng, (ctx, rot))
    pos = rng.integers(0, ctx, rows)
    q, k = bf16_normal(rng, (rows, q_heads * d)), bf16_normal(rng, (rows, k_heads * d))
    positions = torch.from_numpy(pos.astype(dtype)).cuda()
    q3 = device_bf16(torch, q).view(rows, q_heads, d)
    k3 = device_bf16(torch, k).view(rows, k_heads, d)
    q_out, k_out = torch.ops.gaudirt.rotary_embedding_positions.default(q3, k3, device_bf16(torch, cache), positions,
                                                                        d, rot, neox)
    torch.cuda.synchronize()
    assert q_out.shape == q3.shape and k_out.shape == k3.shape
    assert np.array_equal(bits(q_out).reshape(rows, -1), orc.rotary_bf16(q, cache, pos, d, rot, neox))
    assert np.array_equal(bits(k_out).reshape(rows, -1), orc.rotary_bf16(k, cache, pos, d, rot, neox))
    empty = torch.empty(0, q_heads * d, dtype=torch.bfloat16, device="cuda")
    e_q, e_k = torch.ops.gaudirt.rotary_embedding_positions.default(
        empty, torch.empty(0, k_heads * d, dtype=torch.bfloat16, device="cuda"), device_bf16(torch, cache),
        torch.empty(0, dtype=torch.int32, device="cuda"), d, rot, neox)
    assert e_q.shape == (0, q_heads * d) and e_k.shape == (0, k_heads * d)


def test_rotary_rejections(torch):
    # tests/rotary_runtime_smoke.py:104-116: a cache shorter than the context and
    # an odd rotary dimension are rejected before any launch.
    rng = np.random.default_rng(5)
    meta, _ = metadata(torch, 7)
    cache = device_bf16(torch, bf16_normal(rng, (CONTEXT, 62)))
    q, k = device_bf16(torch, bf16_normal(rng, (7, 4 * 96))), device_bf16(torch, bf16_normal(rng, (7, 2 * 96)))
    for bad_cache, bad_rot, message in ((cache[:32], 62, "cache"), (cache, 61, "rotary dimension")):
        with pytest.raises(RuntimeError, match=message):
            torch.ops.gaudirt.rotary_embedding.default(q, k, bad_cache, meta, 96, bad_rot, True)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("d,rot", [(128, 128), (128, 64), (64, 64)])
def test_rotary_kv_store_c_abi(torch, neox, d, rot):
    # gk_rotary_kv_store: rotated keys and the values land at their slots, every
    # other pool element keeps its sentinel, negative slots skip the row.
    from gaudirt_amd import capi

    rng = np.random.default_rng(d + rot + neox)
    rows, q_heads, kv_heads, slots, ctx = 97, 16, 4, 512, 256
    cache = bf16_normal(rng, (ctx, rot))
    pos = rng.integers(0, ctx, rows)
    slot_map = rng.permutation(slots)[:rows].astype(np.int32)
    slot_map[::13] = -1
    q, k, v = (bf16_normal(rng, (rows, w)) for w in (q_heads * d, kv_heads * d, kv_heads * d))
    pool_bits = np.full((2, kv_heads, slots, d), 0x7FC1, dtype=np.uint16)
    pool = device_bf16(torch, pool_bits.reshape(-1, d))
    q_dev, k_dev, v_dev = device_bf16(torch, q), device_bf16(torch, k), device_bf16(torch, v)
    q_out = torch.empty(rows, q_heads * d, dtype=torch.bfloat16, device="cuda")
    positions = torch.from_numpy(pos.astype(np.int64)).cuda()
    slot_dev = torch.from_numpy(slot_map).cuda()
    cache_dev = device_bf16(torch, cache)
    p = capi.RotaryParams()
    p.query, p.q_row_stride, p.q_width = q_dev.data_ptr(), q_dev.stride(0), q_dev.shape[1]
    p.key, p.k_row_stride, p.k_width = k_dev.data_ptr(), k_dev.stride(0), k_dev.shape[1]
    p.positions, p.positions_int64 = positions.data_ptr(), 1
    p.cos_sin, p.cache_rows = cache_dev.data_ptr(), ctx
    p.rows, p.head_dim, p.rotary_dim, p.is_neox = rows, d, rot, int(neox)
    p.q_out, p.q_out_row_stride = q_out.data_ptr(), q_out.stride(0)
    p.value, p.v_row_stride = v_dev.data_ptr(), v_dev.stride(0)
    p.slot_mapping, p.pool, p.slots, p.kv_heads = slot_dev.data_ptr(), pool.data_ptr(), slots, kv_heads
    capi.check(capi.load().gk_rotary_kv_store(ctypes.byref(p), capi.current_stream()))
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_out), orc.rotary_bf16(q, cache, pos, d, rot, neox))
    expected = pool_bits.copy()
    keep = slot_map >= 0  # the oracle's store takes valid slots only
    k_rot = orc.rotary_bf16(k, cache, pos, d, rot, neox)
    orc.kv_store(k_rot[keep], v[keep], slot_map[keep], int(keep.sum()), expected, slots, kv_heads, d)
    assert np.array_equal(bits(pool).reshape(expected.shape), expected)


@pytest.mark.parametrize("rows,neox", [(1, True), (64, False), (200, True)])
def test_rotary_paged_attn_equals_rotary_then_paged_attn(torch, rows, neox):
    # The fused op against the two reference ops on the same inputs: pool and
    # output identical bit for bit (decode rows and multi-row prefill runs).
    import gaudirt_amd

    rng = np.random.default_rng(rows + 3 * neox)
    q_heads, kv_heads, d, rot = 32, 8, 128, 128
    meta, _ = metadata(torch, rows)
    cache = device_bf16(torch, bf16_normal(rng, (CONTEXT, rot)))
    q = device_bf16(torch, bf16_normal(rng, (rows, q_heads * d)))
    k = device_bf16(torch, bf16_normal(rng, (rows, kv_heads * d)))
    v = device_bf16(torch, bf16_normal(rng, (rows, kv_heads * d)))
    scale = float(np.float32(1 / math.sqrt(d)))
    base = torch.randn(2, kv_heads, SLOTS, d, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    outs, pools = [], []
    for fused in (False, True):
        pool = gaudirt_amd.allocate_paged_kv(1, SLOTS, kv_heads, d)
        pool[0].copy_(base.cuda())
        key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
        if fused:
            out = torch.ops.gaudirt.rotary_paged_attn.default(q, k, v, key_pool, value_pool, cache, meta, d, rot,
                                                              neox, scale)
        else:
            q_rot, k_rot = torch.ops.gaudirt.rotary_embedding.default(q, k, cache, meta, d, rot, neox)
            out = torch.ops.gaudirt.paged_attn.default(q_rot, k_rot, v, key_pool, value_pool, meta, d, scale)
        torch.cuda.synchronize()
        outs.append(bits(out))
        pools.append(bits(pool))
    assert np.array_equal(pools[0], pools[1])
    assert np.array_equal(outs[0], outs[1])
