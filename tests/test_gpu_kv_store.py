"""GPU parity of the KV store, tile-index and decode-length kernels (C ABI): bit-exact."""

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def runner():
    import torch
    assert torch.cuda.is_available()
    from tests import gk_runner
    return gk_runner


@pytest.mark.parametrize("head_dim,kv_heads,rows", [(128, 2, 4), (64, 3, 137), (256, 1, 7), (128, 8, 300)])
def test_kv_store_bit_exact(runner, head_dim, kv_heads, rows):
    import torch
    rng = np.random.default_rng(head_dim + rows)
    slots = 8192
    pool = rng.integers(0, 65535, (2, kv_heads, slots, head_dim), dtype=np.uint16)
    # sliced K/V rows (row stride > width), as the reference accepts
    width = kv_heads * head_dim
    k_store = rng.integers(0, 65535, (rows, width + 24), dtype=np.uint16)
    v_store = rng.integers(0, 65535, (rows, width + 24), dtype=np.uint16)
    loc = rng.permutation(slots)[:rows].astype(np.int32)
    loc[rows // 2] = -1  # a negative slot skips the row
    expected = pool.copy()
    keep = loc >= 0
    orc.kv_store(k_store[keep, 8:8 + width], v_store[keep, 8:8 + width], loc[keep], int(keep.sum()), expected,
                 slots, kv_heads, head_dim)
    d_pool = runner.bf16_device(pool)
    d_k = runner.bf16_device(k_store)[:, 8:8 + width]
    d_v = runner.bf16_device(v_store)[:, 8:8 + width]
    runner.kv_store(d_k, d_v, runner.to_device(loc), d_pool, kv_heads, head_dim)
    torch.cuda.synchronize()
    assert np.array_equal(runner.bits_of(d_pool), expected)


def test_tile_indices_bit_exact(runner):
    import torch
    from gaudirt_amd import capi
    rng = np.random.default_rng(3)
    requests_n, context, slots = 5, 300, 4096
    mapping = rng.integers(0, slots, (requests_n, context)).astype(np.int32)
    row_requests = rng.integers(0, requests_n, 40).astype(np.int32)
    work = np.stack([rng.integers(0, 40, 500), rng.integers(0, context - 64, 500), rng.integers(0, 65, 500),
                     rng.integers(0, 4, 500) * slots], axis=1).astype(np.int32)
    expected = orc.tile_indices(mapping.reshape(-1), row_requests, work, context)
    out = torch.full((500 * 64,), -7, dtype=torch.int32, device="cuda")
    lib = capi.load()
    d_map, d_req, d_work = (runner.to_device(a) for a in (mapping, row_requests, work))
    capi.check(lib.gk_attn_tile_indices(capi.ptr(d_map), capi.ptr(d_req), capi.ptr(d_work), 500, context,
                                        capi.ptr(out), capi.current_stream()))
    assert np.array_equal(out.cpu().numpy().reshape(500, 64), expected)


@pytest.mark.parametrize("requests_n,context,slots", [(2, 73, 2), (7, 1000, 4097), (256, 131072, 131072)])
def test_tile_indices_reference_device_cases(runner, requests_n, context, slots):
    # tests/attention_tile_indices_device_test.cpp of the reference, its own
    # construction and closed-form expectation (no oracle): map[r][i] = 1 +
    # (11 r + 7 i) mod (slots - 1); eight tasks alternating row 0 (request 0,
    # keys 0.., 64 lanes) and row 1 (the last request, keys 64.., 9 lanes),
    # base (t / 2) * slots; every one of the 64 lanes written.
    import torch
    from gaudirt_amd import capi
    r = np.arange(requests_n)[:, None]
    i = np.arange(context)[None, :]
    mapping = (1 + (r * 11 + i * 7) % (slots - 1)).astype(np.int32)
    row_requests = np.array([0, requests_n - 1], dtype=np.int32)
    tasks = 8
    work = np.array([[t % 2, (t % 2) * 64, 9 if t % 2 else 64, (t // 2) * slots] for t in range(tasks)],
                    dtype=np.int32)
    out = torch.full((tasks * 64,), -123, dtype=torch.int32, device="cuda")
    d_map, d_req, d_work = (runner.to_device(a) for a in (mapping, row_requests, work))
    capi.check(capi.load().gk_attn_tile_indices(capi.ptr(d_map), capi.ptr(d_req), capi.ptr(d_work), tasks, context,
                                                capi.ptr(out), capi.current_stream()))
    got = out.cpu().numpy().reshape(tasks, 64)
    for t in range(tasks):
        req, first, lanes, base = row_requests[work[t, 0]], work[t, 1], work[t, 2], work[t, 3]
        want = [base + (mapping[req, first + lane] if lane < lanes else 0) for lane in range(64)]
        assert got[t].tolist() == want, t


@pytest.mark.parametrize("count", [1, 3, 16, 70000])
def test_advance_decode_lengths(runner, count):
    # tests/decode_lengths_smoke.py's counts and values (int64 lengths past
    # 2^32), plus a count past one workgroup; the inputs stay as they were.
    import torch
    from gaudirt_amd import capi
    seq = torch.arange(count, dtype=torch.int64) * (2**33) + 17
    orig = torch.arange(count, dtype=torch.int32) + 31
    d_seq, d_orig = seq.cuda(), orig.cuda()
    nxt, onxt = torch.empty_like(d_seq), torch.empty_like(d_orig)
    capi.check(capi.load().gk_advance_decode_lengths(capi.ptr(d_seq), capi.ptr(d_orig), count, capi.ptr(nxt),
                                                     capi.ptr(onxt), capi.current_stream()))
    assert torch.equal(nxt.cpu(), seq + 1) and torch.equal(onxt.cpu(), orig + 1)
    assert torch.equal(d_seq.cpu(), seq) and torch.equal(d_orig.cpu(), orig)
