"""GPU parity of torch.ops.gaudirt.paged_attn (the drop-in boundary) against the CPU oracle.

Follows the reference's device smokes: tests/paged_attention_smoke.py (two
layers, rows 1..4096, sliced K/V, full KV-pool audit, overlapping-pool and
head-dimension rejection), tests/paged_gqa_geometry_smoke.py (32:8 GQA, decode
positions 254/255/511) and tests/paged_attention_generalized_smoke.py (head
dims 64/128/256, kv heads 1/3, sliding window, softcap). The KV pool is checked
bit-exactly; outputs within max-abs 2e-2 / mean-abs 2e-3 of direct_bf16_pv and
the reference's relative-L2 gates.
"""

import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.fixture(scope="module")
def torch_ext():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def randn_bf16(torch, gen, *shape):
    return torch.randn(*shape, generator=gen).to(torch.bfloat16)


def run_case(torch, heads, kv_heads, dim, requests_n, context, rows, *, sliced=False, seed=3127, softcap=0.0,
             window=-1, positions=None, request_ids=None, layers=1):
    import gaudirt_amd

    gen = torch.Generator().manual_seed(seed + rows)
    slots = requests_n * context + 1
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    mapping = torch.arange(1, slots, dtype=torch.int32).reshape(requests_n, context)
    requests = request_ids if request_ids is not None else torch.arange(rows, dtype=torch.int64) % requests_n
    positions = positions if positions is not None else torch.arange(rows, dtype=torch.int64) // requests_n + 3
    locations = mapping[requests, positions].to(torch.int64)
    meta = torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, slots)
    q_cpu = randn_bf16(torch, gen, rows, heads * dim)
    k_cpu = randn_bf16(torch, gen, rows, kv_heads * dim)
    v_cpu = randn_bf16(torch, gen, rows, kv_heads * dim)
    pool = gaudirt_amd.allocate_paged_kv(layers, slots, kv_heads, dim)
    results = []
    for layer in range(layers):
        key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, layer)
        kb, vb = randn_bf16(torch, gen, slots, kv_heads, dim), randn_bf16(torch, gen, slots, kv_heads, dim)
        key_pool.copy_(kb)
        value_pool.copy_(vb)
        q = q_cpu.cuda()
        if sliced:  # K/V as column slices of wider rows (unaligned views)
            ks = torch.empty(rows, kv_heads * dim + 1, dtype=torch.bfloat16, device="cuda")
            vs = torch.empty_like(ks)
            k, v = ks[:, 1:], vs[:, 1:]
            k.copy_(k_cpu)
            v.copy_(v_cpu)
        else:
            k, v = k_cpu.cuda(), v_cpu.cuda()
        out = torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, value_pool, meta, dim, scale, softcap, window)
        torch.cuda.synchronize()
        assert out.shape == q.shape and out.is_contiguous()
        assert out.untyped_storage().nbytes() >= (1 << (rows - 1).bit_length()) * heads * dim * 2
        assert out.untyped_storage().nbytes() % 256 == 0
        # KV pool: bit-exact against the oracle's store into the same base.
        expected = np.stack([bits(kb), bits(vb)]).transpose(0, 2, 1, 3).copy()  # [2, Hkv, S, d]
        orc.kv_store(bits(k_cpu), bits(v_cpu), locations.numpy(), rows, expected, slots, kv_heads, dim)
        actual_pool = np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))])
        assert np.array_equal(actual_pool, expected), "KV pool differs from the oracle store"
        problem = orc.Problem(bits(q_cpu), expected, requests.numpy(), positions.numpy(), mapping.numpy(),
                              heads, kv_heads, dim, scale, softcap, window)
        results.append((bits(out), problem, out, (q, k, v, key_pool, value_pool)))
    return results, meta, scale


def check(actual, problem, fp32_softmax=False):
    if fp32_softmax:
        ref = orc.fp32_softmax_attention(problem)
    else:
        ref = orc.direct_bf16_pv(problem)
    assert np.isfinite(orc.bf16_to_f32(actual)).all()
    max_abs, mean_abs = orc.check_tolerance(actual, ref, MAX_ABS, MEAN_ABS)
    if not fp32_softmax:
        tiled = orc.tiled_bf16_pv(problem, 512)
        orc.isolated_errors(orc.bf16_to_f32(actual), orc.fp64_bf16(problem), orc.bf16_to_f32(tiled))
    return max_abs, mean_abs


@pytest.mark.parametrize("geometry,rows", [
    ("small", 1), ("small", 3), ("small", 17), ("small", 137), ("small", 513), ("small", 1025), ("small", 4096),
    ("nanbeige", 1), ("nanbeige", 7), ("nanbeige", 33), ("nanbeige", 137), ("nanbeige", 1025),
])
def test_paged_attention_two_layers(torch_ext, geometry, rows):
    torch = torch_ext
    heads, kv_heads, dim = (4, 2, 64) if geometry == "small" else (56, 8, 128)
    requests_n, context = (64, 128) if geometry == "small" else (64, 32)
    results, meta, scale = run_case(torch, heads, kv_heads, dim, requests_n, context, rows, layers=2,
                                    sliced=rows in (17, 137))
    for actual, problem, _, _ in results:
        print(geometry, rows, "max/mean abs", check(actual, problem), flush=True)
    if rows == 3:
        q, k, v, key_pool, value_pool = results[0][3]
        before = bits(key_pool)
        with pytest.raises(RuntimeError, match="combined storage"):
            torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, key_pool, meta, dim, scale)
        assert np.array_equal(bits(key_pool), before)
        with pytest.raises(RuntimeError, match="head dimension"):
            torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, value_pool, meta, 96, scale)


def test_paged_attention_at_the_row_limit(torch_ext):
    # 8192 rows, the reference's largest metadata (kMaxRows,
    # src/bridge/paged_metadata.hpp:19; one more is rejected on the CPU): 128
    # requests with 64 interleaved decode rows each, store and attention
    # checked against the oracle.
    torch = torch_ext
    results, _, _ = run_case(torch, 4, 2, 64, 128, 128, 8192)
    for actual, problem, _, _ in results:
        print("rows 8192 max/mean abs", check(actual, problem), flush=True)


def test_repeat_is_deterministic(torch_ext):
    torch = torch_ext
    a, _, _ = run_case(torch, 56, 8, 128, 64, 32, 137)
    b, _, _ = run_case(torch, 56, 8, 128, 64, 32, 137)
    assert np.array_equal(a[0][0], b[0][0])


def test_single_row_replay_matches_batch(torch_ext):
    # tests/paged_attention_smoke.py:137-143: the last row alone reproduces the
    # batched row (within tolerance here: the split-K partition depends on the
    # batch's occupancy, so the last bits may differ).
    import gaudirt_amd

    torch = torch_ext
    results, meta, scale = run_case(torch, 56, 8, 128, 64, 32, 137)
    actual, problem, out, (q, k, v, key_pool, value_pool) = results[0]
    requests = torch.from_numpy(problem.requests[-1:].copy())
    positions = torch.from_numpy(problem.positions[-1:].copy())
    mapping = torch.from_numpy(problem.mapping)
    locations = mapping[requests, positions].to(torch.int64)
    one = torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, problem.slots)
    replay = torch.ops.gaudirt.paged_attn.default(q[-1:], k[-1:], v[-1:], key_pool, value_pool, one, 128, scale)
    max_abs, _ = orc.tolerance_errors(bits(replay), actual[-1:])
    assert max_abs <= 1e-2, max_abs
    del gaudirt_amd


@pytest.fixture
def batch_invariant(torch_ext):
    import gaudirt_amd

    gaudirt_amd.set_batch_invariant_decode(True)
    assert gaudirt_amd.batch_invariant_decode() == gaudirt_amd.BATCH_INVARIANT_PARTITION
    yield gaudirt_amd.BATCH_INVARIANT_PARTITION
    gaudirt_amd.set_batch_invariant_decode(False)
    assert gaudirt_amd.batch_invariant_decode() == 0


def replay_rows(torch, results, meta_rows, scale, heads, dim):
    """paged_attn on each listed row alone (its own one-row metadata); the bits of each output."""
    actual, problem, out, (q, k, v, key_pool, value_pool) = results[0]
    mapping = torch.from_numpy(problem.mapping)
    got = []
    for r in meta_rows:
        requests = torch.from_numpy(problem.requests[r:r + 1].copy())
        positions = torch.from_numpy(problem.positions[r:r + 1].copy())
        locations = mapping[requests, positions].to(torch.int64)
        one = torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, problem.slots)
        replay = torch.ops.gaudirt.paged_attn.default(q[r:r + 1], k[r:r + 1], v[r:r + 1], key_pool, value_pool, one,
                                                      dim, scale)
        got.append(bits(replay))
    return got


def test_single_row_replay_is_bitwise_in_batch_invariant_mode(torch_ext, batch_invariant):
    # tests/paged_attention_smoke.py:145-150 as the reference asserts it: the
    # last row of the 137-row batch replayed alone equals the batched row bit
    # for bit, here with the decode rows on fixed partitions.
    torch = torch_ext
    results, meta, scale = run_case(torch, 56, 8, 128, 64, 32, 137)
    actual, problem = results[0][0], results[0][1]
    check(actual, problem)
    (replay,) = replay_rows(torch, results, [136], scale, 56, 128)
    assert np.array_equal(replay, actual[-1:])


def test_long_rows_are_batch_invariant_in_batch_invariant_mode(torch_ext, batch_invariant):
    # Rows of up to 6000 keys span several fixed partitions (a split-K merge per
    # row); each replayed alone must equal its batched bits, and the batch must
    # still pass the parity gate.
    torch = torch_ext
    rng = np.random.default_rng(2026)
    requests_n, context = 24, 6000
    positions = torch.from_numpy(rng.integers(1, context, requests_n).astype(np.int64))
    positions[:3] = torch.tensor([context - 1, batch_invariant, batch_invariant - 1])
    results, meta, scale = run_case(torch, 32, 8, 128, requests_n, context, requests_n, positions=positions,
                                    request_ids=torch.arange(requests_n, dtype=torch.int64))
    actual, problem = results[0][0], results[0][1]
    print("max/mean abs", check(actual, problem), flush=True)
    rows = [0, 1, 2, 5, 11, 23]
    for r, replay in zip(rows, replay_rows(torch, results, rows, scale, 32, 128)):
        assert np.array_equal(replay, actual[r:r + 1]), r


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("position", [254, 255, 511])
def test_gqa_geometry(torch_ext, dim, position):
    # tests/paged_gqa_geometry_smoke.py: 32 query / 8 kv heads, one decode row per request.
    torch = torch_ext
    requests_n, context = 4, 512
    req = torch.arange(requests_n, dtype=torch.int64)
    pos = torch.full((requests_n,), position, dtype=torch.int64)
    results, _, _ = run_case(torch, 32, 8, dim, requests_n, context, requests_n, positions=pos, request_ids=req)
    check(results[0][0], results[0][1])


@pytest.mark.parametrize("dim,kv_heads,heads", [(64, 1, 4), (128, 3, 12), (256, 1, 8), (256, 3, 6)])
@pytest.mark.parametrize("variant", ["plain", "window", "softcap"])
def test_generalized(torch_ext, dim, kv_heads, heads, variant):
    # tests/paged_attention_generalized_smoke.py: head dims, odd kv-head counts,
    # sliding window and softcap against an fp32-softmax reference.
    torch = torch_ext
    window = 48 if variant == "window" else -1
    softcap = 30.0 if variant == "softcap" else 0.0
    requests_n, context = 12, 96
    rows = 36
    # three rows per request at positions 40, 60, 80: the window of 48 cuts the later two
    pos = torch.arange(rows, dtype=torch.int64) // requests_n * 20 + 40
    results, _, _ = run_case(torch, heads, kv_heads, dim, requests_n, context, rows, window=window,
                             softcap=softcap, seed=77, positions=pos)
    check(results[0][0], results[0][1], fp32_softmax=variant != "plain")


def test_advance_decode_lengths_op(torch_ext):
    torch = torch_ext
    seq = (torch.arange(100, dtype=torch.int64) * 3 + (1 << 40)).cuda()
    orig = (torch.arange(100, dtype=torch.int32) + 5).cuda()
    nxt, onxt = torch.ops.gaudirt._advance_decode_lengths(seq, orig)
    assert torch.equal(nxt, seq + 1) and torch.equal(onxt, orig + 1)
    with pytest.raises(RuntimeError, match="matching contiguous int64 and int32"):
        torch.ops.gaudirt._advance_decode_lengths(orig, seq)


def test_advance_decode_lengths_op_captured(torch_ext):
    # tests/decode_lengths_smoke.py counts one launch and no host copies per
    # call, with the old batch's tensors kept. Captured in a HIP graph (a host
    # copy or a synchronisation inside would fail the capture) and replayed with
    # new inputs copied in between.
    torch = torch_ext
    for count in (1, 3, 16):
        seq = (torch.arange(count, dtype=torch.int64) * (2**33) + 17).cuda()
        orig = (torch.arange(count, dtype=torch.int32) + 31).cuda()
        torch.ops.gaudirt._advance_decode_lengths(seq, orig)  # warm-up outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            nxt, onxt = torch.ops.gaudirt._advance_decode_lengths(seq, orig)
        for step in range(3):
            host_seq = torch.arange(count, dtype=torch.int64) * (2**33) + 17 + step * 1000
            host_orig = torch.arange(count, dtype=torch.int32) + 31 + step
            seq.copy_(host_seq)
            orig.copy_(host_orig)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(nxt.cpu(), host_seq + 1) and torch.equal(onxt.cpu(), host_orig + 1)
            assert torch.equal(seq.cpu(), host_seq) and torch.equal(orig.cpu(), host_orig)


def test_kv_pool_allocation_and_reuse(torch_ext):
    # tests/paged_kv_pool_smoke.py: geometry, zero init, layer-view addresses.
    import gaudirt_amd

    torch = torch_ext
    pool = gaudirt_amd.allocate_paged_kv(3, 1000, 4, 128)
    assert pool.shape == (3, 2, 4, 1000, 128) and pool.dtype == torch.bfloat16
    assert int(pool.view(torch.int16).abs().sum().item()) == 0
    for layer in range(3):
        k, v = gaudirt_amd.kv_pool_views(pool, layer)
        assert k.shape == (1000, 4, 128) and k.stride() == (128, 1000 * 128, 1)
        assert v.data_ptr() == k.data_ptr() + 1000 * 4 * 128 * 2
    assert pool.data_ptr() % 256 == 0
    stats = gaudirt_amd.kv_allocator_stats(0)
    assert stats["allocated_bytes"] >= 3 * 2 * 4 * 1000 * 128 * 2
    before = stats["allocated_bytes"]
    del pool, k, v
    torch.cuda.synchronize()
    assert gaudirt_amd.kv_allocator_stats(0)["allocated_bytes"] < before
    with pytest.raises(RuntimeError, match="unsupported head-major KV pool geometry"):
        gaudirt_amd.allocate_paged_kv(1, 100, 2, 96)


@pytest.mark.parametrize("heads,kv_heads,dim,block", [(32, 8, 128, 64), (8, 2, 64, 128), (16, 16, 128, 32),
                                                      (32, 8, 128, 16), (16, 4, 128, 4), (8, 2, 64, 8),
                                                      (32, 8, 128, 1), (8, 2, 64, 2)])
def test_mixed_prefill_and_decode_batch(torch_ext, heads, kv_heads, dim, block):
    """A batch mixing chunked-prefill runs (>= 8 consecutive positions: MFMA
    prefill kernel) and single decode rows (decode kernel via row_map), with a
    page-aligned request map, as a serving step of the reference would send
    (tests/paged_layer_store_smoke.py: mixed fused and tiled blocks with one
    KV update)."""
    import gaudirt_amd

    torch = torch_ext
    rng = np.random.default_rng(heads * 7 + block)
    requests_n = 6
    prefix = [0, 130, 7, 500, 64, 300]
    chunk = [40, 9, 1, 3, 200, 1]     # runs of 40, 9 and 200 rows go to prefill
    lens = [p + c for p, c in zip(prefix, chunk)]
    blocks_per = [(n + block - 1) // block for n in lens]
    ids = rng.permutation(sum(blocks_per) + 5)
    context = max(lens)
    mapping = np.full((requests_n, context), -1, dtype=np.int32)
    cursor = 0
    for r in range(requests_n):
        for t in range(lens[r]):
            mapping[r, t] = ids[cursor + t // block] * block + t % block
        cursor += blocks_per[r]
    slots = (sum(blocks_per) + 5) * block
    req = np.concatenate([np.full(c, r) for r, c in enumerate(chunk)]).astype(np.int64)
    pos = np.concatenate([p + np.arange(c) for p, c in zip(prefix, chunk)]).astype(np.int64)
    loc = mapping[req, pos].astype(np.int64)
    rows = len(req)
    meta = torch.classes.gaudirt.PagedMetadata(torch.from_numpy(loc), torch.from_numpy(req), torch.from_numpy(pos),
                                               torch.from_numpy(mapping), slots)
    gen = torch.Generator().manual_seed(5)
    q_cpu = randn_bf16(torch, gen, rows, heads * dim)
    k_cpu = randn_bf16(torch, gen, rows, kv_heads * dim)
    v_cpu = randn_bf16(torch, gen, rows, kv_heads * dim)
    pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
    base = randn_bf16(torch, gen, 2, kv_heads, slots, dim)
    pool[0].copy_(base)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    scale = float(np.float32(1 / math.sqrt(dim)))
    out = torch.ops.gaudirt.paged_attn.default(q_cpu.cuda(), k_cpu.cuda(), v_cpu.cuda(), key_pool, value_pool,
                                               meta, dim, scale)
    torch.cuda.synchronize()
    expected = bits(base)
    orc.kv_store(bits(k_cpu), bits(v_cpu), loc, rows, expected, slots, kv_heads, dim)
    assert np.array_equal(bits(pool[0]), expected)
    problem = orc.Problem(bits(q_cpu), expected, req, pos, mapping, heads, kv_heads, dim, scale)
    print("mixed batch", check(bits(out), problem), flush=True)


def test_misaligned_contiguous_views_are_packed(torch_ext):
    """Q/K/V that are contiguous but start at an odd element (not 16-byte
    aligned) are packed into fresh storage before the kernels read them, as the
    reference packs unaligned inputs (src/bridge/paged_attention.cpp:230-245):
    the result equals the aligned call bit for bit, the KV pool included."""
    torch = torch_ext
    aligned, meta, scale = run_case(torch, 8, 2, 128, 16, 64, 37)
    actual, problem, out, (q, k, v, key_pool, value_pool) = aligned[0]

    def odd_view(t):
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
        view = buf[1:].view(t.shape)
        view.copy_(t)
        assert view.is_contiguous() and view.data_ptr() % 16 != 0
        return view

    # The store is idempotent (the same rows to the same slots), so the pool the
    # second call attends equals the first call's.
    again = torch.ops.gaudirt.paged_attn.default(odd_view(q), odd_view(k), odd_view(v), key_pool, value_pool, meta,
                                                 128, scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(again), actual)
    assert np.array_equal(np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))]), problem.pool)
