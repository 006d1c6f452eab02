"""gk_paged_decode_scratch (allocation-free decode) against gk_paged_decode, through the C ABI.

The allocation-free entry point runs the same kernels on a static device
array instead of a caller's workspace, so its output must equal
gk_paged_decode's bit for bit. Three calls in a row share the array: workload
C2 at full size (balanced split-K schedule), then smaller inputs on other
paths (an explicit partition with the partitioned kernel and its merge, then
the fused KV store on C1's shape); each is compared with gk_paged_decode on
identical inputs. Parameters needing more workspace than the array holds are
rejected before anything is written.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch

    from gaudirt_amd import capi
    from tests import gk_runner

    assert torch.cuda.is_available()
    return torch, capi, capi.load(), gk_runner


def both_entry_points(env, make_params):
    """(scratch output bits, workspace output bits, scratch pool bits, workspace pool bits)."""
    torch, capi, lib, runner = env
    results = []
    for scratch in (True, False):
        params, out, pool = make_params()
        if scratch:
            capi.check(lib.gk_paged_decode_scratch(ctypes.byref(params), capi.current_stream()))
        else:
            ws = runner.paged_decode(params)
        torch.cuda.synchronize()
        results.append((runner.bits_of(out), runner.bits_of(pool)))
        if not scratch:
            del ws
    (a_out, a_pool), (b_out, b_pool) = results
    return a_out, b_out, a_pool, b_pool


def test_scratch_decode_equals_workspace_decode_on_consecutive_calls(env):
    torch, capi, lib, runner = env
    from gaudirt_amd import workloads
    from tests import paged_cases as cases

    # 1. C2 at full size: the balanced schedule's partials and span records.
    dc = workloads.DeviceDecodeCase("c2")

    def c2():
        out = torch.full_like(dc.out, float("nan"))
        p = runner.decode_params(dc.query, dc.pool, dc.d_tables, dc.d_lens, dc.heads, dc.kv_heads, dc.head_dim,
                                 dc.block_size, dc.scale, out)
        return p, out, dc.pool

    need = lib.gk_paged_decode_workspace_bytes(ctypes.byref(c2()[0]))
    print(f"call 1: C2, workspace {need} bytes of {capi.GK_DECODE_SCRATCH_BYTES}", flush=True)
    assert 0 < need <= capi.GK_DECODE_SCRATCH_BYTES
    a, b, _, _ = both_entry_points(env, c2)
    assert np.isfinite(a.view(np.uint16).astype(np.float32)).all()
    assert np.array_equal(a, b)
    del dc

    # 2. Smaller: 5 rows, 16 q / 4 kv heads, head_dim 64, 16-token blocks, explicit
    # 64-key partitions (partitioned kernel + split-K merge).
    case = cases.decode_case(31, 5, 16, 4, 64, 16, 256, [1, 70, 300, 999, 64])

    def small():
        q, pool = runner.bf16_device(case.query), runner.bf16_device(case.pool)
        tables, lens = runner.to_device(case.block_tables), runner.to_device(case.lens.astype(np.int32))
        out = torch.full((case.batch, case.heads * case.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda")
        p = runner.decode_params(q, pool, tables, lens, case.heads, case.kv_heads, case.head_dim, case.block_size,
                                 case.scale, out, partition=64)
        small.keep = (q, pool, tables, lens)
        return p, out, pool

    print("call 2: 5 rows, explicit 64-key partitions", flush=True)
    a, b, _, _ = both_entry_points(env, small)
    assert np.array_equal(a, b)

    # 3. C1's shape with the fused KV store of one new token per row.
    case = cases.c1_case()
    rng = np.random.default_rng(5)
    new_k = cases.bf16_normal(rng, (case.batch, case.kv_heads * case.head_dim))
    new_v = cases.bf16_normal(rng, (case.batch, case.kv_heads * case.head_dim))
    slots = np.array([case.block_tables[r, (n - 1) // 128] * 128 + (n - 1) % 128 for r, n in enumerate(case.lens)],
                     dtype=np.int32)

    def fused():
        q, pool = runner.bf16_device(case.query), runner.bf16_device(case.pool)
        tables, lens = runner.to_device(case.block_tables), runner.to_device(case.lens.astype(np.int32))
        k, v, sm = runner.bf16_device(new_k), runner.bf16_device(new_v), runner.to_device(slots)
        out = torch.full((case.batch, case.heads * case.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda")
        p = runner.decode_params(q, pool, tables, lens, case.heads, case.kv_heads, case.head_dim, case.block_size,
                                 case.scale, out, new_key=k, new_value=v, slot_mapping=sm)
        fused.keep = (q, pool, tables, lens, k, v, sm)
        return p, out, pool

    print("call 3: C1 with the fused KV store", flush=True)
    a, b, pa, pb = both_entry_points(env, fused)
    assert np.array_equal(a, b) and np.array_equal(pa, pb)


def test_scratch_decode_rejects_oversized_workspace(env):
    torch, capi, lib, runner = env
    # 4096 rows x 64 heads x 256 partitions of 32 keys: gigabytes of partials.
    rows, heads, kv_heads, d = 4096, 64, 8, 128
    q = torch.zeros((rows, heads * d), dtype=torch.bfloat16, device="cuda")
    pool = torch.zeros((2, kv_heads, 8192, d), dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros((rows, 64), dtype=torch.int32, device="cuda")
    lens = torch.full((rows,), 8192, dtype=torch.int32, device="cuda")
    out = torch.full((rows, heads * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    p = runner.decode_params(q, pool, tables, lens, heads, kv_heads, d, 128, 0.1, out, partition=32,
                             max_context=8192)
    assert lib.gk_paged_decode_workspace_bytes(ctypes.byref(p)) > capi.GK_DECODE_SCRATCH_BYTES
    rc = lib.gk_paged_decode_scratch(ctypes.byref(p), capi.current_stream())
    assert rc == capi.GK_ERR_WORKSPACE
    assert b"static scratch" in lib.gk_last_error()
    torch.cuda.synchronize()
    assert bool(torch.isnan(out).all()), "a rejected call wrote output"


def test_scratch_decode_under_graph_capture(env):
    # The caller this entry point is for: a HIP graph. After one eager call on
    # the device (which looks up the array's address and the grid size), the
    # call is captured into a graph with nothing allocated during capture, and
    # every replay must equal gk_paged_decode on the inputs present at replay
    # time (the query is rewritten in place between replays, with eager work
    # and synchronisations in between).
    torch, capi, lib, runner = env
    from gaudirt_amd import workloads

    dc = workloads.DeviceDecodeCase("c2")
    out = torch.full_like(dc.out, float("nan"))
    params = runner.decode_params(dc.query, dc.pool, dc.d_tables, dc.d_lens, dc.heads, dc.kv_heads, dc.head_dim,
                                  dc.block_size, dc.scale, out)
    assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 0  # balanced schedule + merge
    capi.check(lib.gk_paged_decode_scratch(ctypes.byref(params), capi.current_stream()))  # first call: set-up
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.check(lib.gk_paged_decode_scratch(ctypes.byref(params), capi.current_stream()))
    torch.cuda.synchronize()

    want_out = torch.empty_like(dc.out)
    want_params = runner.decode_params(dc.query, dc.pool, dc.d_tables, dc.d_lens, dc.heads, dc.kv_heads,
                                       dc.head_dim, dc.block_size, dc.scale, want_out)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    for replay in range(3):
        dc.query.copy_(torch.randn(dc.query.shape, generator=gen, device="cuda").to(torch.bfloat16))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ws = runner.paged_decode(want_params)
        torch.cuda.synchronize()
        del ws
        got, want = runner.bits_of(out), runner.bits_of(want_out)
        print(f"replay {replay}: equal={np.array_equal(got, want)}", flush=True)
        assert np.array_equal(got, want), replay
    del graph
