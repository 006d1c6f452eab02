"""GPU parity of the balanced decode schedule (gk_paged_decode with partition_tokens = 0).

With the partition left to the library (any GQA group and block size, the
token-granular map included), gk_paged_decode splits the batch's
key tiles evenly over one resident grid: work units (row, kv head) are cut at
arbitrary tiles, partial states are merged with the log-sum-exp rule, and the
tiles of a unit are visited in rotated order. These cases pin every piece of
that bookkeeping against the CPU oracle: units split over hundreds of
workgroups, hundreds of rows (the schedule scans the contexts 64 rows at a
time), several head groups per kv head, sliding windows that start inside a
tile, rows shorter than one tile, requests shared between rows, and poisoned
pool slots outside every visible range.
"""

import numpy as np
import pytest

from oracle import oracle as orc
from tests import paged_cases as cases

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.fixture(scope="module")
def runner():
    import torch
    assert torch.cuda.is_available()
    from tests import gk_runner
    return gk_runner


def check(case, actual, fp32_softmax=False, rows=None):
    p = case.oracle_problem()
    ref = orc.fp32_softmax_attention(p, 16) if fp32_softmax else orc.direct_bf16_pv(p, 16)
    if rows is not None:
        actual, ref = actual[rows], ref[rows]
    assert np.isfinite(orc.bf16_to_f32(actual)).all()
    max_abs, mean_abs = orc.check_tolerance(actual, ref, MAX_ABS, MEAN_ABS)
    ulp_only = orc.ulp_allowance_count(actual, ref, MAX_ABS)
    print(f"max_abs={max_abs:.3e} mean_abs={mean_abs:.3e} ulp_allowance_only={ulp_only} of {actual.size}",
          flush=True)
    return max_abs, mean_abs


def test_library_choice_is_the_balanced_schedule(runner):
    import ctypes
    import torch
    from gaudirt_amd import capi

    case = cases.decode_case(1, 3, 32, 8, 128, 128, 64, [100, 2000, 7])
    params = runner.decode_params(runner.bf16_device(case.query), runner.bf16_device(case.pool),
                                  runner.to_device(case.block_tables), runner.to_device(case.lens),
                                  32, 8, 128, 128, case.scale, torch.empty(3, 32 * 128, dtype=torch.bfloat16,
                                                                              device="cuda"))
    lib = capi.load()
    assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 0
    assert lib.gk_paged_decode_workspace_bytes(ctypes.byref(params)) > 0
    params.partition_tokens = 256
    assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 256


@pytest.mark.parametrize("geometry", [(14, 2, 64), (56, 8, 128), (64, 8, 128), (8, 1, 256), (32, 2, 128),
                                      (64, 2, 128), (24, 1, 64), (40, 2, 256),
                                      # GQA groups 1-3: 1-3 of the tile's 16 head columns used
                                      (8, 8, 128), (2, 2, 64), (16, 8, 64), (9, 3, 128), (3, 1, 256), (4, 2, 256)])
def test_stream_geometries(runner, geometry):
    heads, kv_heads, d = geometry
    rng = np.random.default_rng(heads * 1000 + kv_heads * 10 + d)
    lens = np.concatenate([[1, 2, 15, 16, 17, 31, 32, 33, 127, 128, 129], rng.integers(1, 2500, 5)])
    block = 16 if d == 256 else 32
    case = cases.decode_case(11, len(lens), heads, kv_heads, d, block, 4096 // block * 4, lens)
    print("geometry", geometry, flush=True)
    check(case, runner.run_case(case))


@pytest.mark.parametrize("block_size", [32, 64, 256, 1024])
def test_stream_block_sizes(runner, block_size):
    lens = np.array([5, 300, 777, 1024, 63, 2048, 1])
    case = cases.decode_case(block_size + 3, len(lens), 32, 8, 128, block_size, 8192 // block_size * 2, lens)
    check(case, runner.run_case(case))


@pytest.mark.parametrize("geometry", [(128, 1), (128, 2), (128, 4), (128, 8), (128, 16), (64, 1), (64, 4),
                                      (64, 8), (64, 16), (256, 1), (256, 2), (256, 4), (256, 8)])
def test_stream_small_blocks(runner, geometry):
    # Blocks shorter than a tile: every 16-byte load of a tile (64 / (d / 8)
    # keys) reads its own block-table entry; shorter blocks, down to the
    # token-granular map, one entry per key.
    d, block = geometry
    heads, kv_heads = (16, 2) if d == 256 else (32, 8)
    lens = np.array([1, 2, 3, 4, 5, 31, 33, 300, 777, 1024, 2047])
    case = cases.decode_case(7 * block + d, len(lens), heads, kv_heads, d, block, 8192 // block * 2, lens)
    print("head_dim", d, "block", block, flush=True)
    check(case, runner.run_case(case))


@pytest.mark.parametrize("block", [1, 2, 4, 16])
def test_stream_small_blocks_window_evicted(runner, block):
    # Sliding window over blocks shorter than a tile, with every slot outside
    # the visible keys poisoned (NaN) and the table entries of blocks wholly
    # below the window set to -1, as after eviction: a tile's masked runs must
    # read only blocks the row still owns.
    import copy

    lens = np.array([40, 300, 1000, 64, 65, 3000, 1, 77, 78, 79])
    case = cases.decode_case(33 + block, len(lens), 16, 4, 128, block, 16384 // block, lens)
    case.window, case.softcap = 77, 30.0
    used = np.zeros(case.slots, dtype=bool)
    evicted = case.block_tables.copy()
    for b, n in enumerate(case.lens):
        left = max(0, int(n) - case.window)
        for t in range(left, n):
            used[case.block_tables[b, t // block] * block + t % block] = True
        evicted[b, :left // block] = -1
    case.pool[:, :, ~used, :] = 0x7fc0
    reference = copy.copy(case)
    case.block_tables = evicted
    print("block", block, flush=True)
    check(reference, runner.run_case(case), fp32_softmax=True)


def test_library_choice_small_blocks(runner):
    # Every block size and GQA group takes the balanced schedule (partition 0)
    # when the partition is left to the library.
    import ctypes
    import torch
    from gaudirt_amd import capi

    lib = capi.load()
    for d, block, heads in [(128, 1, 16), (128, 2, 16), (64, 4, 16), (256, 1, 16), (128, 1, 6), (64, 16, 2),
                            (256, 128, 4)]:
        case = cases.decode_case(1, 2, heads, 2, d, block, 256, [30, 60])
        params = runner.decode_params(runner.bf16_device(case.query), runner.bf16_device(case.pool),
                                      runner.to_device(case.block_tables), runner.to_device(case.lens), heads, 2, d,
                                      block, case.scale, torch.empty(2, heads * d, dtype=torch.bfloat16, device="cuda"))
        assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 0, (d, block, heads)
        params.partition_tokens = 512
        assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 512, (d, block, heads)


def test_one_long_row_split_over_the_grid(runner):
    # 2 kv heads x 20000 keys: ~1250 tiles over ~1000 workgroups, so each unit's
    # partial states come from hundreds of workgroups.
    case = cases.decode_case(21, 1, 16, 2, 128, 128, 200, [20000])
    check(case, runner.run_case(case))


def test_many_rows_skewed(runner):
    # More than 64 rows (the schedule's row scan runs in 64-row windows), lengths
    # from 1 key to 40 tiles, including rows shorter than one tile.
    rng = np.random.default_rng(5)
    lens = np.concatenate([rng.integers(1, 40, 150), rng.integers(1, 1300, 150), [1, 1, 2]]).astype(np.int32)
    rng.shuffle(lens)
    case = cases.decode_case(22, len(lens), 8, 2, 64, 32, 8192, lens)
    check(case, runner.run_case(case))


def test_rows_beyond_the_prefetched_windows(runner):
    # 700 rows: the schedule reads the first 512 rows' contexts in one batch
    # and the rest 64 rows at a time; workgroups start in both parts.
    rng = np.random.default_rng(17)
    lens = rng.integers(1, 400, 700).astype(np.int32)
    case = cases.decode_case(24, len(lens), 8, 2, 64, 16, int(((lens + 15) // 16).sum()) + 8, lens)
    check(case, runner.run_case(case))


def test_tiny_batch_fewer_tiles_than_workgroups(runner):
    case = cases.decode_case(23, 2, 8, 2, 128, 64, 8, [3, 40])
    check(case, runner.run_case(case))


@pytest.mark.parametrize("block", [1, 4, 32])
@pytest.mark.parametrize("variant", ["window", "softcap", "both"])
def test_stream_window_and_softcap(runner, variant, block):
    lens = np.array([40, 300, 1000, 64, 65, 3000, 1])
    case = cases.decode_case(31, len(lens), 16, 4, 128, block, 16384 // block, lens)
    if variant in ("window", "both"):
        case.window = 77  # starts inside a 32-key tile
    if variant in ("softcap", "both"):
        case.softcap = 30.0
    check(case, runner.run_case(case), fp32_softmax=True)


@pytest.mark.parametrize("geometry", [(8, 8, 128), (6, 3, 64), (9, 3, 128), (4, 2, 64)])
@pytest.mark.parametrize("block", [1, 4, 32])
@pytest.mark.parametrize("variant", ["plain", "window", "softcap", "both"])
def test_stream_small_groups_window_softcap_blocks(runner, geometry, variant, block):
    # GQA groups 1-3: units of one to three query heads, with a window that
    # starts inside a tile, softcap, short rows and sub-tile blocks.
    heads, kv_heads, d = geometry
    lens = np.array([1, 31, 33, 40, 300, 1000, 64, 65, 2100])
    case = cases.decode_case(heads * 100 + d + block, len(lens), heads, kv_heads, d, block, 16384 // block, lens)
    if variant in ("window", "both"):
        case.window = 77
    if variant in ("softcap", "both"):
        case.softcap = 30.0
    print("geometry", geometry, "block", block, variant, flush=True)
    check(case, runner.run_case(case), fp32_softmax=variant != "plain")


def test_stream_window_head_dim_256(runner):
    lens = np.array([40, 300, 1000, 64, 65])
    case = cases.decode_case(99, len(lens), 8, 2, 256, 32, 256, lens)
    case.softcap, case.window = 50.0, 64
    check(case, runner.run_case(case), fp32_softmax=True)


def test_stream_poisoned_unused_slots(runner):
    # NaN in every slot outside the visible prefixes: masked keys of a row's
    # first and last tiles must not reach the output.
    lens = np.array([3, 50, 129, 1000, 33])
    case = cases.decode_case(5, len(lens), 16, 4, 128, 32, 128, lens)
    used = np.zeros(case.slots, dtype=bool)
    for b, n in enumerate(case.lens):
        for t in range(n):
            used[case.block_tables[b, t // 32] * 32 + t % 32] = True
    case.pool[:, :, ~used, :] = 0x7fc0
    check(case, runner.run_case(case))


def test_stream_row_requests_shared(runner):
    """Rows index block-table rows through row_request (rows of one request share its table)."""
    import torch

    rng = np.random.default_rng(8)
    base = cases.decode_case(41, 4, 32, 8, 128, 128, 128, [2000, 900, 3000, 50])
    row_request = np.array([2, 0, 2, 1, 3, 0], dtype=np.int32)
    lens = np.array([2999, 1500, 3000, 900, 1, 2000], dtype=np.int32)  # within each request's table
    query = cases.bf16_normal(rng, (len(row_request), 32 * 128))
    q = runner.bf16_device(query)
    pool = runner.bf16_device(base.pool)
    out = torch.full((len(row_request), 32 * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.decode_params(q, pool, runner.to_device(base.block_tables), runner.to_device(lens), 32, 8, 128,
                                  128, base.scale, out, row_request=runner.to_device(row_request))
    ws = runner.paged_decode(params)
    torch.cuda.synchronize()
    del ws
    mapping = orc.mapping_from_block_table(base.block_tables, 128, int(lens.max()))
    p = orc.Problem(query, base.pool, row_request.astype(np.int64), lens.astype(np.int64) - 1, mapping, 32, 8, 128,
                    base.scale)
    ref = orc.direct_bf16_pv(p, 16)
    got = runner.bits_of(out)
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    orc.check_tolerance(got, ref, MAX_ABS, MEAN_ABS)


def test_stream_empty_rows_write_zeros(runner):
    lens = np.array([0, 700, 0, 33], dtype=np.int32)
    case = cases.decode_case(51, len(lens), 16, 4, 128, 32, 64, np.maximum(lens, 1))
    case.lens = lens
    actual = runner.run_case(case)
    assert (orc.bf16_to_f32(actual[[0, 2]]) == 0).all()
    case.lens = np.maximum(lens, 1)
    check(case, actual, rows=[1, 3])


def test_stream_matches_partitioned_path(runner):
    # The two schedules agree on the same inputs (each within the oracle's
    # tolerance, and with each other to a bf16 ulp or two).
    lens = np.array([1, 100, 4000, 2222, 31, 512])
    case = cases.decode_case(61, len(lens), 32, 8, 128, 128, 256, lens)
    a = runner.run_case(case)
    b = runner.run_case(case, partition=512)
    check(case, a)
    check(case, b)
    max_abs, _ = orc.tolerance_errors(a, b)
    assert max_abs <= 1e-2, max_abs


def test_stream_graph_capture_matches_eager(runner):
    """Captured into a graph on a fresh stream (the merge then runs as its own
    kernel), replayed with eager calls in between: every replay equals the
    eager result bit for bit."""
    import ctypes
    import torch
    from gaudirt_amd import capi

    lens = np.array([1, 100, 4000, 2222, 31, 512, 3000, 7])
    case = cases.decode_case(71, len(lens), 32, 8, 128, 128, 256, lens)
    q = runner.bf16_device(case.query)
    pool = runner.bf16_device(case.pool)
    tables = runner.to_device(case.block_tables)
    d_lens = runner.to_device(case.lens.astype(np.int32))
    out = torch.zeros(len(lens), 32 * 128, dtype=torch.bfloat16, device="cuda")
    params = runner.decode_params(q, pool, tables, d_lens, 32, 8, 128, 128, case.scale, out)
    lib = capi.load()
    need = lib.gk_paged_decode_workspace_bytes(ctypes.byref(params))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")

    eager = runner.paged_decode(params)
    torch.cuda.synchronize()
    del eager
    want = out.clone()
    check(case, runner.bits_of(want))

    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            capi.check(lib.gk_paged_decode(ctypes.byref(params), ctypes.c_void_p(ws.data_ptr()), need,
                                           ctypes.c_void_p(stream.cuda_stream)))
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        eager = runner.paged_decode(params)  # eager call between replays (default stream)
        torch.cuda.synchronize()
        del eager


def _stream_grid_workgroups(lib, params):
    """Workgroups of the balanced grid, read back from the workspace size the
    library asks for: units * 8 bytes of span records plus, for head_dim 128 and
    4 heads per workgroup, wgs * 4 * (128 * 4 * 2 + 2 * 4 * 2) bytes of partial
    slots (both sections multiples of 256 bytes when 4 divides wgs)."""
    import ctypes

    units = params.rows * params.kv_heads
    partial = lib.gk_paged_decode_workspace_bytes(ctypes.byref(params)) - units * 8
    per_wg = 4 * (128 * 4 * 2 + 2 * 4 * 2)
    assert partial > 0 and partial % per_wg == 0, partial
    return partial // per_wg


def test_stream_routing_boundary_includes_the_grid(runner):
    # Host only (no launch): the balanced schedule numbers a batch's positions
    # (tiles plus a fixed cost per unit) in 32 bits, so gk_paged_decode takes it
    # exactly while units * (max_context / 32 + 2 + cost) + workgroups + cost
    # < 2^31, and the partitioned kernel (a non-zero partition) from there on.
    # The rows are chosen so that the workgroup term decides: without it the
    # boundary would lie one tile per row later.
    import ctypes
    from gaudirt_amd import capi

    lib = capi.load()
    dummy = runner.to_device(np.zeros(16, dtype=np.int32))
    params = capi.DecodeParams()
    params.query = params.pool = params.out = dummy.data_ptr()
    params.block_tables = params.row_context = dummy.data_ptr()
    params.q_row_stride = params.out_row_stride = 32 * 128
    params.slots, params.bt_stride, params.block_size = 1 << 20, 1, 128
    params.q_heads, params.kv_heads, params.head_dim = 32, 8, 128
    params.scale, params.softcap, params.sliding_window = 0.088, 0.0, -1
    params.partition_tokens = 0
    params.rows, params.max_context = 1, 64
    wgs = _stream_grid_workgroups(lib, params)
    print("balanced grid workgroups", wgs, flush=True)
    limit = 1 << 31
    checked = 0
    cost = capi.STREAM_UNIT_COST
    fixed = 2 + cost  # per-row position bound n = max_context / 32 + fixed
    for rows in range(65535, 0, -1):
        units = rows * 8
        n = (limit - 1) // units  # largest position bound without the grid term
        if units * n + wgs + cost < limit or n < fixed + 1:
            continue  # the grid term does not decide for this batch
        params.rows = rows
        params.max_context = (n - fixed) * 32 - 1  # bound n - 1: fits with the grid term
        assert units * (n - 1) + wgs + cost < limit
        assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 0, (rows, params.max_context)
        params.max_context = (n - fixed) * 32  # bound n: fits only without the grid term
        assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) != 0, (rows, params.max_context)
        checked += 1
        if checked == 3:
            break
    assert checked == 3


def test_stream_contexts_beyond_max_context_give_nan_not_stale_output(runner):
    # A caller that breaks the contract row_context <= max_context can make the
    # balanced schedule's tile count reach 2^31 although the host routed the
    # batch to it. The kernel then writes NaN into every output row and marks
    # every span record unwritten, so the merge keeps the NaN; no key is read.
    # A first call on the same workspace leaves valid span records behind.
    import torch

    rows, heads, kv_heads, d, block = 65535, 32, 8, 128, 128
    ctx = 4097 * 32  # 65535 rows * 8 kv heads * 4097 tiles > 2^31
    blocks_per_row = (ctx + block - 1) // block
    pool = torch.zeros(2, kv_heads, 4 * block, d, dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros(rows, blocks_per_row, dtype=torch.int32, device="cuda")
    query = torch.ones(rows, heads * d, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(rows, heads * d, dtype=torch.bfloat16, device="cuda")
    lens = torch.full((rows,), 100, dtype=torch.int32, device="cuda")
    params = runner.decode_params(query, pool, tables, lens, heads, kv_heads, d, block, 0.088, out, max_context=100)
    ws = runner.paged_decode(params)  # a valid call: every span record written
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    lens.fill_(ctx)  # max_context stays 100: the contract is broken
    import ctypes
    from gaudirt_amd import capi
    lib = capi.load()
    assert lib.gk_paged_decode_partition_tokens(ctypes.byref(params)) == 0  # routed to the balanced schedule
    need = lib.gk_paged_decode_workspace_bytes(ctypes.byref(params))
    capi.check(lib.gk_paged_decode(ctypes.byref(params), ctypes.c_void_p(ws.data_ptr()), need,
                                   capi.current_stream()))
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
