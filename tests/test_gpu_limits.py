"""GPU parity at the pool-size limit.

The kernels address one kv head's K (or V) region with 32-bit buffer offsets,
so the library accepts pools up to slots * head_dim * 2 < 2^32 bytes per
region (gk_paged_decode / gk_paged_prefill reject larger ones). These cases
use the largest such pool at head_dim 128 (16,777,088 slots, an 8 GiB pool for
one kv head), and at head_dim 256, and put every attended block among the last
blocks of the pool, where the offsets are largest. The oracle sees the same blocks renumbered
into a compact pool.
"""

import numpy as np
import pytest

from oracle import oracle as orc
from tests import paged_cases as cases

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
D, HKV, HQ, BLOCK = 128, 1, 8, 128
SLOTS = ((2**32 - 1) // (D * 2)) // BLOCK * BLOCK


@pytest.fixture(scope="module")
def big_pool():
    import torch
    assert torch.cuda.is_available()
    pool = torch.empty((2, HKV, SLOTS, D), dtype=torch.bfloat16, device="cuda")
    yield pool
    del pool
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def big_pool_256():
    """The largest pool at head_dim 256 (8,388,480 slots, also 8 GiB for one kv head)."""
    import torch
    assert torch.cuda.is_available()
    pool = torch.empty((2, HKV, SLOTS_256, 256), dtype=torch.bfloat16, device="cuda")
    yield pool
    del pool
    torch.cuda.empty_cache()


SLOTS_256 = ((2**32 - 1) // (256 * 2)) // BLOCK * BLOCK


def to_big(pool, small_pool, small_tables, seed):
    """Copy the compact pool's blocks to the last blocks of the big pool (shuffled); return the big tables."""
    import torch
    from tests import gk_runner as runner

    slots, d = pool.shape[2], pool.shape[3]
    blocks = small_pool.shape[2] // BLOCK
    ids = slots // BLOCK - 1 - np.random.default_rng(seed).permutation(blocks)
    view = pool.view(2, HKV, slots // BLOCK, BLOCK, d)
    view[:, :, torch.from_numpy(ids).cuda()] = runner.bf16_device(small_pool).view(2, HKV, blocks, BLOCK, d)
    torch.cuda.synchronize()
    return np.where(small_tables >= 0, ids[np.maximum(small_tables, 0)], -1).astype(np.int32)


def test_region_limit_is_enforced():
    import ctypes
    import torch
    from gaudirt_amd import capi
    assert torch.cuda.is_available()
    assert SLOTS * D * 2 < 2**32 <= (SLOTS + BLOCK) * D * 2
    p = capi.PrefillParams()
    p.head_dim, p.q_heads, p.kv_heads, p.block_size, p.slots, p.scale = D, HQ, HKV, BLOCK, SLOTS + BLOCK, 0.1
    assert capi.load().gk_paged_prefill(ctypes.byref(p), None) == capi.GK_ERR_UNSUPPORTED


@pytest.mark.parametrize("partition", [0, 256])
def test_decode_at_the_end_of_the_largest_pool(big_pool, partition):
    import torch
    from tests import gk_runner as runner

    lens = np.array([1, 300, 2049, 777], dtype=np.int32)
    need = int(((lens + BLOCK - 1) // BLOCK).sum())
    case = cases.decode_case(3, len(lens), HQ, HKV, D, BLOCK, need, lens)
    tables = to_big(big_pool, case.pool, case.block_tables, 11)
    out = torch.full((len(lens), HQ * D), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.decode_params(runner.bf16_device(case.query), big_pool, runner.to_device(tables),
                                  runner.to_device(lens), HQ, HKV, D, BLOCK, case.scale, out, partition=partition)
    ws = runner.paged_decode(params)
    torch.cuda.synchronize()
    del ws
    got = runner.bits_of(out)
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    print("partition", partition, orc.check_tolerance(got, orc.direct_bf16_pv(case.oracle_problem(), 16),
                                                       MAX_ABS, MEAN_ABS), flush=True)


def test_prefill_at_the_end_of_the_largest_pool(big_pool):
    import ctypes
    import torch
    from gaudirt_amd import capi
    from tests import gk_runner as runner

    case = cases.PrefillCase(7, HQ, HKV, D, BLOCK, prefixes=[300, 0], chunks=[200, 129])
    tables = to_big(big_pool, case.pool, case.block_tables, 13)
    seqs = len(case.chunks)
    out = torch.full((case.rows, HQ * D), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.prefill_params(runner.bf16_device(case.query), big_pool, runner.to_device(tables),
                                   runner.to_device(np.arange(seqs, dtype=np.int32)),
                                   runner.to_device(case.first_rows), runner.to_device(case.chunks),
                                   runner.to_device(case.prefixes), HQ, HKV, D, BLOCK, case.scale, out,
                                   int(case.chunks.max()))
    capi.check(capi.load().gk_paged_prefill(ctypes.byref(params), capi.current_stream()))
    torch.cuda.synchronize()
    got = runner.bits_of(out)
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    print(orc.check_tolerance(got, orc.direct_bf16_pv(case.oracle_problem()), MAX_ABS, MEAN_ABS), flush=True)


def test_head_dim_256_at_the_end_of_the_largest_pool(big_pool_256):
    # The same at head_dim 256, whose regions reach the 32-bit limit with half
    # the slots: a decode batch and a chunked prefill over the last blocks.
    import ctypes
    import torch
    from gaudirt_amd import capi
    from tests import gk_runner as runner

    d = 256
    assert SLOTS_256 * d * 2 < 2**32 <= (SLOTS_256 + BLOCK) * d * 2
    lens = np.array([1, 300, 2049, 777], dtype=np.int32)
    need = int(((lens + BLOCK - 1) // BLOCK).sum())
    case = cases.decode_case(5, len(lens), HQ, HKV, d, BLOCK, need, lens)
    tables = runner.to_device(to_big(big_pool_256, case.pool, case.block_tables, 17))
    query, d_lens = runner.bf16_device(case.query), runner.to_device(lens)
    out = torch.full((len(lens), HQ * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.decode_params(query, big_pool_256, tables, d_lens, HQ, HKV, d, BLOCK, case.scale, out)
    ws = runner.paged_decode(params)
    torch.cuda.synchronize()
    del ws
    got = runner.bits_of(out)
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    print("decode", orc.check_tolerance(got, orc.direct_bf16_pv(case.oracle_problem(), 16), MAX_ABS, MEAN_ABS),
          flush=True)

    case = cases.PrefillCase(9, HQ, HKV, d, BLOCK, prefixes=[300, 0], chunks=[200, 129])
    seqs = len(case.chunks)
    tables = runner.to_device(to_big(big_pool_256, case.pool, case.block_tables, 19))
    query = runner.bf16_device(case.query)
    seq_args = [runner.to_device(x) for x in (np.arange(seqs, dtype=np.int32), case.first_rows, case.chunks,
                                              case.prefixes)]
    out = torch.full((case.rows, HQ * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = runner.prefill_params(query, big_pool_256, tables, *seq_args, HQ, HKV, d, BLOCK, case.scale, out,
                                   int(case.chunks.max()))
    capi.check(capi.load().gk_paged_prefill(ctypes.byref(params), capi.current_stream()))
    torch.cuda.synchronize()
    got = runner.bits_of(out)
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    print("prefill", orc.check_tolerance(got, orc.direct_bf16_pv(case.oracle_problem()), MAX_ABS, MEAN_ABS),
          flush=True)
