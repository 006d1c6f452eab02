"""GPU parity of the MFMA chunked / prefix-shared prefill (gk_paged_prefill) against the CPU oracle.

Cases follow the reference's prefill coverage: chunked prefill over a cached
prefix (tests/paged_attention_same_prefix_smoke.py), the last chunked row
against a single-row decode on the same prefix
(tests/paged_attention_prefix_equivalence_smoke.py), GQA geometries, sliding
window / softcap (tests/paged_attention_generalized_smoke.py) and poisoned
unused slots (tests/multitile_paged_attention_unit_test.cpp:1722-1767).
Workload C4 (8 x 512-row chunks on a shared 2048-token prefix) is run at
full size and checked on sampled rows plus the cross-path property.
"""

import ctypes

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


def check(case, actual, rows=None, fp32_softmax=False):
    sel = np.arange(case.rows) if rows is None else np.asarray(rows)
    p = case.oracle_problem(sel)
    ref = orc.fp32_softmax_attention(p) if fp32_softmax else orc.direct_bf16_pv(p)
    got = actual[sel]
    assert np.isfinite(orc.bf16_to_f32(got)).all()
    max_abs, mean_abs = orc.check_tolerance(got, ref, MAX_ABS, MEAN_ABS)
    ulp_only = orc.ulp_allowance_count(got, ref, MAX_ABS)
    print(f"max_abs={max_abs:.3e} mean_abs={mean_abs:.3e} ulp_allowance_only={ulp_only} of {got.size}", flush=True)
    if not fp32_softmax:
        orc.isolated_errors(orc.bf16_to_f32(got), orc.fp64_bf16(p), orc.bf16_to_f32(orc.tiled_bf16_pv(p, 512)))
    return max_abs, mean_abs


@pytest.mark.parametrize("geometry", [(32, 8, 128), (8, 8, 64), (14, 2, 64), (64, 8, 128), (128, 1, 64),
                                      (4, 4, 128), (24, 3, 128)])
def test_prefill_geometries(runner, geometry):
    heads, kv_heads, d = geometry
    case = cases.PrefillCase(heads + kv_heads, heads, kv_heads, d, 64, prefixes=[0, 37, 300, 64],
                             chunks=[1, 45, 130, 77])
    print("geometry", geometry, check(case, runner.run_prefill_case(case)), flush=True)


@pytest.mark.parametrize("block_size", [1, 2, 4, 8, 16, 32, 128, 256])
def test_prefill_block_sizes(runner, block_size):
    # Blocks shorter than a 32-key step: every load instruction of a step (4
    # keys at d 128) reads its own block-table entry; below 4 keys (down to the
    # token-granular map) every lane reads its own key's entry.
    case = cases.PrefillCase(block_size, 32, 8, 128, block_size, prefixes=[5, 600, 0], chunks=[300, 31, 129])
    check(case, runner.run_prefill_case(case))


@pytest.mark.parametrize("block_size", [1, 4, 8, 16])
def test_prefill_small_blocks_head_dim_64(runner, block_size):
    case = cases.PrefillCase(50 + block_size, 14, 2, 64, block_size, prefixes=[3, 257], chunks=[140, 66])
    check(case, runner.run_prefill_case(case))


@pytest.mark.parametrize("block_size", [1, 2, 4, 16])
def test_prefill_small_blocks_window_evicted(runner, block_size):
    # Sliding window over short blocks: every slot no row sees is poisoned
    # (NaN) and the table entries of blocks wholly before every row's window
    # are -1, as after eviction. Runs of a step outside a workgroup's keys read
    # the nearest owned block, and their V rows are zeroed.
    import copy

    case = cases.PrefillCase(60 + block_size, 16, 4, 128, block_size, prefixes=[100, 0, 333, 64], chunks=[90, 200, 17, 1],
                             window=70)
    used = np.zeros(case.slots, dtype=bool)
    evicted = case.block_tables.copy()
    for s, (prefix, chunk) in enumerate(zip(case.prefixes, case.chunks)):
        first = max(0, int(prefix) - case.window + 1)
        for t in range(first, int(prefix + chunk)):
            used[case.block_tables[s, t // block_size] * block_size + t % block_size] = True
        evicted[s, :first // block_size] = -1
    case.pool[:, :, ~used, :] = 0x7fc0
    reference = copy.copy(case)
    case.block_tables = evicted
    check(reference, runner.run_prefill_case(case), fp32_softmax=True)


@pytest.mark.parametrize("geometry", [(16, 8, 256), (8, 1, 256), (6, 6, 256), (24, 2, 256), (128, 1, 256)])
@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_prefill_head_dim_256(runner, geometry, block_size):
    # head_dim 256 (the reference accepts 64, 128 and 256:
    # src/bridge/attention_plan.cpp:169): one 16-row query tile per wave,
    # 32-key steps, GQA groups 1-128 (group 128: one chunk row per workgroup).
    heads, kv_heads, d = geometry
    case = cases.PrefillCase(700 + heads + block_size, heads, kv_heads, d, block_size, prefixes=[0, 37, 300, 64],
                             chunks=[1, 45, 130, 77])
    print("geometry", geometry, "block", block_size, check(case, runner.run_prefill_case(case)), flush=True)


@pytest.mark.parametrize("variant", ["window", "softcap", "both"])
def test_prefill_head_dim_256_window_softcap(runner, variant):
    # Gemma-2-style attention: head_dim 256, logit softcap and sliding window.
    case = cases.PrefillCase(31, 16, 8, 256, 16, prefixes=[100, 0, 333], chunks=[90, 200, 17],
                             softcap=50.0 if variant != "window" else 0.0,
                             window=70 if variant != "softcap" else -1)
    check(case, runner.run_prefill_case(case), fp32_softmax=True)


def test_prefill_shared_prefix_small(runner):
    case = cases.PrefillCase(4, 32, 8, 128, 128, prefixes=[256] * 4, chunks=[64, 65, 1, 100],
                             shared_prefix_blocks=2)
    check(case, runner.run_prefill_case(case))


@pytest.mark.parametrize("block", [1, 4, 32])
@pytest.mark.parametrize("variant", ["window", "softcap"])
def test_prefill_window_and_softcap(runner, variant, block):
    case = cases.PrefillCase(9, 16, 4, 128, block, prefixes=[100, 0, 333], chunks=[90, 200, 17],
                             softcap=40.0 if variant == "softcap" else 0.0,
                             window=70 if variant == "window" else -1)
    check(case, runner.run_prefill_case(case), fp32_softmax=True)


def test_prefill_poisoned_unused_slots(runner):
    case = cases.PrefillCase(21, 32, 8, 128, 64, prefixes=[10, 70], chunks=[50, 33], num_blocks=16)
    used = np.zeros(case.slots, dtype=bool)
    for r, p in zip(case.requests, case.positions):
        for t in range(p + 1):
            used[case.block_tables[r, t // 64] * 64 + t % 64] = True
    case.pool[:, :, ~used, :] = 0x7fc0
    check(case, runner.run_prefill_case(case))


def test_prefill_rejects_bad_blocks(runner):
    from gaudirt_amd import capi
    import torch
    for d, block in [(128, 3), (64, 24), (128, 1 << 21), (128, 0)]:
        p = capi.PrefillParams()
        p.head_dim, p.q_heads, p.kv_heads, p.block_size, p.slots, p.scale = d, 8, 2, block, 1024, 0.1
        assert capi.load().gk_paged_prefill(ctypes.byref(p), None) == capi.GK_ERR_UNSUPPORTED, (d, block)
    del torch


def test_c4_prefix_shared_chunked_prefill(runner):
    """Workload C4 at full size: 8 sequences, shared 2048-token prefix
    (identical block ids 0..15 of the pool), 512-row causal chunks, 32 q / 8 kv
    heads, d 128. Sampled rows against the oracle; every chunk's last row
    against a single-row decode over the same prefix (cross-path property)."""
    import torch

    case = cases.PrefillCase(2026, 32, 8, 128, 128, prefixes=[2048] * 8, chunks=[512] * 8, shared_prefix_blocks=16)
    actual = runner.run_prefill_case(case)
    rng = np.random.default_rng(3)
    sample = np.unique(np.concatenate([case.first_rows, case.first_rows + 511,
                                       rng.integers(0, case.rows, 40)]))
    print("c4 sampled rows", check(case, actual, sample), flush=True)
    # decode of each chunk's last row over the same keys
    last = case.first_rows + case.chunks - 1
    dcase = cases.DecodeCase(case.query[last], case.pool, case.block_tables, (case.positions[last] + 1).astype(np.int32),
                             32, 8, 128, 128)
    decoded = runner.run_case(dcase)
    max_abs, _ = orc.tolerance_errors(decoded, actual[last])
    assert max_abs <= 1e-2, max_abs
    del torch
