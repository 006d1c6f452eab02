"""GPU parity of the standalone split-K merge (gk_split_k_merge).

The merge replaces gk_attn_online_merge_f32_v1 + gk_attn_online_finalize_bf16_v1
(semantics: tests/multitile_paged_attention_unit_test.cpp:684-738): partial
softmax states of disjoint key ranges combine with the log-sum-exp rule, an
empty range (m = -inf, l = 0) contributes nothing, and the result is
normalised once. The check does not restate that rule: partials are cut from
random attention problems (scores and values drawn here), and the merged
output must equal the softmax over all of the row's keys computed in binary64
(within the bf16 output gate), whatever the cut. Rows have uneven part counts,
empty parts and parts whose scores are far apart (so the merge must rescale);
slots past a row's part count hold NaN and must be ignored; a row with no part
gives zeros; the output rows are strided and the bytes between them stay
untouched.
"""

import ctypes

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def partial_states(rng, rows, heads, max_parts, d, part_counts):
    """Random problems cut into parts: (part_o, part_ml, exact [rows, heads * d])."""
    part_o = np.full((rows, heads, max_parts, d), np.nan, dtype=np.float32)
    part_ml = np.full((rows, heads, max_parts, 2), np.nan, dtype=np.float32)
    exact = np.zeros((rows, heads * d))
    for r in range(rows):
        for h in range(heads):
            n = int(rng.integers(1, 400))
            scores = rng.standard_normal(n) * 3.0
            scores[: n // 3] += rng.uniform(-40, 40)  # a distant block: parts must be rescaled
            values = rng.standard_normal((n, d))
            parts = part_counts[r]
            if parts == 0:
                continue  # no keys: the output is zero
            cuts = np.sort(rng.integers(0, n + 1, parts - 1))
            bounds = np.concatenate([[0], cuts, [n]])
            for p in range(parts):
                lo, hi = bounds[p], bounds[p + 1]
                if lo == hi:
                    part_o[r, h, p] = 0.0
                    part_ml[r, h, p] = (-np.inf, 0.0)
                    continue
                s2 = scores[lo:hi] * LOG2E           # log2 units, as the kernels keep them
                m = s2.max()
                w = np.exp2(s2 - m)
                part_o[r, h, p] = (w[:, None] * values[lo:hi]).sum(0)
                part_ml[r, h, p] = (m, w.sum())
            e = np.exp(scores - scores.max())
            exact[r, h * d:(h + 1) * d] = (e[:, None] * values).sum(0) / e.sum()
    return part_o, part_ml, exact


@pytest.mark.parametrize("d", [64, 128, 256])
def test_split_k_merge_matches_full_softmax(d):
    import torch

    from gaudirt_amd import capi

    assert torch.cuda.is_available()
    rng = np.random.default_rng(d)
    rows, heads, max_parts = 37, 6, 9
    part_counts = rng.integers(1, max_parts + 1, rows).astype(np.int32)
    part_counts[[0, 5]] = [0, max_parts]
    part_counts[7] = 1
    part_o, part_ml, exact = partial_states(rng, rows, heads, max_parts, d, part_counts)
    stride = heads * d + 24
    sentinel = np.int16(0x1234)
    out = torch.full((rows, stride), 0, dtype=torch.int16, device="cuda")
    out.fill_(int(sentinel))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    po, pm, pc = dev(part_o), dev(part_ml), dev(part_counts)
    print(f"split-K merge d={d}: rows={rows} heads={heads} parts {part_counts.tolist()}", flush=True)
    capi.check(capi.load().gk_split_k_merge(ctypes.c_void_p(po.data_ptr()), ctypes.c_void_p(pm.data_ptr()),
                                            ctypes.c_void_p(pc.data_ptr()), rows, heads, max_parts, d,
                                            ctypes.c_void_p(out.data_ptr()), stride, capi.current_stream()))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert (got[:, heads * d:] == sentinel).all(), "bytes between output rows were written"
    actual = got[:, :heads * d].view(np.uint16)
    assert np.isfinite(orc.bf16_to_f32(actual)).all()
    assert not orc.bf16_to_f32(actual[0]).any(), "a row without parts must be zero"
    want = orc.bf16_from_f64(exact)
    max_abs, mean_abs = orc.check_tolerance(actual, want, 2e-2, 2e-3)
    # Far inside the gate: the fp32 partials carry ~1e-6 relative noise (the
    # maxima are rounded to fp32), so every element is within one bf16 ulp of
    # the exact answer plus that noise.
    err = np.abs(orc.bf16_to_f32(actual).astype(np.float64) - exact)
    assert (err <= orc.bf16_ulp(exact) + 1e-5).all(), float((err - orc.bf16_ulp(exact)).max())
    exact_bits = int((actual == want).sum())
    print(f"split-K merge d={d}: max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}, "
          f"{exact_bits} of {actual.size} correctly rounded", flush=True)


def test_split_k_merge_rejects_bad_arguments():
    import torch

    from gaudirt_amd import capi

    assert torch.cuda.is_available()
    lib = capi.load()
    x = torch.zeros(64, device="cuda")
    p = ctypes.c_void_p(x.data_ptr())
    assert lib.gk_split_k_merge(p, p, p, 1, 1, 1, 96, p, 96, None) == capi.GK_ERR_UNSUPPORTED
    assert lib.gk_split_k_merge(p, p, p, 1, 2, 1, 64, p, 64, None) == capi.GK_ERR_INVALID_ARGUMENT  # stride < width
    assert lib.gk_split_k_merge(p, p, None, 1, 1, 1, 64, p, 64, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert lib.gk_split_k_merge(p, p, p, 0, 1, 1, 64, p, 64, None) == capi.GK_OK  # no rows: nothing to do
