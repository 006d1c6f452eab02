"""Pin the CPU oracle against the reference's known answers, closed forms and brute force.

Every check here is chosen so that a plausible mistake in the oracle (a dropped
scale, a wrong head or slot index, K/V swapped, a missing bf16 rounding, a
wrong merge weight) fails at least one of them.
"""

import fractions
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc


# ---------------------------------------------------------------------------
# bf16 conversions
# ---------------------------------------------------------------------------

def test_bf16_from_f32_matches_torch_rne():
    rng = np.random.default_rng(11)
    values = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.float32([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38, 1e-40, -1e-42]),
        # exact ties between two bf16 neighbours (round to even in both directions)
        (np.arange(1, 2001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    ours = orc.bf16_from_f32(values)
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    nan = orc.bf16_from_f32(np.float32([np.nan]))
    assert (nan[0] & 0x7f80) == 0x7f80 and (nan[0] & 0x7f) != 0 and (nan[0] & 0x40)


def _exact_bf16_from_f64(x):
    """Brute-force RNE of a double to bf16 through exact rationals."""
    if x == 0:
        return 0x8000 if math.copysign(1, x) < 0 else 0
    sign = 0x8000 if x < 0 else 0
    r = fractions.Fraction(abs(x))
    best = None
    # enumerate the two bf16 neighbours by scanning finite positive encodings near x
    approx = int(np.float32(min(abs(x), 3.4e38)).view(np.uint32) >> 16)
    for code in range(max(0, approx - 2), min(0x7f80, approx + 3) + 1):
        v = fractions.Fraction(float((np.uint32(code) << 16).view(np.float32))) if code < 0x7f80 else None
        if v is None:
            continue
        d = abs(v - r)
        if best is None or d < best[0] or (d == best[0] and code % 2 == 0):
            best = (d, code)
    # overflow: above the largest finite bf16 by at least half an ulp
    largest = fractions.Fraction(float((np.uint32(0x7f7f) << 16).view(np.float32)))
    half_ulp = fractions.Fraction(2) ** (127 - 8)
    if r >= largest + half_ulp:
        return sign | 0x7f80
    return sign | best[1]


def test_bf16_from_f64_known_answer_and_brute_force():
    # tests/decoder_cpu_reference_test.py:66-68: direct rounding keeps the
    # 2^-32 sticky bit that fp32 double rounding loses.
    midpoint = np.float64([1 + 2**-8 + 2**-32])
    assert orc.bf16_to_f32(orc.bf16_from_f64(midpoint))[0] == 1 + 2**-7
    assert np.float32(midpoint[0]) == np.float32(1 + 2**-8)  # fp32 first would tie to even -> 1
    rng = np.random.default_rng(5)
    samples = list(rng.standard_normal(3000) * 10.0 ** rng.integers(-45, 40, 3000))
    samples += [1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 2.0**-133, 2.0**-134, 3 * 2.0**-134,
                2.0**-126 * (1 - 2**-9), 2.0**-126 * (1 - 2**-8), 1e-45, 0.0, -0.0,
                3.3895313892515355e38, 3.3961775292304e38, 3.402e38, 1e300, -1e300]
    values = np.float64(samples)
    ours = orc.bf16_from_f64(values)
    for x, code in zip(values, ours):
        assert int(code) == _exact_bf16_from_f64(float(x)), (x, hex(code))
    with pytest.raises(ValueError):
        orc.bf16_from_f64(np.float64([1.0, np.nan]))
    with pytest.raises(ValueError):
        orc.bf16_from_f64(np.float64([np.inf]))


# ---------------------------------------------------------------------------
# KV store and indexing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("valid_rows", [0, 1, 7, 37])
def test_kv_store_targets_only_valid_rows(valid_rows):
    rng = np.random.default_rng(valid_rows + 3)
    slots, kv_heads, d, rows = 97, 3, 64, 37
    key_sentinel, value_sentinel = 0x1234, 0x4321
    pool = np.empty((2, kv_heads, slots, d), dtype=np.uint16)
    pool[0], pool[1] = key_sentinel, value_sentinel
    # strided rows (row stride > width), as the reference accepts sliced K/V
    storage_k = rng.integers(0, 65535, (rows, kv_heads * d + 8), dtype=np.uint16)
    storage_v = rng.integers(0, 65535, (rows, kv_heads * d + 8), dtype=np.uint16)
    key, value = storage_k[:, 8:], storage_v[:, 8:]
    locations = rng.permutation(slots)[:rows].astype(np.int32)
    orc.kv_store(key, value, locations, valid_rows, pool, slots, kv_heads, d)
    source_for_slot = np.full(slots, -1)
    source_for_slot[locations[:valid_rows]] = np.arange(valid_rows)
    for h in range(kv_heads):
        for s in range(slots):
            r = source_for_slot[s]
            if r >= 0:
                assert np.array_equal(pool[0, h, s], key[r, h * d:(h + 1) * d])
                assert np.array_equal(pool[1, h, s], value[r, h * d:(h + 1) * d])
            else:
                assert (pool[0, h, s] == key_sentinel).all() and (pool[1, h, s] == value_sentinel).all()


def test_tile_indices_match_attention_plan_smoke():
    # tests/attention_plan_smoke.py:20-40: two blocks (visible 6 and 17), four
    # 64-lane tasks each per (kind, head); fully masked tasks give index 0.
    requests_n, context, slots = 3, 40, 1000
    positions = np.array([3, 4, 5, *range(7, 17)], dtype=np.int32)
    row_requests = np.array([0] * 3 + [1] * 10, dtype=np.int32)
    mapping = ((np.arange(requests_n)[:, None] * 256 + np.arange(context)[None, :]) % slots).astype(np.int32)
    work = []
    for first_row, visible in ((0, 6), (3, 17)):
        for kind in range(2):
            for head in range(2):
                for key in range(0, 128, 64):
                    work.append([first_row, key, int(np.clip(visible - key, 0, 64)), (kind * 2 + head) * slots])
    out = orc.tile_indices(mapping.reshape(-1), row_requests, np.array(work), context)
    out = out.reshape(2, 2, 2, 128)
    for block, (request, visible) in enumerate(((0, 6), (1, 17))):
        for kind in range(2):
            for head in range(2):
                expected = np.full(128, (kind * 2 + head) * slots, dtype=np.int32)
                expected[:visible] += mapping[request, :visible]
                expected[64:] = 0
                assert np.array_equal(out[block, kind, head], expected)


def test_mapping_from_block_table():
    bt = np.array([[5, 2, -1], [0, 7, 3]], dtype=np.int32)
    m = orc.mapping_from_block_table(bt, 4, 12)
    assert m[0, :8].tolist() == [20, 21, 22, 23, 8, 9, 10, 11] and (m[0, 8:] == -1).all()
    assert m[1].tolist() == [0, 1, 2, 3, 28, 29, 30, 31, 12, 13, 14, 15]


# ---------------------------------------------------------------------------
# Attention references
# ---------------------------------------------------------------------------

def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _problem_from_slot_major(query, keys, values, requests, positions, mapping, heads, kv_heads, d, scale):
    """Build an oracle problem from the reference tests' slot-major [S, Hkv, d] pools."""
    pool = np.stack([_bits(keys).transpose(1, 0, 2), _bits(values).transpose(1, 0, 2)])
    return orc.Problem(_bits(query), pool, np.asarray(requests), np.asarray(positions),
                       np.asarray(mapping, dtype=np.int32), heads, kv_heads, d, scale)


def _reference_test_inputs():
    # Inputs of tests/paged_attention_reference_test.py:40-47 regenerated from its seed.
    torch.manual_seed(771)
    heads, kv_heads, d = 4, 2, 4
    query = torch.randn(3, heads * d).bfloat16()
    keys = torch.randn(13, kv_heads, d).bfloat16()
    values = torch.randn_like(keys).bfloat16()
    mapping = [[9, 2, 11, 5, 3, 10, 6, 1, 12, 4, 8, 7]]
    return _problem_from_slot_major(query, keys, values, [0, 0, 0], [1, 7, 11], mapping,
                                    heads, kv_heads, d, 0.5)


def test_tiled_equals_direct_tiled_on_reference_inputs():
    # tests/paged_attention_reference_test.py:48-50 asserts that the two tiled
    # formulations are bitwise equal. They round differently (probabilities
    # normalised before vs after the bf16 rounding): the reference's own two
    # functions differ by up to 8 bf16 ulp on these inputs under torch 2.10
    # (tests/golden/reference_vectors.npz, tests/test_golden.py, where the
    # oracle matches each of them bit for bit), so the claim is pinned here as
    # the reference's own tiled gate: per-row relative L2 within 5e-3
    # (tests/paged_attention_reference.py:68).
    p = _reference_test_inputs()
    for tile in (2, 3, 5, 16):
        a = orc.bf16_to_f32(orc.tiled_bf16_pv(p, tile)).astype(np.float64)
        b = orc.bf16_to_f32(orc.direct_tiled(p, tile)).astype(np.float64)
        rel = np.linalg.norm(a - b, axis=-1) / np.linalg.norm(b, axis=-1)
        assert rel.max() <= 5e-3, (tile, rel)


def test_references_agree_with_fp64_on_reference_inputs():
    p = _reference_test_inputs()
    fp64 = orc.fp64_bf16(p)
    direct = orc.bf16_to_f32(orc.direct_bf16_pv(p))
    for tile in (2, 3, 5, 16):
        tiled = orc.bf16_to_f32(orc.tiled_bf16_pv(p, tile))
        orc.isolated_errors(direct, fp64, tiled)
    # a single tile covering every key is the direct softmax up to one bf16 ulp
    one_tile = orc.tiled_bf16_pv(p, 16).astype(np.int32)
    assert np.abs(one_tile - orc.direct_bf16_pv(p).astype(np.int32)).max() <= 1


def _random_problem(seed, rows, heads, kv_heads, d, slots, context, scale=None):
    rng = np.random.default_rng(seed)
    query = orc.bf16_from_f32(rng.standard_normal((rows, heads * d)).astype(np.float32))
    pool = orc.bf16_from_f32(rng.standard_normal((2, kv_heads, slots, d)).astype(np.float32))
    mapping = rng.permutation(slots)[:context].astype(np.int32).reshape(1, context)
    positions = rng.integers(0, context, rows)
    return orc.Problem(query, pool, np.zeros(rows, np.int64), positions, mapping, heads, kv_heads, d,
                       scale if scale is not None else 1 / math.sqrt(d))


def _numpy_fp64(p):
    """Independent vectorised float64 attention (gather, einsum, softmax)."""
    q = orc.bf16_to_f32(p.query).astype(np.float64).reshape(p.query.shape[0], p.heads, p.head_dim)
    pool = orc.bf16_to_f32(p.pool).astype(np.float64).reshape(2, p.kv_heads, -1, p.head_dim)
    head_map = np.arange(p.heads) // (p.heads // p.kv_heads)
    out = np.zeros_like(q)
    for r in range(q.shape[0]):
        idx = p.mapping[p.requests[r], :p.positions[r] + 1]
        k = pool[0][head_map][:, idx, :]
        v = pool[1][head_map][:, idx, :]
        s = np.einsum("hd,htd->ht", q[r], k) * np.float64(np.float32(p.scale))
        w = np.exp(s - s.max(-1, keepdims=True))
        w /= w.sum(-1, keepdims=True)
        out[r] = np.einsum("ht,htd->hd", w, v)
    return out.reshape(q.shape[0], -1)


def test_fp64_matches_numpy_brute_force():
    p = _random_problem(3, rows=6, heads=8, kv_heads=2, d=64, slots=300, context=200)
    assert np.allclose(orc.fp64_attention(p), _numpy_fp64(p), rtol=1e-12, atol=1e-12)


def test_closed_forms_single_key_and_ties():
    # One visible key: the softmax is exactly 1 and the output is that value row.
    heads, kv_heads, d, slots = 4, 2, 8, 16
    rng = np.random.default_rng(1)
    pool = orc.bf16_from_f32(rng.standard_normal((2, kv_heads, slots, d)).astype(np.float32))
    query = orc.bf16_from_f32(rng.standard_normal((1, heads * d)).astype(np.float32))
    mapping = np.array([[6, 3, 9]], dtype=np.int32)
    p = orc.Problem(query, pool, [0], [0], mapping, heads, kv_heads, d, 0.3)
    for fn in (orc.direct_bf16_pv, lambda q: orc.tiled_bf16_pv(q, 2), lambda q: orc.direct_tiled(q, 2),
               orc.fp32_softmax_attention, lambda q: orc.guid_attention(q, [3], 2)):
        out = fn(p).reshape(heads, d)
        for h in range(heads):
            assert np.array_equal(out[h], pool[1, h // 2, 6]), h
    # Identical keys at two positions: weights are exactly 1/2 each.
    pool2 = pool.copy()
    pool2[0, :, 3] = pool2[0, :, 6]
    p2 = orc.Problem(query, pool2, [0], [1], mapping, heads, kv_heads, d, 0.3)
    v = orc.bf16_to_f32(pool2[1]).astype(np.float64)
    for fn in (orc.direct_bf16_pv, orc.fp32_softmax_attention):
        out = orc.bf16_to_f32(fn(p2)).reshape(heads, d)
        for h in range(heads):
            expected = orc.bf16_to_f32(orc.bf16_from_f32(
                ((v[h // 2, 6] + v[h // 2, 3]) / 2).astype(np.float32)))
            assert np.array_equal(out[h], expected)


def test_scale_and_head_mapping_are_applied():
    # Scores are a known closed form: q = a e0, k_t = b_t e0 -> s_t = a b_t scale.
    heads, kv_heads, d, slots = 4, 2, 8, 8
    a, b = 2.0, np.float32([0.5, -1.0, 1.5, 0.25])
    scale = 0.75
    pool = np.zeros((2, kv_heads, slots, d), dtype=np.uint16)
    for kvh in range(kv_heads):
        for t in range(4):
            kf = np.zeros(d, np.float32); kf[0] = b[t] * (kvh + 1)
            pool[0, kvh, t] = orc.bf16_from_f32(kf)
            pool[1, kvh, t] = orc.bf16_from_f32(np.full(d, t + 10 * kvh, np.float32))
    qf = np.zeros((1, heads * d), np.float32)
    for h in range(heads):
        qf[0, h * d] = a
    p = orc.Problem(orc.bf16_from_f32(qf), pool, [0], [3], np.array([[0, 1, 2, 3]], np.int32),
                    heads, kv_heads, d, scale)
    out = orc.fp64_attention(p).reshape(heads, d)
    for h in range(heads):
        kvh = h // 2
        s = a * b.astype(np.float64) * (kvh + 1) * scale
        w = np.exp(s - s.max()); w /= w.sum()
        assert abs(out[h, 0] - (w * (np.arange(4) + 10 * kvh)).sum()) < 1e-12
    direct = orc.bf16_to_f32(orc.direct_bf16_pv(p)).reshape(heads, d)
    assert np.abs(direct - out).max() < 0.05


@pytest.mark.parametrize("tile", [64, 128, 512])
def test_tiled_and_guid_within_gates_on_random_problem(tile):
    p = _random_problem(tile, rows=12, heads=8, kv_heads=2, d=128, slots=3000, context=2000)
    fp64 = orc.fp64_bf16(p)
    tiled = orc.bf16_to_f32(orc.tiled_bf16_pv(p, tile))
    for candidate in (orc.direct_bf16_pv(p), orc.tiled_bf16_pv(p, tile), orc.direct_tiled(p, tile),
                      orc.guid_attention(p, np.full(12, -(-2000 // tile)), tile)):
        orc.isolated_errors(orc.bf16_to_f32(candidate), fp64, tiled)


def test_guid_single_tile_is_direct_softmax():
    p = _random_problem(9, rows=10, heads=8, kv_heads=2, d=64, slots=1000, context=500)
    guid = orc.guid_attention(p, np.ones(10), 512).astype(np.int32)
    direct = orc.direct_bf16_pv(p).astype(np.int32)
    assert np.abs(guid - direct).max() <= 1


def test_softcap_and_window_follow_generalized_reference():
    p = _random_problem(21, rows=8, heads=8, kv_heads=4, d=64, slots=400, context=300)
    p.softcap, p.sliding_window = 30.0, 64
    out64 = orc.fp64_attention(p)
    # brute force: cap the scores and keep only the last `window` keys
    q = orc.bf16_to_f32(p.query).astype(np.float64).reshape(8, 8, 64)
    pool = orc.bf16_to_f32(p.pool).astype(np.float64)
    for r in range(8):
        pos = p.positions[r]
        left = max(0, pos - 64 + 1)
        idx = p.mapping[0, left:pos + 1]
        for h in range(8):
            s = pool[0, h // 2, idx] @ q[r, h] * np.float64(np.float32(p.scale))
            s = 30.0 * np.tanh(s / 30.0)
            w = np.exp(s - s.max()); w /= w.sum()
            assert np.allclose(out64[r, h * 64:(h + 1) * 64], w @ pool[1, h // 2, idx], atol=1e-12)
    approx = orc.bf16_to_f32(orc.fp32_softmax_attention(p))
    assert np.abs(approx - out64).max() < 2e-2


def test_isolated_errors_known_answers():
    # tests/paged_attention_reference_test.py:52-59. Its rejection of
    # (candidate, fp64, fp64) needs the device tests' 1e-3 tiled gate: the
    # tiled error there is 3.9e-3, inside the 5e-3 gate of
    # tests/paged_attention_reference.py:68.
    fp64 = np.array([[1.0, 0.2]])
    candidate = np.array([[1.004, 0.2]])
    e64, et = orc.isolated_errors(candidate, fp64, candidate)
    assert 3e-3 < e64 < 1e-2 and et == 0
    _, et = orc.isolated_errors(candidate, fp64, fp64)
    assert 3e-3 < et < 5e-3
    with pytest.raises(AssertionError):
        orc.isolated_errors(candidate, fp64, fp64, tiled_gate=1e-3)
    for bad in ((np.array([[1.02, 0.2]]), fp64, np.array([[1.02, 0.2]])),
                (np.array([[np.nan, 0.2]]), fp64, fp64)):
        with pytest.raises(AssertionError):
            orc.isolated_errors(*bad)


def test_reference_tiling_policy_matches_unit_test_plans():
    # tests/multitile_paged_attention_unit_test.cpp:1509-1586 (56 q heads, 8 kv heads, d 128)
    for ctx in (128, 1025, 4096, 4097):
        assert orc.reference_tiles_per_row([(0, 1, ctx - 1)], 56, 8, 128, 1).tolist() == [1]
    tiles = orc.reference_tiles_per_row([(0, 1024, 0)], 56, 8, 128, 1024)
    assert [tiles[b * 256] for b in range(4)] == [1, 1, 2, 2]
    tiles = orc.reference_tiles_per_row([(0, 4096, 0)], 56, 8, 128, 4096)
    assert [tiles[b * 512] for b in range(8)] == list(range(1, 9))
    tiles = orc.reference_tiles_per_row([(0, 4096, 28672)], 56, 8, 128, 4096)
    assert tiles[-1] == 64 and tiles[0] == 57


def test_bf16_ulp_and_tolerance_gate():
    assert orc.bf16_ulp(np.float64([1.0, 1.5, 2.0, 3.99, 4.0, 7.9, -4.0]))[[0, 1, 2, 3, 4, 5, 6]].tolist() == [
        2 ** -7, 2 ** -7, 2 ** -6, 2 ** -6, 2 ** -5, 2 ** -5, 2 ** -5]
    ref = orc.bf16_from_f32(np.float32([4.0, 1.0, 0.5]))
    one_ulp_up = orc.bf16_from_f32(np.float32([4.03125, 1.0, 0.5]))
    orc.check_tolerance(one_ulp_up, ref, 2e-2, 2e-2)  # one ulp at |x| >= 4 is allowed
    two_ulp_up = orc.bf16_from_f32(np.float32([4.0625, 1.0, 0.5]))
    with pytest.raises(AssertionError):
        orc.check_tolerance(two_ulp_up, ref, 2e-2, 2e-2)
    off_small = orc.bf16_from_f32(np.float32([4.0, 1.03125, 0.5]))  # 0.031 at |x| = 1 breaks 2e-2
    with pytest.raises(AssertionError):
        orc.check_tolerance(off_small, ref, 2e-2, 2e-2)


def test_flat_gate_known_answers():
    # The literal benchmark gate: 2e-2 flat, no ulp allowance.
    ref = orc.bf16_from_f32(np.float32([0.5, 1.0, -2.0, 0.0]))
    # 163 / 8192 and 164 / 8192: the bf16 numbers on either side of 0.02.
    at_bound = orc.bf16_from_f32(np.float32([0.5, 1.0, -2.0, 163 / 8192]))
    orc.check_flat_gate(at_bound, ref, 2e-2, 2e-2)
    over = orc.bf16_from_f32(np.float32([0.5, 1.0, -2.0, 164 / 8192]))
    with pytest.raises(AssertionError):
        orc.check_flat_gate(over, ref, 2e-2, 2e-2)
    # One ulp at |x| >= 4 passes check_tolerance but not the flat gate.
    big = orc.bf16_from_f32(np.float32([4.0]))
    big_up = orc.bf16_from_f32(np.float32([4.03125]))
    orc.check_tolerance(big_up, big, 2e-2, 5e-2)
    with pytest.raises(AssertionError):
        orc.check_flat_gate(big_up, big, 2e-2, 5e-2)
    with pytest.raises(AssertionError):
        orc.check_flat_gate(orc.bf16_from_f32(np.float32([np.nan])), big, 2e-2, 2e-2)
    # The mean bound: 0.015 on every element is within max_abs but not a 2e-3 mean.
    base = orc.bf16_from_f32(np.float32([0.25] * 8))
    shifted = orc.bf16_from_f32(np.float32([0.265625] * 8))
    with pytest.raises(AssertionError):
        orc.check_flat_gate(shifted, base, 2e-2, 2e-3)
    assert orc.check_flat_gate(shifted, base, 2e-2, 2e-2) == (0.015625, 0.015625)


def test_exact_answer_is_one_ulp_from_direct_bf16_pv_at_large_outputs():
    """Why the output gate allows one bf16 ulp where it exceeds 2e-2: on the
    nanbeige-geometry case of the device tests (56 q / 8 kv heads, d 128,
    137 rows, seed 3127 + 137), the fp64 attention rounded once to bf16 differs
    from the reference's direct_bf16_pv by 0.03125 at an output of magnitude 4."""
    heads, kv_heads, dim, requests_n, context, rows = 56, 8, 128, 64, 32, 137
    gen = torch.Generator().manual_seed(3127 + rows)
    slots = requests_n * context + 1
    scale = float(np.float32(1 / math.sqrt(dim)))
    mapping = torch.arange(1, slots, dtype=torch.int32).reshape(requests_n, context)
    req = torch.arange(rows) % requests_n
    pos = torch.arange(rows) // requests_n + 3
    loc = mapping[req, pos].to(torch.int64)

    def rn(*shape):
        return torch.randn(*shape, generator=gen).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)

    q, k, v = rn(rows, heads * dim), rn(rows, kv_heads * dim), rn(rows, kv_heads * dim)
    kb, vb = rn(slots, kv_heads, dim), rn(slots, kv_heads, dim)
    pool = np.stack([kb, vb]).transpose(0, 2, 1, 3).copy()
    orc.kv_store(k, v, loc.numpy(), rows, pool, slots, kv_heads, dim)
    p = orc.Problem(q, pool, req.numpy(), pos.numpy(), mapping.numpy(), heads, kv_heads, dim, scale)
    direct = orc.direct_bf16_pv(p)
    exact = orc.bf16_from_f64(orc.fp64_attention(p))
    max_abs, _ = orc.tolerance_errors(exact, direct)
    assert max_abs == 0.03125
    worst = np.argmax(np.abs(orc.bf16_to_f32(exact) - orc.bf16_to_f32(direct)))
    assert abs(orc.bf16_to_f32(direct).flat[worst]) >= 4.0
    orc.check_tolerance(exact, direct)
