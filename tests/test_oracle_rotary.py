"""Pins the oracle's rotary restatement (tests/rotary_runtime_smoke.py:34-60 of the
reference) without importing the reference: closed forms, an independent brute
force with complex products, and the reference's own fp64 acceptance gate on the
shapes its test uses."""

import numpy as np
import pytest

from oracle import oracle as orc


def bf16(rng, shape, scale=1.0):
    return orc.bf16_from_f32((rng.standard_normal(shape) * scale).astype(np.float32))


def table(cos, sin):
    """cos/sin cache rows (bf16 bits) from float arrays [positions, half]."""
    return orc.bf16_from_f32(np.concatenate([cos, sin], axis=-1).astype(np.float32))


@pytest.mark.parametrize("neox", [True, False])
def test_closed_forms(neox):
    rng = np.random.default_rng(1)
    rows, heads, d, rot = 5, 3, 16, 12
    x = bf16(rng, (rows, heads * d))
    half = rot // 2
    cache = table(np.stack([np.ones(half), np.zeros(half), -np.ones(half)]),
                  np.stack([np.zeros(half), np.ones(half), np.zeros(half)]))
    # Identity (cos 1, sin 0).
    assert np.array_equal(orc.rotary_bf16(x, cache, np.zeros(rows), d, rot, neox), x)
    # Quarter turn: (a, b) -> (-b, a); half turn: negation. Sign flips are exact in bf16.
    xr = x.reshape(rows, heads, d)
    a, b = (xr[..., :half], xr[..., half:rot]) if neox else (xr[..., 0:rot:2], xr[..., 1:rot:2])
    out = orc.rotary_bf16(x, cache, np.ones(rows), d, rot, neox).reshape(rows, heads, d)
    oa, ob = (out[..., :half], out[..., half:rot]) if neox else (out[..., 0:rot:2], out[..., 1:rot:2])
    assert np.array_equal(oa, b ^ 0x8000) and np.array_equal(ob, a)
    assert np.array_equal(out[..., rot:], xr[..., rot:])
    out = orc.rotary_bf16(x, cache, np.full(rows, 2), d, rot, neox).reshape(rows, heads, d)
    oa, ob = (out[..., :half], out[..., half:rot]) if neox else (out[..., 0:rot:2], out[..., 1:rot:2])
    assert np.array_equal(oa, a ^ 0x8000) and np.array_equal(ob, b ^ 0x8000)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("d,rot", [(8, 8), (10, 6), (12, 4)])
def test_brute_force_complex(neox, d, rot):
    # (a + ib)(cos + i sin) in Python complex arithmetic: bf16 x bf16 products and
    # their sum are exact in binary64, so float32() then bf16 rounds exactly as
    # the fp32 reference does. Pairs follow the layout's definition directly.
    rng = np.random.default_rng(d * 10 + rot + neox)
    rows, heads, ctx = 4, 2, 7
    x = bf16(rng, (rows, heads * d))
    cache = bf16(rng, (ctx, rot))
    pos = rng.integers(0, ctx, rows)
    got = orc.rotary_bf16(x, cache, pos, d, rot, neox)
    xf, cf = orc.bf16_to_f32(x), orc.bf16_to_f32(cache)
    half = rot // 2
    for r in range(rows):
        for h in range(heads):
            base = h * d
            want = list(x[r, base:base + d])
            for i in range(half):
                i0, i1 = (i, i + half) if neox else (2 * i, 2 * i + 1)
                z = complex(float(xf[r, base + i0]), float(xf[r, base + i1])) * complex(
                    float(cf[pos[r], i]), float(cf[pos[r], half + i]))
                want[i0], want[i1] = orc.bf16_from_f32(np.array([z.real, z.imag], dtype=np.float32))
            assert np.array_equal(got[r, base:base + d], np.array(want, dtype=np.uint16)), (r, h)


@pytest.mark.parametrize("q_heads,k_heads,d,rot,neox,rows", [
    (56, 8, 128, 128, True, 33), (56, 8, 128, 128, False, 7), (4, 2, 96, 62, True, 7), (4, 2, 96, 62, False, 7)])
def test_reference_gate_on_reference_shapes(q_heads, k_heads, d, rot, neox, rows):
    # tests/rotary_runtime_smoke.py:83-85 shapes; the fp32 form passes its own
    # gate with error == floor, and a plausible mistake (cos and sin swapped) fails it.
    rng = np.random.default_rng(1403 + rows)
    cache = bf16(rng, (64, rot))
    pos = np.arange(rows) // 64 + 3
    for width in (q_heads * d, k_heads * d):
        x = bf16(rng, (rows, width))
        got = orc.rotary_bf16(x, cache, pos, d, rot, neox)
        err, floor = orc.rotary_gate(got, x, cache, pos, d, rot, neox)
        assert err == floor
        swapped = np.concatenate([cache[:, rot // 2:], cache[:, :rot // 2]], axis=1)
        with pytest.raises(AssertionError):
            orc.rotary_gate(orc.rotary_bf16(x, swapped, pos, d, rot, neox), x, cache, pos, d, rot, neox)
