"""CPU checks that pin the oracle's fused Q/K RMSNorm + RoPE
(orc_qk_norm_rope; src/cuda/fused_attn_kernels.cu:39-313): identity and
quarter-turn rotations (exact), the rotation against complex multiplication
in float64, the RMSNorm against float64 within the element type's rounding,
per-head weights, and the neox / GPT-J pairings.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import f32_to_bf16_bits

D = 128


def _bits(x, bf16):
    return f32_to_bf16_bits(x) if bf16 else np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _vals(b, bf16):
    b = np.asarray(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32) if bf16 else b.view(np.float16).astype(np.float32)


def _cache(angles, bf16):
    """rows [pos][cos(D/2) | sin(D/2)] for angle[pos][d]"""
    return _bits(np.concatenate([np.cos(angles), np.sin(angles)], axis=1).astype(np.float32), bf16)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("neox", [True, False])
def test_identity_and_quarter_turn(bf16, neox):
    rng = np.random.default_rng(1)
    T, Hq, Hkv = 3, 4, 2
    q = _bits(rng.standard_normal((T, Hq, D)).astype(np.float32), bf16)
    k = _bits(rng.standard_normal((T, Hkv, D)).astype(np.float32), bf16)
    ang = np.zeros((2, D // 2))
    ang[1] = np.pi / 2
    cs = _cache(ang, bf16)
    cs[1, :D // 2] = 0                      # cos exactly 0 at the quarter turn
    q0, k0 = O.qk_norm_rope(q, k, None, None, cs, np.zeros(T, np.int64), 1e-6, neox, bf16)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q1, _ = O.qk_norm_rope(q, k, None, None, cs, np.ones(T, np.int64), 1e-6, neox, bf16)
    ia = np.arange(D // 2) if neox else 2 * np.arange(D // 2)
    ib = ia + D // 2 if neox else ia + 1
    x, y = _vals(q, bf16), _vals(q1, bf16)
    np.testing.assert_array_equal(y[..., ia], -x[..., ib])
    np.testing.assert_array_equal(y[..., ib], x[..., ia])


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("neox", [True, False])
def test_rotation_is_complex_product(bf16, neox):
    rng = np.random.default_rng(2)
    T, Hq, Hkv = 5, 2, 1
    q = _bits(rng.standard_normal((T, Hq, D)).astype(np.float32), bf16)
    k = _bits(rng.standard_normal((T, Hkv, D)).astype(np.float32), bf16)
    pos = rng.integers(0, 40, T)
    theta = 10000.0 ** (-np.arange(D // 2) * 2.0 / D)
    cs = _cache(np.arange(40)[:, None] * theta[None, :], bf16)
    q1, k1 = O.qk_norm_rope(q, k, None, None, cs, pos, 1e-6, neox, bf16)
    c = _vals(cs, bf16)[:, :D // 2].astype(np.float64)
    s = _vals(cs, bf16)[:, D // 2:].astype(np.float64)
    ia = np.arange(D // 2) if neox else 2 * np.arange(D // 2)
    ib = ia + D // 2 if neox else ia + 1
    for src, got in ((q, q1), (k, k1)):
        x = _vals(src, bf16).astype(np.float64)
        z = (x[..., ia] + 1j * x[..., ib]) * (c[pos] + 1j * s[pos])[:, None, :]
        g = _vals(got, bf16).astype(np.float64)
        ulp = 2.0 ** (-8 if bf16 else -11)
        # two products and a sum, each rounded in fp32, then one rounding to the
        # element type (cos and sin are the stored element-type values)
        tol = ulp * (np.abs(z) + 1e-6 * np.abs(x).max())
        assert np.all(np.abs(g[..., ia] - z.real) <= tol)
        assert np.all(np.abs(g[..., ib] - z.imag) <= tol)


@pytest.mark.parametrize("bf16", [False, True])
def test_rmsnorm_per_head_weights(bf16):
    rng = np.random.default_rng(3)
    T, Hq, Hkv, eps = 4, 3, 2, 1e-6
    q = _bits((rng.standard_normal((T, Hq, D)) * 3).astype(np.float32), bf16)
    k = _bits((rng.standard_normal((T, Hkv, D)) * 0.2).astype(np.float32), bf16)
    qw = _bits(rng.uniform(0.5, 1.5, Hq * D).astype(np.float32), bf16)
    kw = _bits(rng.uniform(0.5, 1.5, Hkv * D).astype(np.float32), bf16)
    cs = _cache(np.zeros((1, D // 2)), bf16)   # identity rotation
    q1, k1 = O.qk_norm_rope(q, k, qw, kw, cs, np.zeros(T, np.int64), eps, True, bf16)
    for src, w, got, H in ((q, qw, q1, Hq), (k, kw, k1, Hkv)):
        x = _vals(src, bf16).astype(np.float64)
        wv = _vals(w, bf16).astype(np.float64).reshape(H, D)
        ref = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * wv[None]
        g = _vals(got, bf16).astype(np.float64)
        ulp = 2.0 ** (-8 if bf16 else -11)
        # absolute floor: fp16 subnormal spacing
        np.testing.assert_allclose(g, ref, rtol=1.5 * ulp, atol=0.0 if bf16 else 2.0 ** -24)
    # no weight: the rows are only rotated (here: unchanged)
    q2, k2 = O.qk_norm_rope(q, k, None, kw, cs, np.zeros(T, np.int64), eps, True, bf16)
    assert np.array_equal(q2, q) and np.array_equal(k2, k1)
