"""The oracle's OCP 8-bit float conversion (orc_f32_to_ofp8) and the fp8
page append / cache conversion built on it, pinned against the OCP OFP8
v1.0 format definitions restated here independently: the 256 codes decoded
from their fields, the nearest code found by search (ties to the even code,
i.e. the even mantissa), saturation of |x| >= max (infinities included) to
the largest finite code, NaN to 0x7f.  Inputs: every fp16 and every bf16
value, 200k random fp32 values over 2^-30 .. 2^20, every midpoint between
neighbouring codes and the floats either side of it."""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import f32_to_bf16_bits

FORMATS = {False: (3, 7, 0x7E), True: (2, 15, 0x7B)}  # e5m2 -> (mantissa bits, bias, max code)


def _code_values(e5m2):
    """Values of the positive codes 0 .. max code, from the fields."""
    M, B, maxc = FORMATS[e5m2]
    vals = []
    for c in range(maxc + 1):
        e, m = c >> M, c & ((1 << M) - 1)
        vals.append(m * 2.0 ** (1 - B - M) if e == 0 else (1 + m / 2 ** M) * 2.0 ** (e - B))
    return np.array(vals)


def _expected(x, e5m2):
    M, B, maxc = FORMATS[e5m2]
    vals = _code_values(e5m2)
    x = np.asarray(x, np.float32)
    a = np.abs(x.astype(np.float64))
    sign = np.where(np.signbit(x), 0x80, 0)
    i = np.clip(np.searchsorted(vals, a), 1, maxc)  # vals[i - 1] <= a <= vals[i] when in range
    lo, hi = vals[i - 1], vals[i]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & (i % 2 == 0))
    code = np.where(pick_hi, i, i - 1)
    code = np.where(a >= vals[maxc], maxc, code)
    out = (code | sign).astype(np.uint8)
    return np.where(np.isnan(x), 0x7F, out).astype(np.uint8)


def _inputs():
    f16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    bf16 = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    rng = np.random.default_rng(5)
    rnd = (np.exp2(rng.uniform(-30, 20, 200000)) * rng.choice([-1.0, 1.0], 200000)).astype(np.float32)
    return np.concatenate([f16, bf16, rnd])


def _midpoints(e5m2):
    vals = _code_values(e5m2)
    mid = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (vals[1:] + vals[:-1]) / 2)  # exact in fp32
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(0))
    m = np.concatenate([mid, up, dn])
    return np.concatenate([m, -m])


@pytest.mark.parametrize("e5m2", [False, True])
def test_ofp8_every_half_random_and_midpoints(e5m2):
    x = np.concatenate([_inputs(), _midpoints(e5m2)])
    got = O.ofp8_encode(x, e5m2)
    exp = _expected(x, e5m2)
    bad = np.flatnonzero(got != exp)
    assert bad.size == 0, f"{bad.size} differ, first x={x[bad[:4]]} got={got[bad[:4]]} exp={exp[bad[:4]]}"


@pytest.mark.parametrize("e5m2", [False, True])
def test_ofp8_specification_values(e5m2):
    M, B, maxc = FORMATS[e5m2]
    mx = 448.0 if not e5m2 else 57344.0
    x = np.array([0.0, -0.0, mx, -mx, np.inf, -np.inf, np.nan, 2.0 ** (1 - B - M), 2.0 ** (1 - B)], np.float32)
    got = O.ofp8_encode(x, e5m2)
    assert list(got) == [0x00, 0x80, maxc, 0x80 | maxc, maxc, 0x80 | maxc, 0x7F, 0x01, 1 << M]
    # decoding the codes gives the spec's values back (and every finite code round-trips)
    for c in range(256):
        v = O.ofp8_decode(np.uint8(c), e5m2)
        if np.isfinite(v):
            assert O.ofp8_encode(np.float32(v), e5m2) == (c if c not in (0x80,) else 0x80)
    assert O.ofp8_decode(np.uint8(maxc), e5m2) == mx


@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("src_bf16", [False, True])
def test_reshape_and_cache_fp8_layout(hnd, src_bf16):
    """Page bytes of the fp8 append: E4M3 of x / scale at the reference's NHD /
    HND offsets with a padded block stride; a negative slot writes nothing."""
    T, H, D, bs = 37, 3, 64, 16
    rng = np.random.default_rng(11 + hnd + 2 * src_bf16)
    x = (rng.standard_normal((2, T, H, D)) * 60).astype(np.float32)
    x[0, 3, 1, :4] = [1e6, -1e6, 1e-12, 0.0]
    bits = (f32_to_bf16_bits(x) if src_bf16 else x.astype(np.float16).view(np.uint16))
    vals = O.bf16_to_f32(bits) if src_bf16 else O.f16_to_f32(bits)
    nblk = 4
    stride = bs * H * D + 48
    slots = rng.permutation(nblk * bs)[:T].astype(np.int64)
    slots[5] = -1
    kc = np.full(nblk * stride, 0xAA, np.uint8)
    vc = np.full(nblk * stride, 0xAA, np.uint8)
    O.reshape_and_cache_fp8(bits[0], bits[1], slots, kc, vc, bs, k_scale=0.5, v_scale=3.0, hnd=hnd,
                            src_bf16=src_bf16, stride=stride)
    ek = np.full_like(kc, 0xAA)
    ev = np.full_like(vc, 0xAA)
    for t in range(T):
        if slots[t] < 0:
            continue
        blk, off = divmod(int(slots[t]), bs)
        for h in range(H):
            o = blk * stride + (h * bs * D + off * D if hnd else off * H * D + h * D)
            ek[o:o + D] = O.ofp8_encode(vals[0, t, h] / np.float32(0.5))
            ev[o:o + D] = O.ofp8_encode(vals[1, t, h] / np.float32(3.0))
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)


@pytest.mark.parametrize("e5m2", [False, True])
def test_convert_fp8(e5m2):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096) * 1000).astype(np.float16)
    got = O.convert_fp8(x.view(np.uint16), 0.25, e5m2=e5m2)
    assert np.array_equal(got, O.ofp8_encode(x.astype(np.float32) * np.float32(0.25), e5m2))
