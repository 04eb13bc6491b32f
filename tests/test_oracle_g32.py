"""CPU checks that pin the oracle's per-32-group TurboQuant variant
(orc_g32_*: seeded random-sign Walsh-Hadamard rotation, 4-bit codes with a
scale and a minimum per 32 values, 3-bit codes with a scale per 32 values).

The format comes from the benchmark configuration text; the reference has no
code for it, so it is pinned by hand-computed known answers (exact bytes),
nearest-level brute force of every code, error bounds, the orthogonality of
the rotation, the slot addressing of a poisoned pool, and an independent
float64 attention (numpy Hadamard matrix, plain softmax) for the decode.
"""
import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle_lib as O
from kvgen import BS

D = 128


def test_signs_seeded():
    assert np.all(O.g32_signs(0) == 1.0)
    s4, s4b, s2 = O.g32_signs(4), O.g32_signs(4), O.g32_signs(2)
    assert np.array_equal(s4, s4b)
    assert set(np.unique(s4)) == {-1.0, 1.0}
    assert 40 <= int((s4 < 0).sum()) <= 88
    assert not np.array_equal(s4, s2)


def test_signed_rotation_is_orthonormal():
    rng = np.random.default_rng(0)
    s = O.g32_signs(7)
    H = hadamard(D).astype(np.float64) / np.sqrt(D)
    for _ in range(4):
        x = rng.standard_normal(D).astype(np.float32)
        y = O.tq_rotate(x, s)
        # y = H (s x) against the matrix product, and s (H y) returns x
        np.testing.assert_allclose(y, H @ (s.astype(np.float64) * x), rtol=0, atol=2e-6)
        back = s * O.tq_rotate(y)
        np.testing.assert_allclose(back, x, rtol=0, atol=4e-6)


def test_4bit_known_answer():
    # group: 0, 1, ..., 15 then 15 x 16 -> d = 1, m = 0, codes = values
    g = np.concatenate([np.arange(16), np.full(16, 15)]).astype(np.float32)
    part = O.g32_quantize_part(np.tile(g, 4), 4)
    assert part.size == 80
    blk = part[:20]
    assert list(blk[:4]) == [0x00, 0x3C, 0x00, 0x00]          # fp16 1.0, fp16 0.0
    assert list(blk[4:]) == [0xF0 | j for j in range(16)]      # q[j] | q[j+16] << 4
    assert np.array_equal(O.g32_dequant_part(part, 4), np.tile(g, 4))


def test_3bit_known_answer():
    # group: -4, -3, ..., 3 four times -> v = -4 (first of largest |y|), d = 1,
    # codes = y + 4 = 0..7 -> 3 bytes 0x88 0xC6 0xFA per 8 codes
    g = np.tile(np.arange(-4, 4), 4).astype(np.float32)
    part = O.g32_quantize_part(np.tile(g, 4), 3)
    assert part.size == 56
    blk = part[:14]
    assert list(blk[:2]) == [0x00, 0x3C]
    assert list(blk[2:]) == [0x88, 0xC6, 0xFA] * 4
    assert np.array_equal(O.g32_dequant_part(part, 3), np.tile(g, 4))


def _f16(x):
    return np.float32(np.float16(x))


@pytest.mark.parametrize("bits", [4, 3])
def test_codes_are_nearest_levels(bits):
    """Brute force: every code is a nearest level of the group's fp32 grid,
    the stored scale/min are the fp16 roundings, and the dequantized value is
    within half a step (4-bit) or one step (3-bit) plus the fp16 rounding of
    the scale and the minimum."""
    rng = np.random.default_rng(bits)
    for trial in range(200):
        y = (rng.standard_normal(D) * rng.uniform(0.01, 3.0)).astype(np.float32)
        if trial % 50 == 0:
            y[:32] = 0.25          # constant group: d = 0
        part = O.g32_quantize_part(y, bits)
        deq = O.g32_dequant_part(part, bits)
        for g in range(4):
            x = y[32 * g:32 * g + 32].astype(np.float64)
            if bits == 4:
                blk = part[20 * g:20 * g + 20]
                d16 = np.frombuffer(blk[:2].tobytes(), np.float16)[0]
                m16 = np.frombuffer(blk[2:4].tobytes(), np.float16)[0]
                mn, mx = np.float32(x.min()), np.float32(x.max())
                d = np.float32((mx - mn) / np.float32(15.0))
                assert d16 == np.float16(d) and m16 == np.float16(mn)
                q = np.concatenate([blk[4:] & 0xF, blk[4:] >> 4]).astype(np.int64)
                levels = np.arange(16) * np.float64(d) + np.float64(mn)
                lo = 0
            else:
                blk = part[14 * g:14 * g + 14]
                d16 = np.frombuffer(blk[:2].tobytes(), np.float16)[0]
                i = int(np.argmax(np.abs(x)))
                d = np.float32(np.float32(x[i]) / np.float32(-4.0))
                assert d16 == np.float16(d)
                w = blk[2:].reshape(4, 3).astype(np.int64)
                w = w[:, 0] | (w[:, 1] << 8) | (w[:, 2] << 16)
                q = ((w[:, None] >> (3 * np.arange(8))) & 7).reshape(-1)
                levels = (np.arange(8) - 4) * np.float64(d)
                lo = -4
            if d == 0:
                assert np.all(deq[32 * g:32 * g + 32] == x)
                continue
            err = np.abs(x[:, None] - levels[None, :])
            best = err.min(axis=1)
            chosen = err[np.arange(32), q]
            # nearest level, up to the fp32 rounding of the grid arithmetic
            assert np.all(chosen <= best + 1e-5 * abs(float(d)) + 1e-7), (bits, trial, g)
            # 4-bit: the levels span [min, max], so half a step; 3-bit: the
            # levels run from -4d to 3d, one step short on the side opposite
            # the largest magnitude
            step = abs(float(d16))
            half = 0.5 if bits == 4 else 1.0
            slack = half * step + 16 * abs(float(d) - float(d16)) + abs(float(m16) - float(mn) if bits == 4 else 0) + 1e-6
            assert np.all(np.abs(deq[32 * g:32 * g + 32] - x) <= slack), (bits, trial, g)
            # the extreme values land on the end codes
            if bits == 4:
                assert q[int(np.argmin(x))] == 0 and q[int(np.argmax(x))] == 15
            else:
                assert q[int(np.argmax(np.abs(x)))] == 0
            _ = lo


@pytest.mark.parametrize("bits", [4, 3])
def test_store_slot_addressing_and_skip(bits):
    rng = np.random.default_rng(11)
    T, H = 37, 4
    P = O.g32_part_bytes(bits)
    S = 2 * P
    nblk = 5
    slots = rng.permutation(nblk * BS)[:T].astype(np.int64)
    slots[3] = -1
    k = rng.standard_normal((T, H, D)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((T, H, D)).astype(np.float16).view(np.uint16)
    cache = np.full(nblk * BS * H * S, 0xA5, np.uint8)
    O.g32_store(k, v, slots, cache, BS, bits, seed=4)
    s = O.g32_signs(4)
    touched = np.zeros(cache.size, bool)
    for t in range(T):
        if slots[t] < 0:
            continue
        blk, off = divmod(int(slots[t]), BS)
        for h in range(H):
            base = blk * BS * H * S + off * H * S + h * S
            for part, src in ((0, k), (1, v)):
                x = src[t, h].view(np.float16).astype(np.float32)
                want = O.g32_quantize_part(O.tq_rotate(x, s), bits)
                assert np.array_equal(cache[base + part * P:base + part * P + P], want)
            touched[base:base + S] = True
    assert np.all(cache[~touched] == 0xA5)


@pytest.mark.parametrize("bits", [4, 3])
def test_decode_exact_vs_independent_attention(bits):
    """orc_g32_decode_exact (rotated domain) against attention over the pages
    dequantized and rotated back with a numpy Hadamard matrix; and within the
    quantization error of attention over the original K/V."""
    rng = np.random.default_rng(20 + bits)
    B, Hq, H = 3, 8, 2
    lens = np.array([1, 37, 70])
    seed = 9
    scale = 1.0 / np.sqrt(D)
    pages = (lens + BS - 1) // BS
    nblk = int(pages.sum())
    perm = rng.permutation(nblk).astype(np.int32)
    bt = np.full((B, int(pages.max())), -1, np.int32)
    kk = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[kk:kk + pages[b]]
        kk += pages[b]
    tb = np.repeat(np.arange(B), lens)
    tp = np.concatenate([np.arange(n) for n in lens])
    slots = bt[tb, tp // BS].astype(np.int64) * BS + tp % BS
    T = slots.size
    kf = rng.standard_normal((T, H, D)).astype(np.float16)
    vf = rng.standard_normal((T, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    P = O.g32_part_bytes(bits)
    cache = np.zeros(nblk * BS * H * 2 * P, np.uint8)
    O.g32_store(kf.view(np.uint16), vf.view(np.uint16), slots, cache, BS, bits, seed)
    got = O.g32_decode_exact(q.view(np.uint16), cache, bt, lens, H, scale, BS, bits, seed)

    s = O.g32_signs(seed).astype(np.float64)
    Hm = hadamard(D).astype(np.float64) / np.sqrt(D)
    G = Hq // H
    for b in range(B):
        idx = np.where(tb == b)[0]
        for hq in range(Hq):
            h = hq // G
            K = np.zeros((idx.size, D))
            V = np.zeros((idx.size, D))
            for r, t in enumerate(idx):
                blk, off = divmod(int(slots[t]), BS)
                base = blk * BS * H * 2 * P + off * H * 2 * P + h * 2 * P
                K[r] = s * (Hm @ O.g32_dequant_part(cache[base:base + P], bits))
                V[r] = s * (Hm @ O.g32_dequant_part(cache[base + P:base + 2 * P], bits))
            sc = K @ q[b, hq].astype(np.float64) * scale
            p = np.exp(sc - sc.max())
            want = (p / p.sum()) @ V
            np.testing.assert_allclose(got[b, hq], want, rtol=0, atol=1e-9)
            # the quantized attention approximates attention over the original K/V
            Ko = kf[idx, h].astype(np.float64)
            Vo = vf[idx, h].astype(np.float64)
            so = Ko @ q[b, hq].astype(np.float64) * scale
            po = np.exp(so - so.max())
            orig = (po / po.sum()) @ Vo
            # per-element V error up to d/2 (4-bit, d ~ range/15) or d (3-bit, d ~ max/4)
            tol = 0.3 if bits == 4 else 0.8
            assert np.max(np.abs(want - orig)) < tol
