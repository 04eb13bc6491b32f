"""CPU checks that pin the oracle's turboquant_k8v4 path (fp8 keys,
src/cuda/turboquant_kernels.cu:47-143 converters, :188-245 store, :407-415
decode): hand-computed codes of the reference's encoder (including its
mantissa carry: the mantissa is taken as (m + 2^18) >> 19, four bits, and a
value > 7 carries into the exponent, so 1.25 is stored as 1.5 and 1.5 as
2.0), every one of the 256 codes decoded against the closed form
(1 + m/8) 2^(e - bias), sign symmetry, the V part equal byte for byte to the
4-bit method's, and the decode against an independent float64 attention
(no rotation, no norm).
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS

D = 128


@pytest.mark.parametrize("e4b15", [False, True])
def test_decode_all_codes_closed_form(e4b15):
    b = np.arange(256, dtype=np.uint8)
    got = O.fp8_decode(b, e4b15)
    e, m, s = (b >> 3) & 15, b & 7, b >> 7
    want = (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - (15 if e4b15 else 7))
    want[(e == 0) & (m == 0)] = 0.0
    want = np.where(s == 1, -want, want)
    assert np.array_equal(got.astype(np.float64), want)
    assert np.signbit(got[0x80]) and not np.signbit(got[0])


def test_encode_known_answers_e4m3():
    cases = [(0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (-2.0, 0xC0), (1.125, 0x3A), (1.25, 0x3C),
             (1.5, 0x40), (448.0, 0x7F), (1e6, 0x7F), (float("inf"), 0x7C), (float("-inf"), 0xFC),
             (2.0 ** -7, 0x0F), (2.0 ** -40, 0x00)]
    for x, code in cases:
        assert int(O.fp8_encode([x])[0]) == code, (x, hex(code))
    # the carry: 1.25 reads back as 1.5, 1.5 as 2.0
    assert O.fp8_decode(O.fp8_encode([1.25, 1.5])).tolist() == [1.5, 2.0]


def test_encode_known_answers_e4b15():
    cases = {1.0: 0x78, 0.5: 0x70, 2.0: 0x7F, -0.75: 0xF8, float("inf"): 0x78}  # -0.75 = -1.5 2^-1 carries
    for x, code in cases.items():
        assert int(O.fp8_encode([x], True)[0]) == code, (x, hex(code))


@pytest.mark.parametrize("e4b15", [False, True])
def test_sign_symmetry_and_monotone(e4b15):
    rng = np.random.default_rng(1)
    x = np.abs(rng.standard_normal(3000).astype(np.float32)) * (0.5 if e4b15 else 40.0)
    x = np.sort(x)
    p, n = O.fp8_encode(x, e4b15), O.fp8_encode(-x, e4b15)
    assert np.array_equal(n, p | 0x80)
    r = O.fp8_decode(p, e4b15)
    assert np.all(np.diff(r) >= 0)
    # stored values are never below the input by more than one step of 1/8
    # nor above it by more than the carry (< 2x) -- the encoder's bounds
    big = x > (2.0 ** -5 if e4b15 else 2.0 ** 3)
    assert np.all(r[big] >= x[big] * (1 - 1 / 8) - 1e-12) and np.all(r[big] <= 2 * x[big])


def _pool(seed, T=37, H=4, nblk=5):
    rng = np.random.default_rng(seed)
    slots = rng.permutation(nblk * BS)[:T].astype(np.int64)
    slots[3] = -1
    k = (rng.standard_normal((T, H, D)) * 2).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((T, H, D)).astype(np.float16).view(np.uint16)
    return rng, slots, k, v, nblk, H


def test_store_layout_and_v_part():
    _, slots, k, v, nblk, H = _pool(3)
    L8, L4 = O.tq_layout("turboquant_k8v4"), O.tq_layout("turboquant_4bit_nc")
    assert (L8.mse_bytes, L8.key_packed_size, L8.slot_size_aligned) == (128, 128, 196)
    c8 = np.full(nblk * BS * H * 196, 0xA5, np.uint8)
    c4 = np.zeros(nblk * BS * H * L4.slot_size_aligned, np.uint8)
    _, mid = O.tq_tables(D, 4)
    O.tq_store(k, v, slots, c8, BS, L8, mid)
    O.tq_store(k, v, slots, c4, BS, L4, mid)
    touched = np.zeros(c8.size, bool)
    for t in range(slots.size):
        if slots[t] < 0:
            continue
        blk, off = divmod(int(slots[t]), BS)
        for h in range(H):
            b8 = (blk * BS * H + off * H + h) * 196
            b4 = (blk * BS * H + off * H + h) * L4.slot_size_aligned
            kk = k[t, h].view(np.float16).astype(np.float32)
            assert np.array_equal(c8[b8:b8 + 128], O.fp8_encode(kk))
            assert np.array_equal(c8[b8 + 128:b8 + 196], c4[b4 + 66:b4 + 134])
            touched[b8:b8 + 196] = True
    assert np.all(c8[~touched] == 0xA5)


@pytest.mark.parametrize("e4b15", [False, True])
def test_decode_exact_vs_independent(e4b15):
    rng, _, _, _, _, _ = _pool(4)
    B, Hq, H = 3, 8, 2
    lens = np.array([1, 40, 70])
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
    scale_k = 0.25 if e4b15 else 1.0
    kf = (rng.standard_normal((T, H, D)) * scale_k).astype(np.float16)
    vf = rng.standard_normal((T, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    L = O.tq_layout("turboquant_k8v4")
    L.fp8_e4b15 = int(e4b15)
    cache = np.zeros(nblk * BS * H * 196, np.uint8)
    _, mid = O.tq_tables(D, 4)
    O.tq_store(kf.view(np.uint16), vf.view(np.uint16), slots, cache, BS, L, mid)
    c, _ = O.tq_tables(D, 4)
    scale = 1.0 / np.sqrt(D)
    got = O.tq_decode_exact(q.view(np.uint16), cache, bt, lens.astype(np.int32), H, scale, BS, L, c)
    G = Hq // H
    for b in range(B):
        idx = np.where(tb == b)[0]
        for hq in range(Hq):
            h = hq // G
            K = np.zeros((idx.size, D))
            V = np.zeros((idx.size, D))
            for r, t in enumerate(idx):
                blk, off = divmod(int(slots[t]), BS)
                base = (blk * BS * H + off * H + h) * 196
                sl = cache[base:base + 196]
                K[r] = O.fp8_decode(sl[:128], e4b15)
                sc = np.frombuffer(sl[192:194].tobytes(), np.float16)[0]
                zr = np.frombuffer(sl[194:196].tobytes(), np.float16)[0]
                codes = np.stack([sl[128:192] & 15, sl[128:192] >> 4], 1).reshape(-1)
                V[r] = codes * np.float64(sc) + np.float64(zr)
            s = K @ q[b, hq].astype(np.float64) * scale
            p = np.exp(s - s.max())
            np.testing.assert_allclose(got[b, hq], (p / p.sum()) @ V, rtol=0, atol=1e-9)
