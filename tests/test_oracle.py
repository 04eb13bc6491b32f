"""CPU checks that pin the oracle (oracle/vmc_oracle.c) before it is trusted
as the checker of the HIP kernels.

Each oracle function is checked against something it does not restate:
golden vectors written by the reference's own code (tests/golden/, from the
vendored ggml built in oracle/_ref), the live reference build when present,
closed forms (Hadamard matrix, Max's Gaussian quantizer tables), invariants
(split-count and block-table permutation invariance, round trips) and
brute force in float64.
"""
import json
import os

import numpy as np
import pytest

import kvgen
import oracle_lib as O
from kvgen import BS, close_report

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D = 128
ATOL, RTOL = 2e-3, 1e-2


def gold(name):
    return np.load(os.path.join(GOLD, name))


# ------------------------------------------------------------ conversions

def test_f16_conversions_exhaustive():
    L = O.lib()
    bits = np.arange(1 << 16, dtype=np.uint16)
    f = np.zeros(bits.size, np.float32)
    L.orc_f16_to_f32_n(O._ptr(bits), O._ptr(f), bits.size)
    ref = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(f[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.isnan(f[~np.isfinite(ref) & np.isnan(ref)]).all()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-6, 1, 3e4)])
    # exact midpoints between fp16 neighbours: round half to even
    mid = ((bits[:31000].view(np.float16).astype(np.float64) +
            bits[1:31001].view(np.float16).astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([x, mid])
    x = x[np.abs(x) < 65504]
    y = np.zeros(x.size, np.uint16)
    L.orc_f32_to_f16_n(O._ptr(x), O._ptr(y), x.size)
    assert np.array_equal(y, x.astype(np.float16).view(np.uint16))


def test_bf16_conversion_matches_torch():
    import torch
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * s for s in (1e-30, 1, 1e30)])
    got = np.array([O.lib().orc_f32_to_bf16(float(v)) for v in x[:3000]], np.uint16)
    ref = torch.from_numpy(x[:3000]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------ GGUF blocks

@pytest.mark.parametrize("fmt,name", [(O.KV_Q8_0, "quant_q8_0.npz"), (O.KV_Q4_0, "quant_q4_0.npz")])
def test_quantizer_golden(fmt, name):
    g = gold(name)
    got = O.quantize_rows(fmt, g["x"])
    assert np.array_equal(got, g["ref"])
    # the CPU set_rows encoder of this reference build is the _ref routine
    assert np.array_equal(g["from_float"], g["ref"])


@pytest.mark.parametrize("fmt", [O.KV_Q8_0, O.KV_Q4_0])
def test_quantizer_error_bound(fmt):
    """Dequantized values lie within half a step (q8_0) / one step (q4_0,
    whose +8.5 truncation rounds half up) of the input; the fp16 scale is
    the block's max magnitude over 127 (or its signed max over -8)."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(32 * 400) * np.repeat(rng.uniform(0.01, 50, 400), 32)).astype(np.float32)
    q = O.quantize_rows(fmt, x)
    y = O.dequantize_rows(fmt, q, x.size)
    E = 34 if fmt == O.KV_Q8_0 else 18
    d = q.reshape(-1, E)[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    xb = x.reshape(-1, 32).astype(np.float64)
    err = np.abs(y.reshape(-1, 32) - xb).max(axis=1)
    # codes use the fp32 step d32, the block stores it rounded to fp16
    if fmt == O.KV_Q8_0:
        d32 = np.abs(xb).max(axis=1) / 127
        assert np.allclose(d, d32, rtol=1e-3)
        assert (err <= 0.5 * d32 * (1 + 1e-6) + 127 * np.abs(d32 - d) + 1e-30).all()
    else:
        idx = np.abs(xb).argmax(axis=1)
        d32 = np.abs(xb[np.arange(len(xb)), idx] / -8)
        assert np.allclose(np.abs(d), d32, rtol=1e-3)
        assert (err <= d32 * (1 + 1e-6) + 8 * np.abs(d32 - np.abs(d))).all()


@pytest.mark.ref
@pytest.mark.skipif(not O.ref_available(), reason="reference build absent (needs the reference sources)")
@pytest.mark.parametrize("fmt", [O.KV_Q8_0, O.KV_Q4_0])
def test_quantizer_vs_live_reference(fmt):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 5000) * np.repeat(rng.uniform(1e-3, 1e3, 5000), 32)).astype(np.float32)
    x[::97] = 0.0
    assert np.array_equal(O.quantize_rows(fmt, x), O.ref_quantize(fmt, x))


def test_kv_append_layouts_and_skip():
    """Every written entry decodes to the quantized input row; slots < 0 and
    unreferenced bytes stay untouched; HND is NHD with token and head
    swapped inside each page."""
    w = kvgen.make_workload([37, 70], Hq=4, Hkv=2, seed=5, pool_slack=2)
    slots = w.slots.copy()
    slots[3] = -1
    for fmt in (O.KV_F16, O.KV_Q8_0, O.KV_Q4_0):
        E = O.entry_bytes(fmt, D)
        n = w.num_blocks * BS * w.Hkv * E
        pools = {}
        for hnd in (False, True):
            kc = np.full(n, 0xAB, np.uint8)
            vc = np.full(n, 0xAB, np.uint8)
            O.kv_append(w.K.view(np.uint16), w.V.view(np.uint16), slots, kc, vc, BS, fmt, hnd=hnd)
            pools[hnd] = (kc, vc)
        nhd = pools[False][0].reshape(w.num_blocks, BS, w.Hkv, E)
        hnd = pools[True][0].reshape(w.num_blocks, w.Hkv, BS, E)
        assert np.array_equal(nhd, hnd.transpose(0, 2, 1, 3))
        written = np.zeros((w.num_blocks, BS), bool)
        for t, s in enumerate(slots):
            if s < 0:
                continue
            blk, off = divmod(int(s), BS)
            written[blk, off] = True
            for h in range(w.Hkv):
                ent = nhd[blk, off, h]
                row = w.K[t, h].astype(np.float32)
                if fmt == O.KV_F16:
                    assert np.array_equal(ent.view(np.uint16), w.K[t, h].view(np.uint16))
                else:
                    assert np.array_equal(ent, O.quantize_rows(fmt, row))
        assert (nhd[~written] == 0xAB).all()


# ------------------------------------------------------------ TurboQuant

def test_tq_layouts():
    sizes = {m: O.tq_layout(m).slot_size_aligned for m in
             ("turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc")}
    assert sizes == {"turboquant_4bit_nc": 134, "turboquant_3bit_nc": 102, "turboquant_k3v4_nc": 118}
    L = O.tq_layout("turboquant_3bit_nc")
    assert (L.mse_bytes, L.key_packed_size, L.val_data_bytes, L.value_packed_size) == (48, 50, 48, 52)
    with pytest.raises(ValueError):
        O.tq_layout("turboquant_bogus")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_hadamard_closed_form(d):
    H = np.zeros((d, d), np.float32)
    O.lib().orc_tq_hadamard(O._ptr(H), d)
    i = np.arange(d)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    ref = np.where(pc % 2, -1.0, 1.0) / np.sqrt(d)
    assert np.allclose(H, ref, atol=1e-7)
    assert np.allclose(H.astype(np.float64) @ H.astype(np.float64), np.eye(d), atol=1e-6)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotate_is_hadamard_product(d):
    H = np.zeros((d, d), np.float32)
    O.lib().orc_tq_hadamard(O._ptr(H), d)
    rng = np.random.default_rng(4)
    for _ in range(20):
        x = rng.standard_normal(d).astype(np.float32)
        y = O.tq_rotate(x)
        ref = H.astype(np.float64) @ x.astype(np.float64)
        assert np.abs(y - ref).max() <= 8 * np.finfo(np.float32).eps * np.abs(x).sum() / np.sqrt(d)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_lloyd_max_matches_max_tables(d):
    """Max (1960) optimal Gaussian quantizers, scaled by sigma = 1/sqrt(d);
    the head_dim 128 tables also bit-pinned."""
    tables = {3: [0.2451, 0.7560, 1.3439, 2.1520],
              4: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326]}
    pinned = json.load(open(os.path.join(GOLD, "tq_tables_d128.json")))
    for bits, half in tables.items():
        c, m = O.tq_tables(d, bits)
        ref = np.concatenate([-np.array(half[::-1]), half]) / np.sqrt(d)
        assert np.allclose(c, ref, rtol=1.5e-3, atol=0)
        assert np.all(np.diff(c) > 0)
        assert np.array_equal(m, ((c[:-1] + c[1:]) / 2).astype(np.float32))
        if d == 128:
            assert [f"{v:08x}" for v in c.view(np.uint32)] == pinned[f"centroids_{bits}bit"]
            assert [f"{v:08x}" for v in m.view(np.uint32)] == pinned[f"midpoints_{bits}bit"]


def _unpack(buf, bits, n=D):
    v = np.frombuffer(bytes(buf), np.uint8)
    if bits == 4:
        return np.stack([v & 15, v >> 4], 1).reshape(-1)[:n].astype(np.int64)
    word = np.zeros(n, np.int64)
    for g in range(n // 8):
        w24 = int(v[3 * g]) | int(v[3 * g + 1]) << 8 | int(v[3 * g + 2]) << 16
        word[8 * g:8 * g + 8] = [(w24 >> (3 * i)) & 7 for i in range(8)]
    return word


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc"])
def test_tq_store_properties(method, d):
    D = d
    L = O.tq_layout(method, D)
    c, m = O.tq_tables(D, L.key_quant_bits)
    H = np.zeros((D, D), np.float32)
    O.lib().orc_tq_hadamard(O._ptr(H), D)
    rng = np.random.default_rng(6)
    T, Hkv = 40, 2
    K = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    V = (rng.standard_normal((T, Hkv, D)) * 3 + 1).astype(np.float16)
    K[5, 1] = 0.0                      # zero key: norm 0, every code the same
    V[7, 0] = np.float16(0.375)        # constant value row: codes 0, zero = v
    slots = rng.permutation(4 * BS)[:T].astype(np.int64)
    slots[9] = -1
    S = L.slot_size_aligned
    cache = np.full(4 * BS * Hkv * S, 0xCD, np.uint8)
    O.tq_store(K.view(np.uint16), V.view(np.uint16), slots, cache, BS, L, m)
    vmax = (1 << L.value_quant_bits) - 1
    for t in range(T):
        for h in range(Hkv):
            s = slots[t]
            off = (s // BS) * BS * Hkv * S + (s % BS) * Hkv * S + h * S
            sp = cache[off:off + S]
            if s < 0:
                continue
            kf = K[t, h].astype(np.float64)
            n = np.sqrt((kf ** 2).sum())
            norm = sp[L.mse_bytes:L.mse_bytes + 2].copy().view(np.float16)[0]
            assert abs(float(norm) - n) <= 1e-3 * max(n, 1e-6)
            codes = _unpack(sp[:L.mse_bytes], L.key_quant_bits, D)
            y = H.astype(np.float64) @ (kf / (n + 1e-8))
            nearest = np.abs(y[:, None] - c[None, :].astype(np.float64)).argmin(1)
            near_mid = np.abs(y[:, None] - m[None, :]).min(1) < 1e-5
            assert np.array_equal(codes[~near_mid], nearest[~near_mid])
            if n == 0:
                assert len(set(codes.tolist())) == 1
            vp = sp[L.key_packed_size:]
            vc = _unpack(vp[:L.val_data_bytes], L.value_quant_bits, D)
            vs, vz = vp[L.val_data_bytes:L.val_data_bytes + 4].copy().view(np.float16).astype(np.float64)
            vf = V[t, h].astype(np.float64)
            assert vz == np.float16(vf.min())
            assert vc.min() >= 0 and vc.max() <= vmax
            if vf.max() == vf.min():
                assert (vc == 0).all()
            else:
                assert abs(vs - (vf.max() - vf.min()) / vmax) <= 1e-3 * vs
                assert np.abs(vc * vs + vz - vf).max() <= 0.5 * vs * 1.01 + 2e-3 * np.abs(vf).max()
            # dequantization follows the same unpacking
            kout = np.zeros(D, np.float32)
            vout = np.zeros(D, np.float32)
            O.lib().orc_tq_dequant_slot(O._ptr(np.ascontiguousarray(sp)), O.C.byref(L), O._ptr(c), 0,
                                       O._ptr(kout), O._ptr(vout))
            cc = c[codes].astype(np.float64)
            kref = cc / np.sqrt((cc ** 2).sum() + 1e-16) * float(norm)
            assert np.allclose(kout, kref, rtol=1e-5, atol=1e-6)
            assert np.allclose(vout, vc * vs + vz, rtol=1e-6, atol=1e-6)
    # slot -1 wrote nothing
    untouched = np.ones(cache.size, bool)
    for s in slots[slots >= 0]:
        base = (s // BS) * BS * Hkv * S + (s % BS) * Hkv * S
        untouched[base:base + Hkv * S] = False
    assert (cache[untouched] == 0xCD).all()


def _tq_case(method, lens, Hq=8, Hkv=2, seed=7, d=D):
    w = kvgen.make_workload(lens, Hq=Hq, Hkv=Hkv, seed=seed, D=d)
    L = O.tq_layout(method, d)
    c, m = O.tq_tables(d, L.key_quant_bits)
    cache = np.zeros(w.num_blocks * BS * w.Hkv * L.slot_size_aligned, np.uint8)
    if w.K.shape[0]:
        O.tq_store(w.K.view(np.uint16), w.V.view(np.uint16), w.slots, cache, BS, L, m)
    return w, L, c, cache


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
def test_tq_decode_matches_exact_and_split_invariant(method):
    w, L, c, cache = _tq_case(method, [1, 33, 0, 700, 1500])
    qb = kvgen.bits16(w.Q)
    ex = O.tq_decode_exact(qb, cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    outs = {}
    for ns in (1, 8, 32):
        outs[ns] = O.f16_to_f32(O.tq_decode(qb, cache, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale),
                                            BS, L, c, num_splits=ns))
        ok, err = close_report(outs[ns], ex, ATOL, RTOL)
        assert ok, f"splits {ns}: {err}"
    assert np.abs(outs[1] - outs[32]).max() < 2e-3
    assert (outs[1][2] == 0).all()  # empty sequence -> zero row


@pytest.mark.parametrize("d", [64, 128, 256])
def test_tq_decode_exact_brute_force(d):
    """fp64 attention over dequantized slots, recomputed here from the slot
    bytes with numpy (rotation undone with the exact Hadamard matrix)."""
    D = d
    w, L, c, cache = _tq_case("turboquant_4bit_nc", [20, 45], Hq=4, Hkv=2, seed=8, d=D)
    H = np.zeros((D, D), np.float32)
    O.lib().orc_tq_hadamard(O._ptr(H), D)
    qb = kvgen.bits16(w.Q)
    ex = O.tq_decode_exact(qb, cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    S = L.slot_size_aligned
    G = w.Hq // w.Hkv
    for b in range(w.B):
        n = int(w.seq_lens[b])
        for hq in range(w.Hq):
            h = hq // G
            Ks, Vs = [], []
            for t in range(n):
                blk = w.bt[b, t // BS]
                off = blk * BS * w.Hkv * S + (t % BS) * w.Hkv * S + h * S
                ko = np.zeros(D, np.float32)
                vo = np.zeros(D, np.float32)
                O.lib().orc_tq_dequant_slot(O._ptr(np.ascontiguousarray(cache[off:off + S])),
                                           O.C.byref(L), O._ptr(c), 0, O._ptr(ko), O._ptr(vo))
                Ks.append(ko)
                Vs.append(vo)
            Kr = np.array(Ks, np.float64)  # rotated-domain keys
            qrot = H.astype(np.float64) @ w.Q[b, hq].astype(np.float64)
            s = Kr @ qrot * w.scale
            p = np.exp(s - s.max())
            ref = (p @ np.array(Vs, np.float64)) / p.sum()
            assert np.abs(ex[b, hq] - ref).max() < 1e-5


def test_tq_decode_block_table_permutation_invariance():
    a = kvgen.make_workload([300, 90], Hq=8, Hkv=2, seed=9)
    b = kvgen.make_workload([300, 90], Hq=8, Hkv=2, seed=9, pool_slack=5)
    b.K, b.V, b.Q = a.K, a.V, a.Q
    L = O.tq_layout("turboquant_3bit_nc")
    c, m = O.tq_tables(D, 3)
    outs = []
    for w in (a, b):
        cache = np.zeros(w.num_blocks * BS * w.Hkv * L.slot_size_aligned, np.uint8)
        O.tq_store(w.K.view(np.uint16), w.V.view(np.uint16), w.slots, cache, BS, L, m)
        outs.append(O.tq_decode(kvgen.bits16(w.Q), cache, w.bt, w.seq_lens, w.Hkv,
                                np.float32(w.scale), BS, L, c))
    assert np.array_equal(outs[0], outs[1])


# ------------------------------------------------------------ paged decode

def _pools(w, fmt):
    E = O.entry_bytes(fmt, D)
    n = w.num_blocks * BS * w.Hkv * E
    kc, vc = np.zeros(n, np.uint8), np.zeros(n, np.uint8)
    if fmt == O.KV_BF16:
        kb = kvgen.f32_to_bf16_bits(w.K.astype(np.float32))
        vb = kvgen.f32_to_bf16_bits(w.V.astype(np.float32))
    else:
        kb, vb = w.K.view(np.uint16), w.V.view(np.uint16)
    O.kv_append(kb, vb, w.slots, kc, vc, BS, fmt, src_bf16=fmt == O.KV_BF16)
    return kc, vc


@pytest.mark.parametrize("fmt,name", [(O.KV_F16, "f16"), (O.KV_BF16, "bf16")])
def test_ggml_decode_restatement_vs_golden_single(fmt, name):
    g = gold(f"fa_decode_{name}.npz")
    w = kvgen.single_seq_fp16_workload()
    assert (kvgen.crc(w.K), kvgen.crc(w.V), kvgen.crc(w.Q)) == (g["crc_k"], g["crc_v"], g["crc_q"])
    kc, vc = _pools(w, fmt)
    q = w.Q.astype(np.float32)
    if fmt == O.KV_BF16:
        q = O.bf16_to_f32(kvgen.f32_to_bf16_bits(q))
    for nth in (1, 4):
        o = O.decode_ggml(q, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale), BS, nth=nth)
        # f16: the reference's SIMD dot-product order differs from the
        # restatement's sequential one; bf16 has no fp16 V accumulator
        tol = 1e-4 if fmt == O.KV_F16 else 1e-6
        assert np.abs(o - g[f"out_nth{nth}"]).max() <= tol
    ex = O.paged_decode_exact(q, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
    ok, err = close_report(g["out_nth1"], ex, ATOL, RTOL)
    assert ok, err


@pytest.mark.parametrize("fmt,name", [(O.KV_Q8_0, "q8_0"), (O.KV_Q4_0, "q4_0")])
def test_ggml_decode_restatement_vs_golden_batched(fmt, name):
    g = gold(f"fa_decode_{name}.npz")
    w = kvgen.batched_q8_0_workload()
    assert (kvgen.crc(w.K), kvgen.crc(w.V), kvgen.crc(w.Q)) == (g["crc_k"], g["crc_v"], g["crc_q"])
    n = len(g["seqs"])
    w.seq_lens, w.bt, w.B = w.seq_lens.copy(), w.bt.copy(), w.B
    kc, vc = _pools(w, fmt)
    o = O.decode_ggml(w.Q.astype(np.float32), kc, vc, fmt, w.bt, w.seq_lens, w.Hkv,
                      np.float32(w.scale), BS, nth=1)
    assert np.abs(o[:n] - g["out"]).max() <= 1e-6
    ex = O.paged_decode_exact(w.Q.astype(np.float32), kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
    ok, err = close_report(g["out"], ex[:n], ATOL, RTOL)
    assert ok, err


def test_paged_decode_exact_known_answers():
    """q = 0 gives the mean of V; a one-token context returns that token's V;
    a block-table hole removes exactly that page's tokens."""
    w = kvgen.make_workload([50, 1, 40], Hq=4, Hkv=2, seed=10)
    w.Q[0] = 0
    kc, vc = _pools(w, O.KV_F16)
    ex = O.paged_decode_exact(w.Q.astype(np.float32), kc, vc, O.KV_F16, w.bt, w.seq_lens, w.Hkv,
                              w.scale, BS)
    V0 = w.V[:50].astype(np.float64)
    for hq in range(4):
        assert np.allclose(ex[0, hq], V0[:, hq // 2].mean(0), atol=1e-12)
        assert np.allclose(ex[1, hq], w.V[50, hq // 2].astype(np.float64), atol=1e-12)
    bt = w.bt.copy()
    bt[2, 1] = -1
    ex2 = O.paged_decode_exact(w.Q.astype(np.float32), kc, vc, O.KV_F16, bt, w.seq_lens, w.Hkv,
                               w.scale, BS)
    K2 = np.concatenate([w.K[51:51 + 16], w.K[51 + 32:51 + 40]]).astype(np.float64)
    V2 = np.concatenate([w.V[51:51 + 16], w.V[51 + 32:51 + 40]]).astype(np.float64)
    for hq in range(4):
        s = K2[:, hq // 2] @ w.Q[2, hq].astype(np.float64) * w.scale
        p = np.exp(s - s.max())
        assert np.allclose(ex2[2, hq], p @ V2[:, hq // 2] / p.sum(), atol=1e-12)


# ------------------------------------------------------------ prefill

def test_prefill_exact_rows_brute_force():
    qb, kb, vb, pos, cu = kvgen.prefill_inputs([9, 30], 4, 2, seed=11)
    toks = np.arange(39).repeat(4)
    heads = np.tile(np.arange(4), 39)
    ex = O.prefill_exact_rows(qb, kb, vb, cu, 2, 1 / np.sqrt(D), toks, heads)
    qf, kf, vf = (O.bf16_to_f32(a).astype(np.float64) for a in (qb, kb, vb))
    for r, (t, h) in enumerate(zip(toks, heads)):
        s0 = t - pos[t]
        s = kf[s0:t + 1, h // 2] @ qf[t, h] / np.sqrt(D)
        p = np.exp(s - s.max())
        assert np.allclose(ex[r], p @ vf[s0:t + 1, h // 2] / p.sum(), atol=1e-12)


def test_prefill_exact_rows_vs_golden():
    g = gold("fa_prefill_bf16.npz")
    qb, kb, vb, pos, cu = kvgen.prefill_inputs([4096] * 4, 32, 8, seed=3)
    assert (kvgen.crc(qb), kvgen.crc(kb), kvgen.crc(vb)) == (g["crc_q"], g["crc_k"], g["crc_v"])
    ex = O.prefill_exact_rows(qb, kb, vb, cu, 8, 1 / np.sqrt(D), g["tokens"], g["heads"])
    # the reference accumulates in fp32 over up to 4096 keys
    assert np.abs(ex - g["out"]).max() < 1e-5


@pytest.mark.ref
@pytest.mark.skipif(not O.ref_available(), reason="reference build absent (needs the reference sources)")
def test_ggml_decode_restatement_vs_live_reference_q8_0():
    w = kvgen.make_workload([700, 64, 1], Hq=8, Hkv=2, seed=12)
    kc, vc = _pools(w, O.KV_Q8_0)
    o = O.decode_ggml(w.Q.astype(np.float32), kc, vc, O.KV_Q8_0, w.bt, w.seq_lens, w.Hkv,
                      np.float32(w.scale), BS, nth=1)
    starts = np.concatenate([[0], np.cumsum(w.seq_lens)])
    for b in range(w.B):
        n = int(w.seq_lens[b])
        K = np.ascontiguousarray(w.K[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2))
        V = np.ascontiguousarray(w.V[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2))
        E = O.entry_bytes(O.KV_Q8_0, D)
        kr = O.ref_quantize(O.KV_Q8_0, K.reshape(-1)).reshape(w.Hkv, n, E)
        vr = O.ref_quantize(O.KV_Q8_0, V.reshape(-1)).reshape(w.Hkv, n, E)
        r = O.ref_flash_attn(w.Q[b].astype(np.float32)[:, None, :], kr, vr, O.KV_Q8_0, n, w.Hkv,
                             np.float32(w.scale))[0]
        assert np.abs(o[b] - r).max() <= 1e-6
