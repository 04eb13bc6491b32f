"""GPU parity of the fused Q/K RMSNorm + RoPE + quantize-on-append
(vmc_fused_qk_norm_rope_store; src/cuda/fused_attn_kernels.cu:39-313).

The oracle runs orc_qk_norm_rope on copies of q/k, then appends the updated k
and the original v with the format's own oracle store (orc_kv_append,
orc_tq_store, orc_g32_store).  Everything is integer / bit work after the
fp32 arithmetic of a declared order, so every output is compared bit-exact:
q and k in place, every byte of the page pools (skipped slots and bytes
outside the slots untouched), for fp16/bf16 inputs, neox and GPT-J pairs,
with and without each norm weight, GQA, partial workgroups and zero rows.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu

D = 128
EPS = 1e-6


def _bits(x, bf16):
    x = np.asarray(x, np.float32)
    return f32_to_bf16_bits(x) if bf16 else x.astype(np.float16).view(np.uint16)


def _tensor(dev, bits, bf16):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev)
    return t.view(torch.bfloat16 if bf16 else torch.float16)


def _inputs(T, Hq, Hkv, bf16, seed, max_pos=300):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((T, Hq, D)) * rng.uniform(0.2, 4.0, (T, Hq, 1))).astype(np.float32)
    k = (rng.standard_normal((T, Hkv, D)) * rng.uniform(0.2, 4.0, (T, Hkv, 1))).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    if T > 3:
        k[1, 0] = 0.0                  # zero row: inv = 1/sqrt(eps), q4_0 d = -0
        q[2, Hq - 1, :64] = 0.0
        v[3, Hkv - 1] = 0.25           # constant V row
    qw = (1.0 + 0.1 * rng.standard_normal(Hq * D)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(Hkv * D)).astype(np.float32)
    theta = 10000.0 ** (-np.arange(D // 2) * 2.0 / D)
    ang = np.arange(max_pos)[:, None] * theta[None, :]
    cs = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    pos = rng.integers(0, max_pos, T).astype(np.int64)
    return (_bits(q, bf16), _bits(k, bf16), _bits(v, bf16), _bits(qw, bf16), _bits(kw, bf16),
            _bits(cs, bf16), pos)


def _run(dev, T, Hq, Hkv, bf16, neox, norms, seed, store=None, poison=0):
    """store: None | ("page", fmt, hnd) | ("tq", method) | ("g32", method, sign_seed)"""
    import torch
    from vm_c_amd import capi
    qb, kb, vb, qwb, kwb, csb, pos = _inputs(T, Hq, Hkv, bf16, seed)
    qw = qwb if norms in ("both", "q") else None
    kw = kwb if norms in ("both", "k") else None
    rq, rk = O.qk_norm_rope(qb, kb, qw, kw, csb, pos, EPS, neox, bf16)

    q, k, v = _tensor(dev, qb, bf16), _tensor(dev, kb, bf16), _tensor(dev, vb, bf16)
    qwt = None if qw is None else _tensor(dev, qw, bf16)
    kwt = None if kw is None else _tensor(dev, kw, bf16)
    cst, post = _tensor(dev, csb, bf16), torch.from_numpy(pos).to(dev)
    res = {}
    if store is None:
        capi.fused_qk_norm_rope_store(q, k, v, qwt, kwt, cst, post, eps=EPS, is_neox=neox)
    else:
        lens = [T // 3, T - T // 3 - 1, 1]
        w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=seed, pool_slack=2)
        slots = w.slots.copy()
        if T > 6:
            slots[5] = -1          # skipped token: its slot stays untouched
        st = torch.from_numpy(slots).to(dev)
        if store[0] == "page":
            fmt, hnd = store[1], store[2]
            n = w.num_blocks * BS * Hkv * O.entry_bytes(fmt, D)
            kc = torch.full((n,), poison, dtype=torch.uint8, device=dev)
            vc = torch.full((n,), poison, dtype=torch.uint8, device=dev)
            capi.fused_qk_norm_rope_store(q, k, v, qwt, kwt, cst, post, kc, vc, st, BS, eps=EPS,
                                          is_neox=neox, kv_format=fmt,
                                          layout=capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD)
            kr = np.full(n, poison, np.uint8)
            vr = np.full(n, poison, np.uint8)
            O.kv_append(rk, vb, slots, kr, vr, BS, fmt, hnd=hnd, src_bf16=bf16)
            res["key_cache"] = (kc, kr)
            res["value_cache"] = (vc, vr)
        else:
            seed_s = store[2] if store[0] == "g32" else 0
            cfg = capi.tq_config(D, store[1], sign_seed=seed_s)
            n = w.num_blocks * BS * Hkv * cfg.slot_size_aligned
            cache = torch.full((n,), poison, dtype=torch.uint8, device=dev)
            capi.fused_qk_norm_rope_store(q, k, v, qwt, kwt, cst, post, cache, None, st, BS,
                                          eps=EPS, is_neox=neox, tq_cfg=cfg)
            ref = np.full(n, poison, np.uint8)
            if store[0] == "tq":
                L = O.tq_layout(store[1])
                _, mid = O.tq_tables(D, 4 if L.key_fp8 else L.key_quant_bits)
                O.tq_store(rk, vb, slots, ref, BS, L, mid, bf16=bf16)
            else:
                O.g32_store(rk, vb, slots, ref, BS, cfg.key_quant_bits, seed_s, bf16=bf16)
            res["slots"] = (cache, ref)
    torch.cuda.synchronize()
    res["q"] = (q, rq)
    res["k"] = (k, rk)
    for name, (got, want) in res.items():
        g = got.cpu().view(torch.int16).numpy().view(np.uint16) if got.dtype != torch.uint8 \
            else got.cpu().numpy()
        g = g.reshape(want.shape)
        bad = np.nonzero(g != want)
        assert bad[0].size == 0, f"{name}: {bad[0].size} differ, first at {[b[:4] for b in bad]}"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("norms", ["both", "none", "q", "k"])
def test_norm_rope_only(dev, bf16, neox, norms):
    _run(dev, 37, 16, 4, bf16, neox, norms, seed=1)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("hnd", [False, True])
def test_paged_append(dev, bf16, fmt, hnd):
    _run(dev, 45, 16, 4, bf16, True, "both", seed=2 + fmt, store=("page", fmt, hnd), poison=0xA5)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc",
                                    "turboquant_k8v4"])
def test_turboquant_append(dev, bf16, method):
    _run(dev, 40, 8, 8, bf16, True, "both", seed=7, store=("tq", method), poison=0x5A)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("method", ["turboquant_4bit_g32", "turboquant_3bit_g32"])
def test_g32_append(dev, bf16, method):
    _run(dev, 40, 32, 8, bf16, False, "k", seed=9, store=("g32", method, 4), poison=0x3C)


def test_gqa_shapes_and_single_token(dev):
    # decode-shaped calls: one token per sequence, wide GQA; head counts that
    # give one, two or four rows per 16-lane group
    _run(dev, 1, 64, 8, False, True, "both", seed=11, store=("page", O.KV_Q8_0, False))
    _run(dev, 32, 32, 8, True, True, "both", seed=12, store=("page", O.KV_Q4_0, True))
    _run(dev, 3, 8, 1, False, False, "none", seed=13)         # one row per group
    _run(dev, 19, 6, 2, True, False, "both", seed=14, store=("tq", "turboquant_4bit_nc"))  # two rows
    _run(dev, 9, 12, 2, False, True, "k", seed=15, store=("page", O.KV_F16, True))


def test_zero_tokens_and_bad_args(dev):
    import torch
    from vm_c_amd import capi
    q = torch.zeros((0, 8, D), dtype=torch.float16, device=dev)
    k = torch.zeros((0, 2, D), dtype=torch.float16, device=dev)
    cs = torch.zeros((4, D), dtype=torch.float16, device=dev)
    pos = torch.zeros(0, dtype=torch.int64, device=dev)
    capi.fused_qk_norm_rope_store(q, k, k, None, None, cs, pos)
    q1 = torch.zeros((1, 8, 64), dtype=torch.float16, device=dev)
    k1 = torch.zeros((1, 2, 64), dtype=torch.float16, device=dev)
    with pytest.raises(capi.VmcError):
        capi.fused_qk_norm_rope_store(q1, k1, k1, None, None, cs, pos[:0])
