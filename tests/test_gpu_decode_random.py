"""Seeded random decode cases against the oracle's fp64 attention over the
same pages: f16 / bf16 / q8_0 / q4_0 pages (NHD, HND) through
vmc_paged_attention_decode, and 3-bit, 4-bit, k3v4, fp8-key and per-32-group
TurboQuant slots through vmc_turboquant_decode_attention.  Each case draws
1-6 sequences of 0-900 tokens (empty sequences included), 0-3 block-table
holes, a head shape from (8, 8), (12, 4), (16, 4), (24, 8), (64, 8), (32, 2)
and (64, 2) (G = 1, 3, 4, 3, 8, 16, 32: the tuned kernels and the
one-wave-per-row kernel past 16 query heads per KV head), and a split mode
(one pass per sequence; pages split evenly with at most 8 x batch pieces;
no cap).
Tolerance |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu

SHAPES = [(8, 8), (12, 4), (16, 4), (24, 8), (64, 8), (32, 2), (64, 2)]
SPLITS = [1, 8, 0]


def _case(seed):
    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 7))
    lens = rng.integers(0, 901, B).astype(np.int32)
    if seed % 3 == 0:
        lens[int(rng.integers(0, B))] = 0
    Hq, Hkv = SHAPES[seed % len(SHAPES)]
    holes = int(rng.integers(0, 4))
    splits = SPLITS[seed % len(SPLITS)]
    return rng, lens, Hq, Hkv, holes, splits


def _as(dev, bits, bf16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(
        torch.bfloat16 if bf16 else torch.float16)


@pytest.mark.parametrize("seed", range(12))
def test_paged_decode_random(dev, seed):
    import torch
    from vm_c_amd import capi
    rng, lens, Hq, Hkv, holes, splits = _case(seed)
    fmt = [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0][seed % 4]
    hnd = bool(rng.integers(0, 2))
    bf16 = fmt == O.KV_BF16
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=6000 + seed, holes=holes, pool_slack=2)
    kb = f32_to_bf16_bits(w.K.astype(np.float32)) if bf16 else w.K.view(np.uint16)
    vb = f32_to_bf16_bits(w.V.astype(np.float32)) if bf16 else w.V.view(np.uint16)
    qb = f32_to_bf16_bits(w.Q.astype(np.float32)) if bf16 else w.Q.view(np.uint16)
    n = w.num_blocks * BS * Hkv * O.entry_bytes(fmt, 128)
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    layout = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    if w.K.shape[0]:
        capi.reshape_and_cache(_as(dev, kb, bf16), _as(dev, vb, bf16), kc, vc, torch.from_numpy(w.slots).to(dev),
                               BS, kv_format=fmt, layout=layout)
    print(f"case {seed}: lens={lens.tolist()} heads={Hq}/{Hkv} fmt={fmt} hnd={hnd} splits={splits} "
          f"holes={holes}", flush=True)
    q = _as(dev, qb, bf16)
    out = torch.full(w.Q.shape, float("nan"), dtype=q.dtype, device=dev)
    capi.paged_attention_decode(out, q, kc, vc, torch.from_numpy(w.bt).to(dev), torch.from_numpy(lens).to(dev),
                                Hkv, float(w.scale), block_size=BS, kv_format=fmt, layout=layout,
                                max_splits=splits)
    torch.cuda.synchronize()
    qf = O.bf16_to_f32(qb) if bf16 else O.f16_to_f32(qb)
    ex = O.paged_decode_exact(qf, kc.cpu().numpy(), vc.cpu().numpy(), fmt, w.bt, lens, Hkv, float(w.scale), BS,
                              hnd=hnd)
    got = out.float().cpu().numpy()
    ok, err = close_report(got, ex, 2e-3, 1e-2)
    assert ok, f"case {seed}: max err {err}"
    assert (got[lens <= 0] == 0).all()


TQ_METHODS = ["turboquant_3bit_nc", "turboquant_4bit_nc", "turboquant_k3v4_nc", "turboquant_k8v4",
              "turboquant_3bit_g32", "turboquant_4bit_g32"]


@pytest.mark.parametrize("seed", range(12))
def test_turboquant_decode_random(dev, seed):
    import torch
    from vm_c_amd import capi
    rng, lens, Hq, Hkv, holes, splits = _case(100 + seed)
    method = TQ_METHODS[seed % len(TQ_METHODS)]
    g32 = method.endswith("_g32")
    if g32 and (Hkv > 8 or Hq // Hkv > 16):
        Hq, Hkv = 32, 8  # the per-32-group kernels keep the tuned head limits
    bf16 = bool(rng.integers(0, 2)) and not g32
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=7000 + seed, holes=holes, pool_slack=2)
    cfg = capi.tq_config(128, method, sign_seed=9 if g32 else 0)
    cache = torch.zeros(w.num_blocks * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    dt = torch.bfloat16 if bf16 else torch.float16
    if w.K.shape[0]:
        capi.turboquant_store(torch.from_numpy(w.K).to(dev).to(dt), torch.from_numpy(w.V).to(dev).to(dt), cache,
                              torch.from_numpy(w.slots).to(dev), BS, cfg)
    qf = w.Q.astype(np.float32)
    qbits = f32_to_bf16_bits(qf) if bf16 else bits16(w.Q)
    q = _as(dev, qbits, bf16)
    print(f"case {seed}: lens={lens.tolist()} heads={Hq}/{Hkv} {method} bf16={bf16} splits={splits} "
          f"holes={holes}", flush=True)
    out = torch.full(w.Q.shape, float("nan"), dtype=dt, device=dev)
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(w.bt).to(dev), torch.from_numpy(lens).to(dev),
                                     Hkv, float(w.scale), cfg, block_size=BS, max_splits=splits)
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    if g32:
        ex = O.g32_decode_exact(qbits, got_cache, w.bt, lens, Hkv, float(w.scale), BS,
                                4 if "4bit" in method else 3, 9)
    else:
        L = O.tq_layout(method)
        c, _ = O.tq_tables(128, 4 if L.key_fp8 else L.key_quant_bits)
        ex = O.tq_decode_exact(qbits, got_cache, w.bt, lens, Hkv, float(w.scale), BS, L, c, bf16=bf16)
    got = out.float().cpu().numpy()
    ok, err = close_report(got, ex, 2e-3, 1e-2)
    assert ok, f"case {seed}: max err {err}"
    assert (got[lens <= 0] == 0).all()
