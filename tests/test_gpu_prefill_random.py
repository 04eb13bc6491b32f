"""Seeded random cases of the tiled prefill over the paged cache against the
per-token path (one decode row per token), which the other tests pin to the
oracle's fp64 attention:

  * vmc_flash_attention_prefill_v2 over f16 / bf16 / q8_0 / q4_0 pages, NHD
    and HND, fp16 or bf16 q;
  * vmc_turboquant_prefill_attention over 3-bit, 4-bit, k3v4 and fp8-key
    slots (a step of >= 16 tokens takes the tiled prefill; the comparison
    runs the same rows in steps of 15 tokens, one decode row per token).

Each case draws 1-5 sequences with prefixes of 0-700 tokens and chunks of
1-140 tokens, head shapes from (8, 8), (16, 4), (24, 8), (32, 8) and
(12, 4) (G = 1, 4, 3, 4, 3), and 0-3 block-table holes in the prefixes.
Tolerance |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, close_report, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu

SHAPES = [(8, 8), (16, 4), (24, 8), (32, 8), (12, 4)]
PAGE_FMTS = [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0]
TQ_METHODS = ["turboquant_3bit_nc", "turboquant_4bit_nc", "turboquant_k3v4_nc", "turboquant_k8v4"]


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 6))
    prefix = rng.integers(0, 701, B)
    new = rng.integers(1, 141, B)
    Hq, Hkv = SHAPES[int(rng.integers(0, len(SHAPES)))]
    holes = int(rng.integers(0, 4))
    return rng, prefix, new, Hq, Hkv, holes


def _rows(prefix, new):
    lens = prefix + new
    tok_seq = np.concatenate([np.full(new[b], b) for b in range(len(lens))]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(prefix[b], lens[b]) for b in range(len(lens))]).astype(np.int32)
    return lens, tok_seq, tok_pos


def _as(dev, bits, bf16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(
        torch.bfloat16 if bf16 else torch.float16)


@pytest.mark.parametrize("seed", range(8))
def test_prefill_v2_random(dev, seed):
    import torch
    from vm_c_amd import capi
    rng, prefix, new, Hq, Hkv, holes = _case(seed)
    fmt = PAGE_FMTS[seed % len(PAGE_FMTS)]
    hnd = bool(rng.integers(0, 2))
    q_bf16 = bool(rng.integers(0, 2))
    lens, tok_seq, tok_pos = _rows(prefix, new)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=2000 + seed, holes=holes, pool_slack=3)
    page_bf16 = fmt == O.KV_BF16
    kbits = f32_to_bf16_bits(w.K.astype(np.float32)) if page_bf16 else w.K.view(np.uint16)
    vbits = f32_to_bf16_bits(w.V.astype(np.float32)) if page_bf16 else w.V.view(np.uint16)
    n = w.num_blocks * BS * Hkv * O.entry_bytes(fmt, 128)
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    layout = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    capi.reshape_and_cache(_as(dev, kbits, page_bf16), _as(dev, vbits, page_bf16), kc, vc,
                           torch.from_numpy(w.slots).to(dev), BS, kv_format=fmt, layout=layout)
    T = tok_seq.size
    qf = rng.standard_normal((T, Hq, 128)).astype(np.float32)
    qbits = f32_to_bf16_bits(qf) if q_bf16 else qf.astype(np.float16).view(np.uint16)
    q = _as(dev, qbits, q_bf16)
    print(f"case {seed}: B={len(lens)} prefix={prefix.tolist()} new={new.tolist()} heads={Hq}/{Hkv} "
          f"fmt={fmt} hnd={hnd} q_bf16={q_bf16} holes={holes}", flush=True)
    args = (kc, vc, torch.from_numpy(w.bt).to(dev), torch.from_numpy(tok_seq).to(dev),
            torch.from_numpy(tok_pos).to(dev), Hkv, float(w.scale))
    out = torch.full((T, Hq, 128), float("nan"), dtype=q.dtype, device=dev)
    capi.flash_attention_prefill_v2(out, q, *args, block_size=BS, kv_format=fmt, layout=layout)
    rows = torch.full_like(out, float("nan"))
    capi.paged_attention_prefill(rows, q, *args, block_size=BS, kv_format=fmt, layout=layout, max_splits=1)
    torch.cuda.synchronize()
    ok, err = close_report(out.float().cpu().numpy(), rows.float().cpu().numpy(), 2e-3, 1e-2)
    assert ok, f"case {seed}: max err {err}"


@pytest.mark.parametrize("seed", range(8))
def test_turboquant_prefill_random(dev, seed):
    import torch
    from vm_c_amd import capi
    rng, prefix, new, Hq, Hkv, holes = _case(100 + seed)
    method = TQ_METHODS[seed % len(TQ_METHODS)]
    bf16 = bool(rng.integers(0, 2))
    lens, tok_seq, tok_pos = _rows(prefix, new)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=3000 + seed, holes=holes, pool_slack=3)
    cfg = capi.tq_config(128, method)
    cache = torch.zeros(w.num_blocks * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    dt = torch.bfloat16 if bf16 else torch.float16
    capi.turboquant_store(torch.from_numpy(w.K).to(dev).to(dt), torch.from_numpy(w.V).to(dev).to(dt), cache,
                          torch.from_numpy(w.slots).to(dev), BS, cfg)
    T = tok_seq.size
    q = torch.from_numpy(rng.standard_normal((T, Hq, 128)).astype(np.float32)).to(dev).to(dt)
    print(f"case {seed}: B={len(lens)} prefix={prefix.tolist()} new={new.tolist()} heads={Hq}/{Hkv} "
          f"{method} bf16={bf16} holes={holes}", flush=True)
    bt = torch.from_numpy(w.bt).to(dev)
    ts, tp = torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev)
    out = torch.full((T, Hq, 128), float("nan"), dtype=dt, device=dev)
    capi.turboquant_prefill_attention(out, q, cache, bt, ts, tp, Hkv, float(w.scale), cfg, block_size=BS)
    rows = torch.full_like(out, float("nan"))
    for a in range(0, T, 15):
        b = min(a + 15, T)
        capi.turboquant_prefill_attention(rows[a:b], q[a:b], cache, bt, ts[a:b], tp[a:b], Hkv, float(w.scale),
                                          cfg, block_size=BS)
    torch.cuda.synchronize()
    ok, err = close_report(out.float().cpu().numpy(), rows.float().cpu().numpy(), 2e-3, 1e-2)
    assert ok, f"case {seed}: max err {err}"
