"""head_dim 128 at head counts past the tuned decode kernels' (more than 8
KV heads, or more than 16 query heads per KV head): multi-head attention
with 16/16 heads and a 64/2 grouping.  The reference's decode takes any
head counts (paged_attention_v1/_v2, attention_kernels.cu; the TurboQuant
stage 1 grid, turboquant_kernels.cu:939-1007).

  * f16 / q8_0 pages, NHD and HND: the paged decode, the per-token prefill
    and vmc_flash_attention_prefill_v2 against fp64 exact attention.
  * TurboQuant 3-bit, 4-bit and fp8-key slots: the decode and both prefill
    paths (15 tokens: one decode row per token; 40 tokens: the tiled
    prefill over codebook slots) against fp64 exact attention.
Tolerance |got - ref| <= 2e-3 + 1e-2 |ref|; batches hold an empty sequence,
a one-token one and a block-table hole.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, make_workload

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
SHAPES = {"mha16": (16, 16), "g32": (64, 2)}


def _rows(lens, rng, T):
    live = np.flatnonzero(lens > 0)
    tok_seq = live[rng.integers(0, live.size, T)].astype(np.int32)
    tok_pos = (rng.random(T) * lens[tok_seq]).astype(np.int32)
    return tok_seq, tok_pos


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_Q8_0])
@pytest.mark.parametrize("hnd", [False, True])
def test_paged_decode_and_prefill_wide(dev, shape, fmt, hnd):
    import torch
    from vm_c_amd import capi
    Hq, Hkv = SHAPES[shape]
    lens = np.array([1, 200, 0, 77], np.int32)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=120 + fmt + 2 * hnd, holes=1, pool_slack=2)
    E = O.entry_bytes(fmt, 128)
    n = w.num_blocks * BS * Hkv * E
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    layout = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    capi.reshape_and_cache(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), kc, vc,
                           torch.from_numpy(w.slots).to(dev), BS, kv_format=fmt, layout=layout)
    bt = torch.from_numpy(w.bt).to(dev)
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.full_like(q, float("nan"))
    capi.paged_attention_decode(out, q, kc, vc, bt, torch.from_numpy(lens).to(dev), Hkv, float(w.scale),
                                block_size=BS, kv_format=fmt, layout=layout)
    tok_seq, tok_pos = _rows(lens, np.random.default_rng(fmt), 40)
    qp = np.random.default_rng(fmt + 1).standard_normal((40, Hq, 128)).astype(np.float16)
    args = (kc, vc, bt, torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev), Hkv, float(w.scale))
    rows = torch.full((40, Hq, 128), float("nan"), dtype=torch.float16, device=dev)
    capi.paged_attention_prefill(rows, torch.from_numpy(qp).to(dev), *args, block_size=BS, kv_format=fmt,
                                 layout=layout, max_splits=1)
    v2 = torch.full_like(rows, float("nan"))
    capi.flash_attention_prefill_v2(v2, torch.from_numpy(qp).to(dev), *args, block_size=BS, kv_format=fmt,
                                    layout=layout)
    torch.cuda.synchronize()
    kr, vr = kc.cpu().numpy(), vc.cpu().numpy()
    ex = O.paged_decode_exact(w.Q.astype(np.float32), kr, vr, fmt, w.bt, lens, Hkv, float(w.scale), BS, hnd=hnd)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"decode: {err}"
    assert (out[2] == 0).all()  # the empty sequence
    exp = O.paged_decode_exact(qp.astype(np.float32), kr, vr, fmt, w.bt[tok_seq], tok_pos + 1, Hkv,
                               float(w.scale), BS, hnd=hnd)
    for name, t in (("per-token prefill", rows), ("prefill_v2", v2)):
        ok, err = close_report(t.float().cpu().numpy(), exp, ATOL, RTOL)
        assert ok, f"{name}: {err}"


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("method", ["turboquant_3bit_nc", "turboquant_4bit_nc", "turboquant_k8v4"])
def test_turboquant_wide(dev, shape, method):
    import torch
    from vm_c_amd import capi
    Hq, Hkv = SHAPES[shape]
    lens = np.array([1, 300, 0, 90], np.int32)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=140 + len(method), holes=1, pool_slack=2)
    cfg = capi.tq_config(128, method)
    L = O.tq_layout(method)
    c, _ = O.tq_tables(128, 4 if L.key_fp8 else L.key_quant_bits)
    cache = torch.zeros(w.num_blocks * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    capi.turboquant_store(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), cache,
                          torch.from_numpy(w.slots).to(dev), BS, cfg)
    bt = torch.from_numpy(w.bt).to(dev)
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, bt, torch.from_numpy(lens).to(dev), Hkv, float(w.scale), cfg,
                                     block_size=BS)
    rng = np.random.default_rng(len(method))
    steps = []
    for T in (15, 40):
        tok_seq, tok_pos = _rows(lens, rng, T)
        qp = rng.standard_normal((T, Hq, 128)).astype(np.float16)
        o = torch.full((T, Hq, 128), float("nan"), dtype=torch.float16, device=dev)
        capi.turboquant_prefill_attention(o, torch.from_numpy(qp).to(dev), cache, bt,
                                          torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev),
                                          Hkv, float(w.scale), cfg, block_size=BS)
        steps.append((qp, tok_seq, tok_pos, o))
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    ex = O.tq_decode_exact(bits16(w.Q), got_cache, w.bt, lens, Hkv, w.scale, BS, L, c)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"decode: {err}"
    for qp, tok_seq, tok_pos, o in steps:
        ex = O.tq_decode_exact(bits16(qp), got_cache, w.bt[tok_seq], tok_pos + 1, Hkv, w.scale, BS, L, c)
        ok, err = close_report(o.float().cpu().numpy(), ex, ATOL, RTOL)
        assert ok, f"prefill of {len(tok_seq)} tokens: {err}"
