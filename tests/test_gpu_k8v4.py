"""GPU parity of turboquant_k8v4 (fp8 keys + 4-bit values; reference
src/cuda/turboquant_kernels.cu:47-143, :188-245, :407-415):

* store: every byte of the pool bit-exact against the oracle's store (the
  reference's fp8 encoder), fp16 and bf16 inputs, e4m3 and e4b15 codes,
  skipped slots and untouched bytes;
* decode: against the oracle's float64 attention over the same pages (keys
  decoded from fp8, q not rotated, no norm), ragged lengths, GQA 2..16, both
  split modes.  This pins the intended fp8-key semantics, not the
  reference's output: its stage 1 also multiplies each fp8 key by the fp16
  it reads at +mse_bytes (turboquant_kernels.cu:443-450), which in the k8v4
  slot is the first two V code bytes, not a norm;
* the fused norm + RoPE + append writing k8v4 slots.
Tolerance: |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
D = 128


def _cfg(e4b15):
    from vm_c_amd import capi
    cfg = capi.tq_config(D, "turboquant_k8v4")
    cfg.fp8_e4b15 = int(e4b15)
    L = O.tq_layout("turboquant_k8v4")
    L.fp8_e4b15 = int(e4b15)
    return cfg, L


def _store(dev, w, e4b15, bf16=False, poison=0, kscale=1.0):
    import torch
    from vm_c_amd import capi
    cfg, L = _cfg(e4b15)
    cache = torch.full((w.num_blocks * BS * w.Hkv * 196,), poison, dtype=torch.uint8, device=dev)
    K = (w.K.astype(np.float32) * kscale)
    if bf16:
        kb, vb = f32_to_bf16_bits(K), f32_to_bf16_bits(w.V.astype(np.float32))
        tdt = torch.bfloat16
    else:
        kb, vb = bits16(K.astype(np.float16)), bits16(w.V)
        tdt = torch.float16
    kt = torch.from_numpy(kb.view(np.int16)).to(dev).view(tdt)
    vt = torch.from_numpy(vb.view(np.int16)).to(dev).view(tdt)
    if K.shape[0]:
        capi.turboquant_store(kt, vt, cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    torch.cuda.synchronize()
    ref = np.full(cache.numel(), poison, np.uint8)
    _, mid = O.tq_tables(D, 4)
    if K.shape[0]:
        O.tq_store(kb, vb, w.slots, ref, BS, L, mid, bf16=bf16)
    return cfg, L, cache, ref


@pytest.mark.parametrize("e4b15", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_k8v4_store_bitexact(dev, e4b15, bf16):
    w = make_workload([37, 300, 1, 64], Hq=16, Hkv=4, seed=5, pool_slack=3)
    w.slots[5] = -1
    _, _, cache, ref = _store(dev, w, e4b15, bf16=bf16, poison=0xA5, kscale=0.3 if e4b15 else 3.0)
    got = cache.cpu().numpy()
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


def _decode(dev, w, cfg, cache, max_splits=0):
    import torch
    from vm_c_amd import capi
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale),
                                     cfg, block_size=BS, max_splits=max_splits)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = {
    "ragged": dict(seq_lens=[1, 17, 0, 300], Hq=16, Hkv=4),
    "gqa16": dict(seq_lens=[300, 1024, 17, 33], Hq=32, Hkv=2),
    "gqa2": dict(seq_lens=[5, 129, 700], Hq=8, Hkv=4),
    "cfg_small": dict(seq_lens=[1024, 4000, 32], Hq=64, Hkv=8),
}


@pytest.mark.parametrize("e4b15", [False, True])
@pytest.mark.parametrize("case", list(CASES))
def test_k8v4_decode(dev, e4b15, case):
    w = make_workload(seed=len(case) + 11, **CASES[case])
    cfg, L, cache, _ = _store(dev, w, e4b15, kscale=0.3 if e4b15 else 1.0)
    c, _ = O.tq_tables(D, 4)
    ex = O.tq_decode_exact(bits16(w.Q), cache.cpu().numpy(), w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    for ms in (0, 1):
        ok, err = close_report(_decode(dev, w, cfg, cache, max_splits=ms), ex, ATOL, RTOL)
        assert ok, f"max_splits={ms}: max err {err}"


@pytest.mark.parametrize("e4b15", [False, True])
@pytest.mark.parametrize("case", ["ragged", "gqa16"])
def test_k8v4_decode_bf16(dev, e4b15, case):
    """bf16 q, out and V scale / zero (the reference's USE_BF16 stage 1 for
    fp8 keys, turboquant_kernels.cu:876-881): the decode and a 20-token
    prefill step against fp64 attention over the same slots."""
    import torch
    from vm_c_amd import capi
    w = make_workload(seed=len(case) + 13, **CASES[case])
    cfg, L, cache, _ = _store(dev, w, e4b15, bf16=True, kscale=0.3 if e4b15 else 1.0)
    qb = f32_to_bf16_bits(w.Q.astype(np.float32))
    as_bf16 = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(dev).view(torch.bfloat16)
    out = torch.full(w.Q.shape, float("nan"), dtype=torch.bfloat16, device=dev)
    bt = torch.from_numpy(w.bt).to(dev)
    capi.turboquant_decode_attention(out, as_bf16(qb), cache, bt, torch.from_numpy(w.seq_lens).to(dev), w.Hkv,
                                     float(w.scale), cfg, block_size=BS)
    rng = np.random.default_rng(len(case))
    live = np.flatnonzero(w.seq_lens > 0)
    tok_seq = live[rng.integers(0, live.size, 20)].astype(np.int32)
    tok_pos = (rng.random(20) * w.seq_lens[tok_seq]).astype(np.int32)
    qp = f32_to_bf16_bits(rng.standard_normal((20, w.Hq, D)).astype(np.float32))
    outp = torch.full((20, w.Hq, D), float("nan"), dtype=torch.bfloat16, device=dev)
    capi.turboquant_prefill_attention(outp, as_bf16(qp), cache, bt, torch.from_numpy(tok_seq).to(dev),
                                      torch.from_numpy(tok_pos).to(dev), w.Hkv, float(w.scale), cfg, block_size=BS)
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    c, _ = O.tq_tables(D, 4)
    ex = O.tq_decode_exact(qb, got_cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c, bf16=True)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"decode: max err {err}"
    ex = O.tq_decode_exact(qp, got_cache, w.bt[tok_seq], tok_pos + 1, w.Hkv, w.scale, BS, L, c, bf16=True)
    ok, err = close_report(outp.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"prefill rows: max err {err}"
