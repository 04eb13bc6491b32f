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
