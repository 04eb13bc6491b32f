"""Quantize-on-append parity: the HIP kernels must write the same bytes as the
oracle (bit-exact), which is itself pinned to ggml's quantize_row_*_ref and
to the TurboQuant store restatement."""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("src_bf16", [False, True])
def test_reshape_and_cache_bitexact(dev, fmt, hnd, src_bf16):
    torch = _torch()
    from vm_c_amd import capi
    w = make_workload([37, 200, 1, 16], Hq=8, Hkv=4, seed=11)
    # a skipped token (slot -1) and extreme magnitudes
    slots = w.slots.copy()
    slots[5] = -1
    K = w.K.astype(np.float32)
    K[3, 1, :32] *= 1e3
    K[4, 2, :] = 0.0
    K[6, 0, 7] = -65000.0
    if src_bf16:
        kb = f32_to_bf16_bits(K)
        vb = f32_to_bf16_bits(w.V.astype(np.float32))
        tdt = torch.bfloat16
    else:
        kb = bits16(K.astype(np.float16))
        vb = bits16(w.V)
        tdt = torch.float16
    E = O.entry_bytes(fmt, w.D)
    nbytes = w.num_blocks * BS * w.Hkv * E
    kc_ref = np.zeros(nbytes, np.uint8)
    vc_ref = np.zeros(nbytes, np.uint8)
    O.kv_append(kb.reshape(K.shape), vb.reshape(K.shape), slots, kc_ref, vc_ref, BS, fmt, hnd=hnd,
                src_bf16=src_bf16)
    kt = torch.from_numpy(kb.reshape(K.shape).view(np.int16)).to(dev).view(tdt)
    vt = torch.from_numpy(vb.reshape(K.shape).view(np.int16)).to(dev).view(tdt)
    kc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    vc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    st = torch.from_numpy(slots).to(dev)
    capi.reshape_and_cache(kt, vt, kc, vc, st, BS, kv_format=fmt,
                           layout=capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD)
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().numpy(), kc_ref)
    assert np.array_equal(vc.cpu().numpy(), vc_ref)


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc"])
def test_turboquant_store_bitexact(dev, method):
    torch = _torch()
    from vm_c_amd import capi
    w = make_workload([100, 33, 16, 1], Hq=8, Hkv=8, seed=5)
    slots = w.slots.copy()
    slots[2] = -1
    K = w.K.copy()
    K[7, 3, :] = 0  # zero vector: norm 0
    V = w.V.copy()
    V[9, 1, :] = np.float16(0.5)  # all-equal V: codes 0, scale 1e-8
    L = O.tq_layout(method)
    c, m = O.tq_tables(128, L.key_quant_bits)
    nbytes = w.num_blocks * BS * w.Hkv * L.slot_size_aligned
    ref = np.zeros(nbytes, np.uint8)
    O.tq_store(bits16(K), bits16(V), slots, ref, BS, L, m)
    cfg = capi.tq_config(128, method)
    cache = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    capi.turboquant_store(torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), cache,
                          torch.from_numpy(slots).to(dev), BS, cfg)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    if not np.array_equal(got, ref):
        diff = np.nonzero(got != ref)[0]
        raise AssertionError(f"{diff.size} bytes differ, first at {diff[:8]}")
