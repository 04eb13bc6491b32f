"""GPU test of vmc_turboquant_decode_attention_noalloc (the decode whose split
partials live in the library's own device array): through the C ABI, its
output equals vmc_turboquant_decode_attention's with a caller workspace, bit
for bit (same kernels, same split), on two calls in a row -- the second with a
smaller batch and shorter contexts, so stale rows of the first call are in the
array -- for fp16 and bf16 activations and for the head_dim-256 decode; and
a shape whose partials exceed the array is rejected with VMC_ENOMEM before
any launch."""
import numpy as np
import pytest

from kvgen import BS, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu


def _pages(dev, w, cfg, bf16):
    import torch
    from vm_c_amd import capi
    cache = torch.zeros(w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    if bf16:
        cv = lambda a: torch.from_numpy(f32_to_bf16_bits(a.astype(np.float32)).view(np.int16)).to(dev).view(
            torch.bfloat16)
    else:
        cv = lambda a: torch.from_numpy(a).to(dev)
    capi.turboquant_store(cv(w.K), cv(w.V), cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    return cache, cv(w.Q)


@pytest.mark.parametrize("bf16", [False, True])
def test_noalloc_decode_matches_workspace_decode(dev, bf16):
    import torch
    from vm_c_amd import capi
    cfg = capi.tq_config(128, "turboquant_3bit_nc")
    big = make_workload([5000, 1024, 77, 32768, 3000, 17], Hq=64, Hkv=8, seed=21)
    small = make_workload([900, 40], Hq=32, Hkv=8, seed=22)
    for w in (big, small):
        cache, q = _pages(dev, w, cfg, bf16)
        bt = torch.from_numpy(w.bt).to(dev)
        sl = torch.from_numpy(w.seq_lens).to(dev)
        ref = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention(ref, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
        got = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention_noalloc(got, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), \
            f"noalloc decode differs from the workspace decode (B={w.B})"


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
def test_noalloc_d256_decode_matches_workspace_decode(dev, method):
    """head_dim 256 with 1, 2 or 4 KV heads runs the MFMA decode whose split
    partials are rows of 256 + 4 floats; the array holds them as well: bit for
    bit against the workspace entry point on two calls in a row, the second
    with a smaller batch, fewer heads and shorter contexts."""
    import torch
    from vm_c_amd import capi
    cfg = capi.tq_config(256, method)
    big = make_workload([9000, 300, 4100, 16], Hq=16, Hkv=2, D=256, seed=24)
    small = make_workload([700, 20], Hq=8, Hkv=1, D=256, seed=25)
    for w in (big, small):
        cache, q = _pages(dev, w, cfg, False)
        bt = torch.from_numpy(w.bt).to(dev)
        sl = torch.from_numpy(w.seq_lens).to(dev)
        ref = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention(ref, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
        got = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention_noalloc(got, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), \
            f"noalloc head_dim-256 decode differs from the workspace decode (B={w.B})"


@pytest.mark.parametrize("D,Hq,Hkv", [(256, 16, 8), (128, 64, 2)])
def test_noalloc_one_wave_per_row_shapes(dev, D, Hq, Hkv):
    """head_dim 256 with 8 KV heads and 32 query heads per KV head run the
    one-wave-per-row kernel, which needs no split partials: the
    allocation-free entry point takes them at any size and matches the
    workspace entry point."""
    import torch
    from vm_c_amd import capi
    cfg = capi.tq_config(D, "turboquant_4bit_nc")
    w = make_workload([700, 33, 1500], Hq=Hq, Hkv=Hkv, D=D, seed=23)
    cache, q = _pages(dev, w, cfg, False)
    bt = torch.from_numpy(w.bt).to(dev)
    sl = torch.from_numpy(w.seq_lens).to(dev)
    ref = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(ref, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
    got = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention_noalloc(got, q, cache, bt, sl, w.Hkv, float(w.scale), cfg, BS)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_rejects_oversized_partials(dev):
    """A tuned-kernel shape whose split partials exceed the array is rejected
    with VMC_ENOMEM.  Every argument is a real allocation of the call's full
    size, with empty sequences and an all-hole block table, so the call could
    not touch memory outside them even if it launched."""
    import ctypes as C
    import torch
    from vm_c_amd import capi
    L = capi.load()
    cfg = capi.tq_config(128, "turboquant_3bit_nc")
    cap = L.vmc_noalloc_scratch_bytes()
    B, Hq, Hkv, mb = 64, 128, 8, 4096  # 16 query heads per KV head: the tuned decode
    need = capi.turboquant_decode_workspace_size(B, Hq, Hkv, 128, mb, BS)
    assert need > cap
    q = torch.zeros(B, Hq, 128, dtype=torch.float16, device=dev)
    out = torch.zeros_like(q)
    bt = torch.full((B, mb), -1, dtype=torch.int32, device=dev)
    sl = torch.zeros(B, dtype=torch.int32, device=dev)
    cache = torch.zeros(BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    p = lambda t: C.c_void_p(t.data_ptr())
    rc = L.vmc_turboquant_decode_attention_noalloc(p(out), p(q), p(cache), p(bt), p(sl), B, Hq, Hkv, 128,
                                                   C.c_float(0.1), BS, mb, C.byref(cfg), 0, 0, None)
    torch.cuda.synchronize()
    assert rc == capi.VMC_ENOMEM
