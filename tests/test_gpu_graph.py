"""The decode step (quantize-on-append + split-KV decode + merge: three
launches) captured in a HIP graph and replayed: every replay, with eager work
and host synchronisations between replays, must equal the eager result bit
for bit (the kernels are deterministic; nothing in the captured calls
allocates or clears memory)."""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, make_workload

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("method", ["turboquant_3bit_nc", "turboquant_3bit_g32", "turboquant_k8v4"])
def test_decode_step_graph_replays(dev, method):
    import torch
    from vm_c_amd import capi
    w = make_workload([300, 1024, 17, 700], Hq=32, Hkv=8, seed=21, pool_slack=2)
    cfg = capi.tq_config(128, method)
    n = w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned
    cache = torch.zeros(n, dtype=torch.uint8, device=dev)
    slots = torch.from_numpy(w.slots).to(dev)
    capi.turboquant_store(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), cache, slots,
                          BS, cfg)
    B = len(w.seq_lens)
    last = torch.from_numpy(w.slots[np.cumsum(w.seq_lens) - 1]).to(dev)  # each sequence's last slot
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    k_new = torch.randn((B, w.Hkv, 128), generator=gen, device=dev).half()
    v_new = torch.randn((B, w.Hkv, 128), generator=gen, device=dev).half()
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.empty_like(q)
    bt, lens = torch.from_numpy(w.bt).to(dev), torch.from_numpy(w.seq_lens).to(dev)
    ws = torch.empty(capi.turboquant_decode_workspace_size(B, 32, w.Hkv, 128, w.bt.shape[1], BS),
                     dtype=torch.uint8, device=dev)

    def step(stream=None):
        capi.turboquant_store(k_new, v_new, cache, last, BS, cfg, stream=stream)
        capi.turboquant_decode_attention(out, q, cache, bt, lens, w.Hkv, float(w.scale), cfg, BS,
                                         workspace=ws, stream=stream)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for r in range(4):
        # eager work between replays: new q and new appended rows
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).half())
        k_new.copy_(torch.randn(k_new.shape, generator=gen, device=dev).half())
        torch.cuda.synchronize()
        step()
        torch.cuda.synchronize()
        want_out, want_cache = out.clone(), cache.clone()
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache, want_cache), f"replay {r}: pool bytes differ"
        assert torch.equal(out.view(torch.int16), want_out.view(torch.int16)), f"replay {r}: output differs"
    assert torch.isfinite(out.float()).all()
