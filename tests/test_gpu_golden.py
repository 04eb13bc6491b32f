"""GPU parity against golden outputs of the reference's own code.

The fixtures in tests/golden/ hold the output of the vendored ggml CPU
flash_attn_ext (ggml-cpu/ops.cpp:8214-8957) on seeded inputs; the inputs are
regenerated here from the same seeds (checked by crc32), appended into the
paged cache by the HIP append kernel, and decoded by the HIP paged decode
through the C ABI.  Tolerance: |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import os

import numpy as np
import pytest

import kvgen
import oracle_lib as O
from kvgen import BS, close_report

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATOL, RTOL = 2e-3, 1e-2


def _decode(dev, w, fmt):
    import torch
    from vm_c_amd import capi
    E = O.entry_bytes(fmt, 128)
    nbytes = w.num_blocks * BS * w.Hkv * E
    kc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    vc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    tdt = torch.bfloat16 if fmt == O.KV_BF16 else torch.float16
    K = torch.from_numpy(w.K).to(dev).float().to(tdt)
    V = torch.from_numpy(w.V).to(dev).float().to(tdt)
    capi.reshape_and_cache(K, V, kc, vc, torch.from_numpy(w.slots).to(dev), BS, kv_format=fmt)
    q = torch.from_numpy(w.Q).to(dev).float().to(tdt)
    out = torch.full_like(q, float("nan"))
    print(f"decode fmt={fmt} B={w.B} lens={w.seq_lens.tolist()[:4]}...", flush=True)
    capi.paged_attention_decode(out, q, kc, vc, torch.from_numpy(w.bt).to(dev),
                                torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale),
                                block_size=BS, kv_format=fmt)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), q.float().cpu().numpy()


@pytest.mark.parametrize("fmt,name", [(O.KV_F16, "f16"), (O.KV_BF16, "bf16")])
def test_single_sequence_2048_vs_reference(dev, fmt, name):
    """Batch 1, 32/8 heads, 2048 tokens, block table a permutation of 128 pages."""
    g = np.load(os.path.join(GOLD, f"fa_decode_{name}.npz"))
    w = kvgen.single_seq_fp16_workload()
    assert (kvgen.crc(w.K), kvgen.crc(w.V), kvgen.crc(w.Q)) == (g["crc_k"], g["crc_v"], g["crc_q"])
    got = _decode(dev, w, fmt)[0]
    for key in ("out_nth1", "out_nth4"):
        ok, err = close_report(got, g[key], ATOL, RTOL)
        assert ok, f"{key}: max err {err}"


@pytest.mark.parametrize("fmt,name", [(O.KV_Q8_0, "q8_0"), (O.KV_Q4_0, "q4_0")])
def test_batched_quantized_vs_reference(dev, fmt, name):
    """Batch 16, 32/8 heads, lengths uniform in [512, 4096] (seed 1), K/V
    quantized on append; the first sequences against the reference's output,
    all of them against the restatement and fp64 exact attention."""
    g = np.load(os.path.join(GOLD, f"fa_decode_{name}.npz"))
    w = kvgen.batched_q8_0_workload()
    assert (kvgen.crc(w.K), kvgen.crc(w.V), kvgen.crc(w.Q)) == (g["crc_k"], g["crc_v"], g["crc_q"])
    got, kc, vc, qf = _decode(dev, w, fmt)
    n = len(g["seqs"])
    ok, err = close_report(got[:n], g["out"], ATOL, RTOL)
    assert ok, f"vs reference: max err {err}"
    ref = O.decode_ggml(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale), BS, nth=1)
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs restatement: max err {err}"
    ex = O.paged_decode_exact(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"
