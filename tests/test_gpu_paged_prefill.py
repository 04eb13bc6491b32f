"""GPU parity of the prefill over a cached prefix (vmc_paged_attention_prefill;
reference paged_attention_prefill, src/cuda/attention_kernels.cu:416-436):
every prefix and new token is appended into the pages first, then each new
token t (position p of sequence s) attends positions 0 .. p of s through the
block table.  Checked against the oracle's fp64 attention over the same
pages with one row per token (block-table row of s, length p + 1), for
f16 / q8_0 / q4_0 pages, NHD and HND, one pass per token and split-KV, and a
sequence with no prefix.  Tolerance |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, f32_to_bf16_bits, make_workload

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("splits", [1, 8])
def test_paged_prefill_over_cached_prefix(dev, fmt, hnd, splits):
    import torch
    from vm_c_amd import capi
    prefix = np.array([100, 0, 513])
    new = np.array([37, 20, 64])
    lens = prefix + new
    Hq, Hkv = 16, 4
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=31 + fmt, pool_slack=2)
    E = O.entry_bytes(fmt, 128)
    n = w.num_blocks * BS * Hkv * E
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    layout = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    capi.reshape_and_cache(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), kc, vc,
                           torch.from_numpy(w.slots).to(dev), BS, kv_format=fmt, layout=layout)
    tok_seq = np.concatenate([np.full(new[b], b) for b in range(len(lens))]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(prefix[b], lens[b]) for b in range(len(lens))]).astype(np.int32)
    T = tok_seq.size
    rng = np.random.default_rng(5)
    q = rng.standard_normal((T, Hq, 128)).astype(np.float16)
    out = torch.full((T, Hq, 128), float("nan"), dtype=torch.float16, device=dev)
    capi.paged_attention_prefill(out, torch.from_numpy(q).to(dev), kc, vc, torch.from_numpy(w.bt).to(dev),
                                 torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev), Hkv,
                                 float(w.scale), block_size=BS, kv_format=fmt, layout=layout,
                                 max_splits=splits)
    torch.cuda.synchronize()
    ex = O.paged_decode_exact(q.astype(np.float32), kc.cpu().numpy(), vc.cpu().numpy(), fmt,
                              w.bt[tok_seq], tok_pos + 1, Hkv, float(w.scale), BS, hnd=hnd)
    ok, err = close_report(out.float().cpu().numpy(), ex, 2e-3, 1e-2)
    assert ok, f"max err {err}"


def _tq_cache(dev, w, cfg, bf16):
    import torch
    from vm_c_amd import capi
    cache = torch.zeros(w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    dt = torch.bfloat16 if bf16 else torch.float16
    k = torch.from_numpy(w.K).to(dev).to(dt)
    v = torch.from_numpy(w.V).to(dev).to(dt)
    capi.turboquant_store(k, v, cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    return cache


def _q_bits(q, bf16):
    return f32_to_bf16_bits(q) if bf16 else q.astype(np.float16).view(np.uint16)


def _q_dev(dev, qbits, bf16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(qbits).view(np.int16)).to(dev).view(
        torch.bfloat16 if bf16 else torch.float16)


def _tq_exact(method, qbits, cache, bt_rows, len_rows, Hkv, scale, bf16):
    if method.endswith("_g32"):
        return O.g32_decode_exact(qbits, cache, bt_rows, len_rows, Hkv, scale, BS, 4 if "4bit" in method else 3,
                                  0, bf16=bf16)
    L = O.tq_layout(method)
    c, _ = O.tq_tables(128, 4 if L.key_fp8 else L.key_quant_bits)
    return O.tq_decode_exact(qbits, cache, bt_rows, len_rows, Hkv, scale, BS, L, c, bf16=bf16)


@pytest.mark.parametrize("method", ["turboquant_3bit_nc", "turboquant_4bit_nc", "turboquant_k3v4_nc",
                                    "turboquant_4bit_g32", "turboquant_k8v4"])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("chunk", ["tiled", "per_token"])
def test_turboquant_prefill_over_cached_prefix(dev, method, bf16, chunk):
    """vmc_turboquant_prefill_attention (no reference counterpart: the
    reference's TurboQuant prefill attends only the step's local K/V).  A
    step of 121 tokens over reference-layout slots (codebook or fp8 keys)
    takes the tiled prefill; one of 15 tokens (and every step over
    per-32-group slots) one decode row per token."""
    import torch
    from vm_c_amd import capi
    if method.endswith("_g32") and bf16:
        pytest.skip("the per-32-group variant takes fp16 queries")
    prefix = np.array([100, 0, 513])
    new = np.array([37, 20, 64]) if chunk == "tiled" else np.array([5, 3, 7])
    lens = prefix + new
    Hq, Hkv = 16, 4
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=41, pool_slack=2, holes=3)
    cfg = capi.tq_config(128, method)
    cache = _tq_cache(dev, w, cfg, bf16)
    tok_seq = np.concatenate([np.full(new[b], b) for b in range(len(lens))]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(prefix[b], lens[b]) for b in range(len(lens))]).astype(np.int32)
    T = tok_seq.size
    qbits = _q_bits(np.random.default_rng(6).standard_normal((T, Hq, 128)).astype(np.float32), bf16)
    out = torch.full((T, Hq, 128), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16, device=dev)
    capi.turboquant_prefill_attention(out, _q_dev(dev, qbits, bf16), cache, torch.from_numpy(w.bt).to(dev),
                                      torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev),
                                      Hkv, float(w.scale), cfg, block_size=BS)
    torch.cuda.synchronize()
    ex = _tq_exact(method, qbits, cache.cpu().numpy(), w.bt[tok_seq], (tok_pos + 1).astype(np.int32), Hkv,
                   float(w.scale), bf16)
    ok, err = close_report(out.float().cpu().numpy(), ex, 2e-3, 1e-2)
    assert ok, f"max err {err}"


@pytest.mark.parametrize("method", ["turboquant_3bit_nc", "turboquant_4bit_nc", "turboquant_k8v4"])
def test_turboquant_prefill_chunk_over_long_prefix(dev, method):
    """A 2048-token chunk over a 30720-token prefix of reference-layout slots
    (codebook or fp8 keys), 32/8 heads (the tiled prefill): every row against
    the per-token path (steps of 15 tokens, which the test above pins to the
    oracle), 32 sampled tokens x all heads against the oracle's fp64
    attention."""
    import torch
    from vm_c_amd import capi
    prefix, new = 30720, 2048
    Hq, Hkv = 32, 8
    w = make_workload([prefix + new], Hq=Hq, Hkv=Hkv, seed=62)
    cfg = capi.tq_config(128, method)
    cache = _tq_cache(dev, w, cfg, False)
    tok_seq = np.zeros(new, np.int32)
    tok_pos = np.arange(prefix, prefix + new, dtype=np.int32)
    q = np.random.default_rng(10).standard_normal((new, Hq, 128)).astype(np.float16)
    qt = torch.from_numpy(q).to(dev)
    bt = torch.from_numpy(w.bt).to(dev)
    ts, tp = torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev)
    out = torch.full_like(qt, float("nan"))
    capi.turboquant_prefill_attention(out, qt, cache, bt, ts, tp, Hkv, float(w.scale), cfg, block_size=BS)
    rows = torch.full_like(qt, float("nan"))
    for a in range(0, new, 15):
        b = min(a + 15, new)
        capi.turboquant_prefill_attention(rows[a:b], qt[a:b], cache, bt, ts[a:b], tp[a:b], Hkv, float(w.scale),
                                          cfg, block_size=BS)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ok, err = close_report(got, rows.float().cpu().numpy(), 2e-3, 1e-2)
    assert ok, f"vs per-token path: max err {err}"
    pick = np.concatenate([[0, 1, 63, 64, new - 1], np.random.default_rng(11).integers(0, new, 27)])
    ex = _tq_exact(method, bits16(q[pick]), cache.cpu().numpy(), w.bt[tok_seq[pick]],
                   (tok_pos[pick] + 1).astype(np.int32), Hkv, float(w.scale), False)
    ok, err = close_report(got[pick], ex, 2e-3, 1e-2)
    assert ok, f"vs exact: max err {err}"


def _pages(dev, w, fmt, hnd):
    import torch
    from vm_c_amd import capi
    E = O.entry_bytes(fmt, 128)
    n = w.num_blocks * BS * w.Hkv * E
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    capi.reshape_and_cache(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), kc, vc,
                           torch.from_numpy(w.slots).to(dev), BS, kv_format=fmt,
                           layout=capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD)
    return kc, vc


def _q_as_page_type(q16, q_bf16, fmt):
    """The query values the tiled kernel multiplies: q rounded to the page
    type (q8_0 / q4_0 pages: fp16)."""
    from kvgen import f32_to_bf16_bits
    qf = O.bf16_to_f32(q16) if q_bf16 else O.f16_to_f32(q16)
    if fmt == O.KV_BF16 and not q_bf16:
        return O.bf16_to_f32(f32_to_bf16_bits(qf))
    if fmt != O.KV_BF16 and q_bf16:
        return qf.astype(np.float16).astype(np.float32)
    return qf


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("q_bf16", [False, True])
def test_prefill_v2_vs_exact(dev, fmt, hnd, q_bf16):
    """vmc_flash_attention_prefill_v2 (tiled MFMA over the pages) against the
    oracle's fp64 attention over the same pages, one row per token.  The
    batch mixes a 100-token prefix, none, and a 513-token prefix, chunks of
    37 / 20 / 64 tokens (so 64-row query blocks hold several sequences), a
    hole in a block table and a token of an out-of-range sequence (zeros)."""
    import torch
    from kvgen import f32_to_bf16_bits
    from vm_c_amd import capi
    prefix = np.array([100, 0, 513])
    new = np.array([37, 20, 64])
    lens = prefix + new
    Hq, Hkv = 16, 4
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, seed=51 + fmt, pool_slack=2)
    w.bt[2, 5] = -1  # a hole inside the third sequence's prefix
    kc, vc = _pages(dev, w, fmt, hnd)
    tok_seq = np.concatenate([np.full(new[b], b) for b in range(len(lens))]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(prefix[b], lens[b]) for b in range(len(lens))]).astype(np.int32)
    tok_seq[40] = 7  # outside the batch: zeros
    T = tok_seq.size
    qf = np.random.default_rng(7).standard_normal((T, Hq, 128)).astype(np.float32)
    q16 = f32_to_bf16_bits(qf) if q_bf16 else qf.astype(np.float16).view(np.uint16)
    tdt = torch.bfloat16 if q_bf16 else torch.float16
    qt = torch.from_numpy(q16.view(np.int16)).to(dev).view(tdt)
    out = torch.full_like(qt, float("nan"))
    capi.flash_attention_prefill_v2(out, qt, kc, vc, torch.from_numpy(w.bt).to(dev),
                                    torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev),
                                    Hkv, float(w.scale), block_size=BS, kv_format=fmt,
                                    layout=capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ok_rows = tok_seq < len(lens)
    assert np.all(got[~ok_rows] == 0)
    qe = _q_as_page_type(q16, q_bf16, fmt)[ok_rows]
    ex = O.paged_decode_exact(qe, kc.cpu().numpy(), vc.cpu().numpy(), fmt, w.bt[tok_seq[ok_rows]],
                              tok_pos[ok_rows] + 1, Hkv, float(w.scale), BS, hnd=hnd)
    ok, err = close_report(got[ok_rows], ex, 2e-3, 1e-2)
    assert ok, f"max err {err}"


@pytest.mark.parametrize("fmt", [O.KV_Q8_0, O.KV_F16])
def test_prefill_v2_chunk_over_long_prefix(dev, fmt):
    """Chunked prefill at its serving shape: a 2048-token chunk over a
    30720-token cached prefix, 32/8 heads, fp16 q.  Every row against the
    per-token path (vmc_paged_attention_prefill, which the tests above pin
    to the oracle), 32 sampled tokens x all heads against the oracle's fp64
    attention."""
    import torch
    from vm_c_amd import capi
    prefix, new = 30720, 2048
    Hq, Hkv = 32, 8
    w = make_workload([prefix + new], Hq=Hq, Hkv=Hkv, seed=61)
    kc, vc = _pages(dev, w, fmt, False)
    tok_seq = np.zeros(new, np.int32)
    tok_pos = np.arange(prefix, prefix + new, dtype=np.int32)
    q = np.random.default_rng(8).standard_normal((new, Hq, 128)).astype(np.float16)
    qt = torch.from_numpy(q).to(dev)
    args = (kc, vc, torch.from_numpy(w.bt).to(dev), torch.from_numpy(tok_seq).to(dev),
            torch.from_numpy(tok_pos).to(dev), Hkv, float(w.scale))
    out = torch.full_like(qt, float("nan"))
    capi.flash_attention_prefill_v2(out, qt, *args, block_size=BS, kv_format=fmt)
    rows = torch.full_like(qt, float("nan"))
    capi.paged_attention_prefill(rows, qt, *args, block_size=BS, kv_format=fmt, max_splits=1)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ok, err = close_report(got, rows.float().cpu().numpy(), 2e-3, 1e-2)
    assert ok, f"vs per-token path: max err {err}"
    pick = np.concatenate([[0, 1, 63, 64, new - 1], np.random.default_rng(9).integers(0, new, 27)])
    ex = O.paged_decode_exact(q[pick].astype(np.float32), kc.cpu().numpy(), vc.cpu().numpy(), fmt,
                              w.bt[tok_seq[pick]], tok_pos[pick] + 1, Hkv, float(w.scale), BS)
    ok, err = close_report(got[pick], ex, 2e-3, 1e-2)
    assert ok, f"vs exact: max err {err}"
