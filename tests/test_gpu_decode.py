"""Paged decode parity on the GPU.

Each case appends K/V with the HIP append kernel (bit-exactness of which is
tested separately), runs the HIP decode through the C ABI, and compares with
(i) exact fp64 attention over the dequantized pages and (ii) the oracle's
restatement of the reference algorithm (ggml CPU flash-attention for
f16/q8_0/q4_0, the two-stage TurboQuant decode for TQ).  Tolerance (the
reference's): |got - ref| <= 2e-3 + 1e-2 * |ref|.
"""
import zlib

import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, make_workload

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _run_paged(dev, w, fmt, hnd=False, max_splits=0):
    import torch
    from vm_c_amd import capi
    E = O.entry_bytes(fmt, w.D)
    nbytes = w.num_blocks * BS * w.Hkv * E
    kc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    vc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    tdt = torch.bfloat16 if fmt == O.KV_BF16 else torch.float16
    Kt = torch.from_numpy(w.K).to(dev).to(tdt)
    Vt = torch.from_numpy(w.V).to(dev).to(tdt)
    lay = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    if w.K.shape[0]:
        capi.reshape_and_cache(Kt, Vt, kc, vc, torch.from_numpy(w.slots).to(dev), BS,
                               kv_format=fmt, layout=lay)
    q = torch.from_numpy(w.Q).to(dev).to(tdt)
    out = torch.full_like(q, float("nan"))
    capi.paged_attention_decode(out, q, kc, vc, torch.from_numpy(w.bt).to(dev),
                                torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale),
                                block_size=BS, kv_format=fmt, layout=lay, max_splits=max_splits)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), q.float().cpu().numpy()


CASES = {
    "cfg1_small": dict(seq_lens=[2048], Hq=32, Hkv=8),
    "ragged": dict(seq_lens=[1, 15, 16, 17, 100, 513, 0, 700], Hq=16, Hkv=4),
    "gqa8": dict(seq_lens=[300, 1200], Hq=64, Hkv=8),
    "mha": dict(seq_lens=[64, 250], Hq=8, Hkv=8),
}


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("case", list(CASES))
def test_paged_decode_vs_exact(dev, fmt, case):
    w = make_workload(seed=zlib.crc32(case.encode()) % 1000, **CASES[case])
    got, kc, vc, qf = _run_paged(dev, w, fmt)
    ex = O.paged_decode_exact(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
    # zero-length sequences produce a zero row
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"max err {err}"
    assert np.isfinite(got).all()


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_Q8_0])
def test_paged_decode_more_than_64_pieces(dev, fmt):
    """One 8192-token sequence over ~256 page ranges of 2 pages: the merge
    combines ~254 pieces per head in rounds of 64, rescaling its running max
    when a later round holds a larger one."""
    w = make_workload([8192, 40], Hq=32, Hkv=8, seed=31)
    got, kc, vc, qf = _run_paged(dev, w, fmt)
    ex = O.paged_decode_exact(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"max err {err}"


@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_Q8_0, O.KV_Q4_0])
def test_paged_decode_vs_ggml_restatement(dev, fmt):
    w = make_workload(seq_lens=[2048, 777], Hq=32, Hkv=8, seed=3)
    got, kc, vc, qf = _run_paged(dev, w, fmt)
    ref = O.decode_ggml(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale), BS, nth=1)
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"max err {err}"


def test_paged_decode_hnd_layout(dev):
    w = make_workload(seq_lens=[333, 64], Hq=16, Hkv=4, seed=9)
    for fmt in (O.KV_F16, O.KV_Q8_0):
        got, kc, vc, qf = _run_paged(dev, w, fmt, hnd=True)
        ex = O.paged_decode_exact(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS, hnd=True)
        ok, err = close_report(got, ex, ATOL, RTOL)
        assert ok, f"fmt {fmt}: max err {err}"


def test_paged_decode_block_table_holes(dev):
    w = make_workload(seq_lens=[400, 900, 64], Hq=16, Hkv=8, seed=21, holes=4)
    for fmt in (O.KV_F16, O.KV_Q8_0):
        got, kc, vc, qf = _run_paged(dev, w, fmt)
        ex = O.paged_decode_exact(qf, kc, vc, fmt, w.bt, w.seq_lens, w.Hkv, w.scale, BS)
        ok, err = close_report(got, ex, ATOL, RTOL)
        assert ok, f"fmt {fmt}: max err {err}"


def test_paged_decode_split_invariance(dev):
    w = make_workload(seq_lens=[3000, 1500, 40], Hq=32, Hkv=8, seed=4)
    outs = [_run_paged(dev, w, O.KV_Q8_0, max_splits=ms)[0] for ms in (1, 2, 7, 64)]
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 1e-3


def test_paged_decode_permutation_invariance(dev):
    """Same K/V in a differently permuted pool gives the same output."""
    a = make_workload(seq_lens=[500, 260], Hq=16, Hkv=4, seed=8, pool_slack=0)
    b = make_workload(seq_lens=[500, 260], Hq=16, Hkv=4, seed=8, pool_slack=7)
    # same RNG stream for K/V/Q needs the same draws: rebuild b's data from a
    b.K, b.V, b.Q = a.K, a.V, a.Q
    oa = _run_paged(dev, a, O.KV_F16)[0]
    ob = _run_paged(dev, b, O.KV_F16)[0]
    assert np.abs(oa - ob).max() < 1e-3


# ---------------------------------------------------------------- TurboQuant

def _run_tq(dev, w, method, max_splits=0):
    import torch
    from vm_c_amd import capi
    L = O.tq_layout(method)
    cfg = capi.tq_config(128, method)
    nbytes = w.num_blocks * BS * w.Hkv * L.slot_size_aligned
    cache = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    if w.K.shape[0]:
        capi.turboquant_store(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), cache,
                              torch.from_numpy(w.slots).to(dev), BS, cfg)
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale),
                                     cfg, block_size=BS, max_splits=max_splits)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), cache.cpu().numpy(), L


TQ_CASES = {
    "cfg3_small": dict(seq_lens=[1024, 1024], Hq=32, Hkv=8),
    "cfg5_small": dict(seq_lens=[1024, 4000, 32], Hq=64, Hkv=8),
    "ragged": dict(seq_lens=[1, 17, 0, 300], Hq=16, Hkv=4),
    # 16 query heads per KV head: the S tile's columns all hold heads of one page
    "gqa16": dict(seq_lens=[300, 1024, 17, 33], Hq=32, Hkv=2),
}


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc"])
@pytest.mark.parametrize("case", list(TQ_CASES))
def test_tq_decode(dev, method, case):
    w = make_workload(seed=len(case) * 7, **TQ_CASES[case])
    got, cache, L = _run_tq(dev, w, method)
    c, _ = O.tq_tables(128, L.key_quant_bits)
    qb = bits16(w.Q)
    ex = O.tq_decode_exact(qb, cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"
    ref = O.f16_to_f32(O.tq_decode(qb, cache, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale), BS, L, c,
                                   num_splits=32))
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs reference restatement: max err {err}"


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
def test_tq_decode_more_than_64_pieces(dev, method):
    """The ring kernel and the merge on one 8192-token sequence cut into
    ~254 pieces (rounds of 64 with a running max)."""
    w = make_workload([8192, 40], Hq=32, Hkv=8, seed=32)
    got, cache, L = _run_tq(dev, w, method)
    c, _ = O.tq_tables(128, L.key_quant_bits)
    ex = O.tq_decode_exact(bits16(w.Q), cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"


@pytest.mark.parametrize("max_splits", [0, 1])
def test_tq_4bit_without_norm_correction(dev, max_splits):
    """4-bit keys and values with the norm correction off (the reference's
    4/4 decode without it, turboquant_kernels.cu:901-912: keys are the
    centroids times the stored norm, no division by ||C[codes]||).  The decode
    and both prefill paths (15 tokens: one decode row per token; 40 tokens:
    the tiled prefill) against fp64 attention over the same slots."""
    import torch
    from vm_c_amd import capi
    w = make_workload(seq_lens=[300, 1024, 17, 0], Hq=16, Hkv=4, seed=90 + max_splits)
    L = O.tq_layout("turboquant_4bit_nc")
    L.norm_correction = 0
    cfg = capi.tq_config(128, "turboquant_4bit_nc")
    cfg.norm_correction = 0
    cache = torch.zeros(w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    capi.turboquant_store(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), cache,
                          torch.from_numpy(w.slots).to(dev), BS, cfg)
    bt = torch.from_numpy(w.bt).to(dev)
    q = torch.from_numpy(w.Q).to(dev)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, bt, torch.from_numpy(w.seq_lens).to(dev), w.Hkv,
                                     float(w.scale), cfg, block_size=BS, max_splits=max_splits)
    rng = np.random.default_rng(max_splits)
    outs = []
    for T in (15, 40):
        tok_seq = rng.integers(0, 3, T).astype(np.int32)
        tok_pos = (rng.random(T) * w.seq_lens[tok_seq]).astype(np.int32)
        qp = rng.standard_normal((T, 16, 128)).astype(np.float16)
        o = torch.full((T, 16, 128), float("nan"), dtype=torch.float16, device=dev)
        capi.turboquant_prefill_attention(o, torch.from_numpy(qp).to(dev), cache, bt,
                                          torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev),
                                          w.Hkv, float(w.scale), cfg, block_size=BS)
        outs.append((qp, tok_seq, tok_pos, o))
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    c, _ = O.tq_tables(128, 4)
    ex = O.tq_decode_exact(bits16(w.Q), got_cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"decode: max err {err}"
    L1 = O.tq_layout("turboquant_4bit_nc")
    ex1 = O.tq_decode_exact(bits16(w.Q), got_cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L1, c)
    assert not close_report(out.float().cpu().numpy(), ex1, ATOL, RTOL)[0], "the flag changed nothing"
    for qp, tok_seq, tok_pos, o in outs:
        ex = O.tq_decode_exact(bits16(qp), got_cache, w.bt[tok_seq], tok_pos + 1, w.Hkv, w.scale, BS, L, c)
        ok, err = close_report(o.float().cpu().numpy(), ex, ATOL, RTOL)
        assert ok, f"prefill of {len(tok_seq)} tokens: max err {err}"


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc"])
@pytest.mark.parametrize("case", ["cfg5_small", "ragged", "gqa16"])
@pytest.mark.parametrize("max_splits", [0, 1])
def test_tq_decode_bf16(dev, method, case, max_splits):
    """bf16 activations: the store writes bf16 norms/scales/zeros (the
    reference's compute-dtype dispatch, turboquant_kernels.cu:808, :966) and
    the decode reads bf16 q and those pages and writes bf16 rows (its USE_BF16
    stage 1, :353, :445-461).  Pool bytes bit-exact against the oracle's bf16
    store; output against fp64 attention over the same pages and against the
    oracle's two-stage restatement with bf16 halves."""
    import torch
    from kvgen import f32_to_bf16_bits
    from vm_c_amd import capi
    w = make_workload(seed=len(case) * 11 + max_splits, **TQ_CASES[case])
    kb16, vb16, qb16 = (f32_to_bf16_bits(x.astype(np.float32)) for x in (w.K, w.V, w.Q))
    L = O.tq_layout(method)
    cfg = capi.tq_config(w.D, method)
    cache = torch.zeros(w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    as_bf16 = lambda b: torch.from_numpy(b.view(np.int16)).to(dev).view(torch.bfloat16)
    if w.K.shape[0]:
        capi.turboquant_store(as_bf16(kb16), as_bf16(vb16), cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    q = as_bf16(qb16)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale), cfg,
                                     block_size=BS, max_splits=max_splits)
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    c, m = O.tq_tables(128, L.key_quant_bits)
    ref_cache = np.zeros_like(got_cache)
    O.tq_store(kb16, vb16, w.slots, ref_cache, BS, L, m, bf16=True)
    assert np.array_equal(got_cache, ref_cache), "bf16 TurboQuant store bytes differ from the oracle"
    got = out.float().cpu().numpy()
    ex = O.tq_decode_exact(qb16, ref_cache, w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c, bf16=True)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"
    ref = O.tq_decode(qb16, ref_cache, w.bt, w.seq_lens, w.Hkv, np.float32(w.scale), BS, L, c,
                      num_splits=32, bf16=True)
    ref = (ref.astype(np.uint32) << 16).view(np.float32)
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs reference restatement: max err {err}"


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
@pytest.mark.parametrize("heads", [(64, 8), (16, 4), (32, 2)])
@pytest.mark.parametrize("bf16", [False, True])
def test_tq_decode_large_value_scales(dev, method, heads, bf16):
    """V of magnitude ~2000 (value scales of ~300-2000 per token) with peaked
    scores (q x 3): P enters the PV product as fp16(P * scale), and with the
    lazy running max P reaches 2^8, so these pages must take the exact max
    (P <= 1) or the product overflows to inf.  Output against fp64 attention
    over the stored pages, with the absolute tolerance scaled to the values:
    the fp16 P * scale operand carries 11 bits relative to the value range
    (up to ~9 sigma), so a dominant token contributes up to 2^-11 * 9 sigma
    ~ 0.0044 sigma of error; atol = 5e-3 * 2000.  Heads (64, 8) run the 3-bit
    streaming kernel, (16, 4) the pipelined kernel, (32, 2) the
    16-heads-per-page kernel."""
    import torch
    from kvgen import f32_to_bf16_bits
    from vm_c_amd import capi
    Hq, Hkv = heads
    w = make_workload([1500, 37, 4000], Hq=Hq, Hkv=Hkv, seed=Hq + Hkv + (5 if bf16 else 0))
    V = w.V.astype(np.float32) * 2000.0
    Q = w.Q.astype(np.float32) * 3.0
    L = O.tq_layout(method)
    cfg = capi.tq_config(w.D, method)
    cache = torch.zeros(w.num_blocks * BS * w.Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    if bf16:
        kb, vb, qb = (f32_to_bf16_bits(x.astype(np.float32)) for x in (w.K, V, Q))
        conv = lambda b: torch.from_numpy(b.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        kb, vb, qb = (x.astype(np.float16).view(np.uint16) for x in (w.K, V, Q))
        conv = lambda b: torch.from_numpy(b.view(np.float16)).to(dev)
    capi.turboquant_store(conv(kb), conv(vb), cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    q = conv(qb)
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(w.seq_lens).to(dev), w.Hkv, float(w.scale), cfg,
                                     block_size=BS)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), "non-finite decode rows with large value scales"
    c, _ = O.tq_tables(128, L.key_quant_bits)
    ex = O.tq_decode_exact(qb, cache.cpu().numpy(), w.bt, w.seq_lens, w.Hkv, w.scale, BS, L, c, bf16=bf16)
    ok, err = close_report(got, ex, 5e-3 * 2000.0, RTOL)
    assert ok, f"vs exact: max err {err}"


@pytest.mark.parametrize("heads", [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4)])
def test_tq_decode_workspace_contents_do_not_matter(dev, heads):
    """The split decode keeps no state in the workspace between calls: every
    partial row the merge reads is written by the same call, so random bytes
    in the workspace, or the leftovers of a call of another shape, give the
    same output bit for bit as a zero-filled one.  G = 1, 2, 3, 4 and 8 query
    heads per KV head; the lengths cut sequences into 2 to ~60 pieces and
    include an empty one (whose rows must come out zero)."""
    import torch
    from vm_c_amd import capi
    Hq, Hkv = heads
    cfg = capi.tq_config(128, "turboquant_3bit_nc")
    gen = torch.Generator(device=dev)
    gen.manual_seed(Hq)
    ws = None
    for i, lens in enumerate(([32768, 1000, 0, 5000, 17], [3000, 64, 12000])):
        w = make_workload(seq_lens=lens, Hq=Hq, Hkv=Hkv, seed=40 + i + Hq)
        cache = torch.zeros(w.num_blocks * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
        capi.turboquant_store(torch.from_numpy(w.K).to(dev), torch.from_numpy(w.V).to(dev), cache,
                              torch.from_numpy(w.slots).to(dev), BS, cfg)
        q = torch.from_numpy(w.Q).to(dev)
        bt, sl = torch.from_numpy(w.bt).to(dev), torch.from_numpy(w.seq_lens).to(dev)
        need = capi.turboquant_decode_workspace_size(len(lens), Hq, Hkv, 128, w.bt.shape[1], BS)
        print(f"heads {Hq}/{Hkv} lens {lens} workspace {need} B", flush=True)
        if ws is None:  # the second shape reuses the first call's workspace as it was left
            ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device=dev, generator=gen)
        assert ws.numel() >= need
        got = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention(got, q, cache, bt, sl, Hkv, float(w.scale), cfg, BS, workspace=ws)
        ref = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention(ref, q, cache, bt, sl, Hkv, float(w.scale), cfg, BS,
                                         workspace=torch.zeros(need, dtype=torch.uint8, device=dev))
        again = torch.full_like(q, float("nan"))
        capi.turboquant_decode_attention(again, q, cache, bt, sl, Hkv, float(w.scale), cfg, BS, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i}: output depends on workspace bytes"
        assert torch.equal(again.view(torch.int16), ref.view(torch.int16)), f"call {i}: second call differs"
        c, _ = O.tq_tables(128, 3)
        ex = O.tq_decode_exact(bits16(w.Q), cache.cpu().numpy(), w.bt, w.seq_lens, Hkv, w.scale, BS,
                               O.tq_layout("turboquant_3bit_nc"), c)
        ok, err = close_report(got.float().cpu().numpy(), ex, ATOL, RTOL)
        assert ok, f"call {i}: max err {err}"
        assert (got.float().cpu().numpy()[np.asarray(lens) == 0] == 0).all()
