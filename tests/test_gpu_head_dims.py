"""head_dim 64 and 256 on the GPU (the reference accepts head_dim <= 256 for
TurboQuant, kernels_turboquant.h:11, and 64 / 128 / 256 for prefill,
attention_kernels.cu:270-371).

  * TurboQuant store (4-bit, 3-bit, k3v4, fp8 keys; fp16 and bf16): every
    pool byte equal to the oracle's store; the decode and the per-token
    prefill over the same pages within |got - ref| <= 2e-3 + 1e-2 |ref| of the
    oracle's two-stage decode and of fp64 exact attention.
  * f16 / bf16 / q8_0 / q4_0 pages, NHD and HND: the append bit-exact
    against the oracle's; the paged decode, the per-token prefill and
    vmc_flash_attention_prefill_v2 against fp64 exact attention.
  * Local causal prefill with the quantize-on-append: rows against exact
    attention, pages against the oracle's append.
Batches hold an empty sequence, a one-token one and a block-table hole.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, close_report, f32_to_bf16_bits, make_workload, prefill_inputs

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
DIMS = [64, 256]


def _bits(x, bf16):
    return f32_to_bf16_bits(np.asarray(x, np.float32)) if bf16 else np.asarray(x).astype(np.float16).view(np.uint16)


def _dev(dev, bits, bf16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(
        torch.bfloat16 if bf16 else torch.float16)


def _f32(bits, bf16):
    return O.bf16_to_f32(bits) if bf16 else O.f16_to_f32(bits)


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc",
                                    "turboquant_k8v4"])
@pytest.mark.parametrize("bf16", [False, True])
def test_turboquant_store_decode(dev, d, method, bf16):
    import torch
    from vm_c_amd import capi
    lens = np.array([1, 37, 0, 300], np.int32)
    Hq, Hkv = 8, 2
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, D=d, seed=70 + d, holes=1)
    cfg = capi.tq_config(d, method)
    L = O.tq_layout(method, d)
    c, m = O.tq_tables(d, 4 if L.key_fp8 else L.key_quant_bits)
    kb, vb, qb = _bits(w.K, bf16), _bits(w.V, bf16), _bits(w.Q, bf16)
    n = w.num_blocks * BS * Hkv * cfg.slot_size_aligned
    cache = torch.zeros(n, dtype=torch.uint8, device=dev)
    capi.turboquant_store(_dev(dev, kb, bf16), _dev(dev, vb, bf16), cache, torch.from_numpy(w.slots).to(dev),
                          BS, cfg)
    ref = np.zeros(n, np.uint8)
    O.tq_store(kb, vb, w.slots, ref, BS, L, m, bf16=bf16)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"store bytes differ at {bad.size} positions (first {bad[:4]})"
    bt = torch.from_numpy(w.bt).to(dev)
    out = torch.full((len(lens), Hq, d), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16,
                     device=dev)
    capi.turboquant_decode_attention(out, _dev(dev, qb, bf16), cache, bt, torch.from_numpy(lens).to(dev), Hkv,
                                     float(w.scale), cfg)
    # a prefill step: the last 5 positions of each non-empty sequence, one row each
    tok_seq = np.concatenate([np.full(min(5, L_), b) for b, L_ in enumerate(lens)]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(max(L_ - 5, 0), L_) for L_ in lens]).astype(np.int32)
    rng = np.random.default_rng(d)
    qp = _bits(rng.standard_normal((tok_seq.size, Hq, d)).astype(np.float32), bf16)
    outp = torch.full((tok_seq.size, Hq, d), float("nan"), dtype=out.dtype, device=dev)
    capi.turboquant_prefill_attention(outp, _dev(dev, qp, bf16), cache, bt, torch.from_numpy(tok_seq).to(dev),
                                      torch.from_numpy(tok_pos).to(dev), Hkv, float(w.scale), cfg, block_size=BS)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    two = _f32(O.tq_decode(qb, ref, w.bt, lens, Hkv, np.float32(w.scale), BS, L, c, bf16=bf16), bf16)
    ok, err = close_report(got, two, ATOL, RTOL)
    assert ok, f"decode vs two-stage: {err}"
    ex = O.tq_decode_exact(qb, ref, w.bt, lens, Hkv, w.scale, BS, L, c, bf16=bf16)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"decode vs exact: {err}"
    assert (got[2] == 0).all()  # the empty sequence
    exp = O.tq_decode_exact(qp, ref, w.bt[tok_seq], tok_pos + 1, Hkv, w.scale, BS, L, c, bf16=bf16)
    ok, err = close_report(outp.float().cpu().numpy(), exp, ATOL, RTOL)
    assert ok, f"prefill rows vs exact: {err}"


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("fmt", [O.KV_F16, O.KV_BF16, O.KV_Q8_0, O.KV_Q4_0])
@pytest.mark.parametrize("hnd", [False, True])
def test_paged_decode_and_prefill(dev, d, fmt, hnd):
    import torch
    from vm_c_amd import capi
    lens = np.array([1, 200, 0, 77], np.int32)
    Hq, Hkv = 8, 2
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, D=d, seed=80 + d + fmt, holes=1, pool_slack=2)
    bf16 = fmt == O.KV_BF16
    kb, vb, qb = _bits(w.K, bf16), _bits(w.V, bf16), _bits(w.Q, bf16)
    E = O.entry_bytes(fmt, d)
    n = w.num_blocks * BS * Hkv * E
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    layout = capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD
    capi.reshape_and_cache(_dev(dev, kb, bf16), _dev(dev, vb, bf16), kc, vc, torch.from_numpy(w.slots).to(dev),
                           BS, kv_format=fmt, layout=layout)
    kr = np.zeros(n, np.uint8)
    vr = np.zeros(n, np.uint8)
    O.kv_append(kb, vb, w.slots, kr, vr, BS, fmt, hnd=hnd, src_bf16=bf16)
    bt = torch.from_numpy(w.bt).to(dev)
    out = torch.full((len(lens), Hq, d), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16, device=dev)
    capi.paged_attention_decode(out, _dev(dev, qb, bf16), kc, vc, bt, torch.from_numpy(lens).to(dev), Hkv,
                                float(w.scale), block_size=BS, kv_format=fmt, layout=layout)
    tok_seq = np.concatenate([np.full(min(6, L_), b) for b, L_ in enumerate(lens)]).astype(np.int32)
    tok_pos = np.concatenate([np.arange(max(L_ - 6, 0), L_) for L_ in lens]).astype(np.int32)
    qp = _bits(np.random.default_rng(d + fmt).standard_normal((tok_seq.size, Hq, d)).astype(np.float32), bf16)
    args = (kc, vc, bt, torch.from_numpy(tok_seq).to(dev), torch.from_numpy(tok_pos).to(dev), Hkv, float(w.scale))
    rows = torch.full((tok_seq.size, Hq, d), float("nan"), dtype=out.dtype, device=dev)
    capi.paged_attention_prefill(rows, _dev(dev, qp, bf16), *args, block_size=BS, kv_format=fmt, layout=layout,
                                 max_splits=1)
    v2 = torch.full_like(rows, float("nan"))
    capi.flash_attention_prefill_v2(v2, _dev(dev, qp, bf16), *args, block_size=BS, kv_format=fmt, layout=layout)
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().numpy(), kr) and np.array_equal(vc.cpu().numpy(), vr)
    ex = O.paged_decode_exact(_f32(qb, bf16), kr, vr, fmt, w.bt, lens, Hkv, float(w.scale), BS, hnd=hnd)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"decode: {err}"
    exp = O.paged_decode_exact(_f32(qp, bf16), kr, vr, fmt, w.bt[tok_seq], tok_pos + 1, Hkv, float(w.scale), BS,
                               hnd=hnd)
    for name, t in (("per-token prefill", rows), ("prefill_v2", v2)):
        ok, err = close_report(t.float().cpu().numpy(), exp, ATOL, RTOL)
        assert ok, f"{name}: {err}"


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("bf16", [False, True])
def test_local_prefill_with_append(dev, d, bf16):
    import torch
    from vm_c_amd import capi
    seq_lens, Hq, Hkv = [70, 1, 130], 8, 2
    qb, kb, vb, pos, cu = prefill_inputs(seq_lens, Hq, Hkv, D=d, seed=d, bf16=bf16)
    T = qb.shape[0]
    nblk = (T + BS - 1) // BS + 1
    slots = np.random.default_rng(d).permutation(nblk * BS)[:T].astype(np.int64)
    slots[3] = -1
    E = O.entry_bytes(O.KV_Q8_0, d)
    n = nblk * BS * Hkv * E
    kc = torch.zeros(n, dtype=torch.uint8, device=dev)
    vc = torch.zeros(n, dtype=torch.uint8, device=dev)
    out = torch.full((T, Hq, d), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16, device=dev)
    capi.flash_attention_prefill(out, _dev(dev, qb, bf16), _dev(dev, kb, bf16), _dev(dev, vb, bf16),
                                 torch.from_numpy(pos).to(dev), Hkv, 1 / np.sqrt(d), key_cache=kc, value_cache=vc,
                                 slot_mapping=torch.from_numpy(slots).to(dev), block_size=BS, kv_format=O.KV_Q8_0)
    torch.cuda.synchronize()
    toks = np.repeat(np.arange(T), Hq)
    heads = np.tile(np.arange(Hq), T)
    ex = O.prefill_exact_rows(qb, kb, vb, cu, Hkv, 1 / np.sqrt(d), toks, heads, is_bf16=bf16)
    ok, err = close_report(out.float().cpu().numpy().reshape(T * Hq, d), ex, ATOL, RTOL)
    assert ok, f"prefill: {err}"
    kr = np.zeros(n, np.uint8)
    vr = np.zeros(n, np.uint8)
    O.kv_append(kb, vb, slots, kr, vr, BS, O.KV_Q8_0, src_bf16=bf16)
    assert np.array_equal(kc.cpu().numpy(), kr) and np.array_equal(vc.cpu().numpy(), vr)


# head_dim 256 over 3- and 4-bit slots runs the MFMA decode of
# tq_decode_d256.hip (1, 2 or 4 KV heads, at most 8 query heads per KV head):
# the reference's deployment shape (16 query / 2 KV heads, 262-byte slots),
# the other head groupings, split counts that exercise the merge (0 = as
# many ranges as the GPU holds, 3) and the per-sequence mode (1), ragged
# lengths with an empty sequence, a one-token one, page-edge lengths and a
# block-table hole
@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
@pytest.mark.parametrize("heads", [(16, 2), (8, 1), (32, 4), (4, 4), (3, 1)])
@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("bf16", [False, True])
def test_tq_d256_decode(dev, method, heads, splits, bf16):
    import torch
    from vm_c_amd import capi
    d = 256
    Hq, Hkv = heads
    lens = np.array([1, 700, 0, 16, 33, 1024, 5, 257], np.int32)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, D=d, seed=300 + Hq + Hkv + splits, holes=1)
    cfg = capi.tq_config(d, method)
    L = O.tq_layout(method, d)
    c, m = O.tq_tables(d, L.key_quant_bits)
    kb, vb, qb = _bits(w.K, bf16), _bits(w.V, bf16), _bits(w.Q, bf16)
    n = w.num_blocks * BS * Hkv * cfg.slot_size_aligned
    cache = torch.zeros(n, dtype=torch.uint8, device=dev)
    capi.turboquant_store(_dev(dev, kb, bf16), _dev(dev, vb, bf16), cache, torch.from_numpy(w.slots).to(dev),
                          BS, cfg)
    out = torch.full((len(lens), Hq, d), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16,
                     device=dev)
    print(f"d256 decode {method} Hq={Hq} Hkv={Hkv} splits={splits} bf16={bf16}", flush=True)
    capi.turboquant_decode_attention(out, _dev(dev, qb, bf16), cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(lens).to(dev), Hkv, float(w.scale), cfg, max_splits=splits)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    pool = cache.cpu().numpy()
    two = _f32(O.tq_decode(qb, pool, w.bt, lens, Hkv, np.float32(w.scale), BS, L, c, bf16=bf16), bf16)
    ok, err = close_report(got, two, ATOL, RTOL)
    assert ok, f"decode vs two-stage: {err}"
    ex = O.tq_decode_exact(qb, pool, w.bt, lens, Hkv, w.scale, BS, L, c, bf16=bf16)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"decode vs exact: {err}"
    assert (got[2] == 0).all()  # the empty sequence


@pytest.mark.parametrize("method", ["turboquant_4bit_nc", "turboquant_3bit_nc"])
@pytest.mark.parametrize("bf16", [False, True])
def test_tq_d256_large_value_scales(dev, method, bf16):
    """V of magnitude ~2000 with peaked scores (q x 3): pages whose value
    scale exceeds 65504 / 2^8 take the exact running max, so fp16(P * scale)
    stays finite; against fp64 attention with atol 5e-3 * 2000 (the fp16
    P * scale operand's 11 bits against values of up to ~9 sigma)."""
    import torch
    from vm_c_amd import capi
    d, Hq, Hkv = 256, 16, 2
    lens = np.array([900, 37, 1600], np.int32)
    w = make_workload(lens, Hq=Hq, Hkv=Hkv, D=d, seed=17 + bf16)
    V = w.V.astype(np.float32) * 2000.0
    Q = w.Q.astype(np.float32) * 3.0
    cfg = capi.tq_config(d, method)
    L = O.tq_layout(method, d)
    c, _ = O.tq_tables(d, L.key_quant_bits)
    kb, vb, qb = _bits(w.K, bf16), _bits(V, bf16), _bits(Q, bf16)
    cache = torch.zeros(w.num_blocks * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
    capi.turboquant_store(_dev(dev, kb, bf16), _dev(dev, vb, bf16), cache, torch.from_numpy(w.slots).to(dev),
                          BS, cfg)
    out = torch.full((len(lens), Hq, d), float("nan"), dtype=torch.bfloat16 if bf16 else torch.float16,
                     device=dev)
    print(f"d256 large value scales {method} bf16={bf16}", flush=True)
    capi.turboquant_decode_attention(out, _dev(dev, qb, bf16), cache, torch.from_numpy(w.bt).to(dev),
                                     torch.from_numpy(lens).to(dev), Hkv, float(w.scale), cfg)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), "non-finite decode rows with large value scales"
    ex = O.tq_decode_exact(qb, cache.cpu().numpy(), w.bt, lens, Hkv, w.scale, BS, L, c, bf16=bf16)
    ok, err = close_report(got, ex, 5e-3 * 2000.0, RTOL)
    assert ok, f"vs exact: {err}"
