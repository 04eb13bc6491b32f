"""TurboQuant store + decode parity at the full benchmark shapes.

  * 4-bit (turboquant_4bit_nc), batch 32, 32/8 heads, 8192 tokens each,
    K/V N(0,1) fp16 (seed 2): every slot byte of the pool bit-exact against
    the oracle's store, every output row against the oracle's two-stage
    decode and fp64 exact attention over the same pages.
  * 3-bit (turboquant_3bit_nc), batch 64, 64/8 heads, lengths log-uniform
    in [1024, 32768] (seed 4) with one at 32768 (745,454 tokens): every slot
    byte of the pool bit-exact against the oracle's store, every one of the
    64 output rows against the oracle's two-stage decode and fp64 exact
    attention.
K/V are drawn on the device (torch generator) and copied back for the
oracle, so the check covers the exact bytes the kernels saw.
Tolerance: |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, close_report

pytestmark = pytest.mark.gpu

D = 128
ATOL, RTOL = 2e-3, 1e-2


def _layout(lens, seed):
    rng = np.random.default_rng(seed)
    pages = (lens + BS - 1) // BS
    nblk = int(pages.sum())
    perm = rng.permutation(nblk).astype(np.int32)
    bt = np.full((len(lens), int(pages.max())), -1, np.int32)
    k = 0
    for b in range(len(lens)):
        bt[b, :pages[b]] = perm[k:k + pages[b]]
        k += pages[b]
    tb = np.repeat(np.arange(len(lens)), lens)
    tp = np.concatenate([np.arange(n) for n in lens])
    slots = bt[tb, tp // BS].astype(np.int64) * BS + tp % BS
    return bt, slots, nblk


def _run(dev, method, lens, Hq, Hkv, seed):
    """Stores every token on the GPU chunk by chunk, the oracle stores the same
    chunk (the exact bytes the kernel read) into its own pool, and the two
    pools must be equal byte for byte; then the GPU decode of the batch."""
    import torch
    from vm_c_amd import capi
    bt, slots, nblk = _layout(lens, seed)
    cfg = capi.tq_config(D, method)
    L = O.tq_layout(method)
    c, m = O.tq_tables(D, L.key_quant_bits)
    S = cfg.slot_size_aligned
    cache = torch.zeros(nblk * BS * Hkv * S, dtype=torch.uint8, device=dev)
    ref_cache = np.zeros(cache.numel(), np.uint8)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    T = slots.size
    chunk = 65536
    print(f"{method}: B={len(lens)} T={T} store", flush=True)
    for s0 in range(0, T, chunk):
        n = min(chunk, T - s0)
        k = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        v = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        sl = slots[s0:s0 + n]
        capi.turboquant_store(k, v, cache, torch.from_numpy(sl).to(dev), BS, cfg)
        O.tq_store(k.cpu().numpy().view(np.uint16), v.cpu().numpy().view(np.uint16), sl, ref_cache, BS, L, m)
    q = torch.randn((len(lens), Hq, D), generator=gen, device=dev).half()
    out = torch.full_like(q, float("nan"))
    print(f"{method}: decode", flush=True)
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(bt).to(dev),
                                     torch.from_numpy(lens).to(dev), Hkv, 1 / np.sqrt(D), cfg, BS)
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    bad = np.flatnonzero(got_cache != ref_cache)
    assert bad.size == 0, f"store bytes differ at {bad.size} of {got_cache.size} bytes (first {bad[:4]})"
    return out.float().cpu().numpy(), q.cpu().numpy().view(np.uint16), got_cache, bt, L, c


def test_tq4_batch32_ctx8192(dev):
    lens = np.full(32, 8192, np.int32)
    got, qb, cache, bt, L, c = _run(dev, "turboquant_4bit_nc", lens, 32, 8, 2)
    ref = O.f16_to_f32(O.tq_decode(qb, cache, bt, lens, 8, np.float32(1 / np.sqrt(D)), BS, L, c))
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs restatement: max err {err}"
    ex = O.tq_decode_exact(qb, cache, bt, lens, 8, 1 / np.sqrt(D), BS, L, c)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"


def test_tq3_ragged_32k(dev):
    rng = np.random.default_rng(4)
    lens = np.exp(rng.uniform(np.log(1024), np.log(32768), 64)).astype(np.int64)
    lens[0] = 32768
    lens = np.clip(lens, 1024, 32768).astype(np.int32)
    got, qb, cache, bt, L, c = _run(dev, "turboquant_3bit_nc", lens, 64, 8, 4)
    print("turboquant_3bit_nc: oracle decode of all 64 rows", flush=True)
    ref = O.f16_to_f32(O.tq_decode(qb, cache, bt, lens, 8, np.float32(1 / np.sqrt(D)), BS, L, c))
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs restatement: max err {err}"
    ex = O.tq_decode_exact(qb, cache, bt, lens, 8, 1 / np.sqrt(D), BS, L, c)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"


def test_tq3_many_sequence_switches(dev):
    """3-bit slots, 160 sequences whose page ranges cross many sequence
    starts: a tenth empty, a seventh shorter than a page pair, the rest
    log-uniform in [1024, 16384] tokens, four of 32768 (seed 5; ~48k pages,
    so the range split also counts every sequence switch as pages).  Every
    row against the two-stage restatement, the non-empty ones against fp64
    exact attention; empty sequences give zero rows."""
    rng = np.random.default_rng(5)
    B = 160
    lens = np.exp(rng.uniform(np.log(1024), np.log(16384), B)).astype(np.int64)
    kind = rng.random(B)
    lens[kind < 0.1] = 0
    short = (kind >= 0.1) & (kind < 0.25)
    lens[short] = rng.integers(1, 40, int(short.sum()))
    lens[:4] = 32768
    lens = lens.astype(np.int32)
    got, qb, cache, bt, L, c = _run(dev, "turboquant_3bit_nc", lens, 64, 8, 5)
    print(f"turboquant_3bit_nc: {int(((lens + BS - 1) // BS).sum())} pages, oracle decode of {B} rows", flush=True)
    ref = O.f16_to_f32(O.tq_decode(qb, cache, bt, lens, 8, np.float32(1 / np.sqrt(D)), BS, L, c))
    ok, err = close_report(got, ref, ATOL, RTOL)
    assert ok, f"vs restatement: max err {err}"
    assert np.all(got[lens == 0] == 0.0)
    nz = lens > 0
    ex = O.tq_decode_exact(qb[nz], cache, bt[nz], lens[nz], 8, 1 / np.sqrt(D), BS, L, c)
    ok, err = close_report(got[nz], ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"
