"""TurboQuant store + decode parity at the full benchmark shapes.

  * 4-bit (turboquant_4bit_nc), batch 32, 32/8 heads, 8192 tokens each,
    K/V N(0,1) fp16 (seed 2): every slot byte of the pool bit-exact against
    the oracle's store, every output row against the oracle's two-stage
    decode and fp64 exact attention over the same pages.
  * 3-bit (turboquant_3bit_nc), batch 64, 64/8 heads, lengths log-uniform
    in [1024, 32768] (seed 4) with one at 32768: store bit-exact on a 64k
    token chunk, decode of the 32768-token sequence and three others
    against the oracle.
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


def _run(dev, method, lens, Hq, Hkv, seed, check_tokens):
    import torch
    from vm_c_amd import capi
    bt, slots, nblk = _layout(lens, seed)
    cfg = capi.tq_config(D, method)
    L = O.tq_layout(method)
    c, m = O.tq_tables(D, L.key_quant_bits)
    S = cfg.slot_size_aligned
    cache = torch.zeros(nblk * BS * Hkv * S, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    T = slots.size
    chunk = 65536
    kept = None
    print(f"{method}: B={len(lens)} T={T} store", flush=True)
    for s0 in range(0, T, chunk):
        n = min(chunk, T - s0)
        k = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        v = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        sl = slots[s0:s0 + n]
        capi.turboquant_store(k, v, cache, torch.from_numpy(sl).to(dev), BS, cfg)
        if check_tokens is None or s0 == 0:
            torch.cuda.synchronize()
            kk = k.cpu().numpy().view(np.uint16)
            vv = v.cpu().numpy().view(np.uint16)
            if check_tokens is None:
                kept = (kept or []) + [(kk, vv, sl)]
            else:
                kept = [(kk[:check_tokens], vv[:check_tokens], sl[:check_tokens])]
    q = torch.randn((len(lens), Hq, D), generator=gen, device=dev).half()
    out = torch.full_like(q, float("nan"))
    print(f"{method}: decode", flush=True)
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(bt).to(dev),
                                     torch.from_numpy(lens).to(dev), Hkv, 1 / np.sqrt(D), cfg, BS)
    torch.cuda.synchronize()
    got_cache = cache.cpu().numpy()
    # store: bit-exact on the kept tokens; slot s owns bytes [s*Hkv*S, (s+1)*Hkv*S)
    ref_only = np.zeros_like(got_cache)
    for kk, vv, sl in kept:
        O.tq_store(kk, vv, sl, ref_only, BS, L, m)
        rows_got = got_cache.reshape(-1, Hkv * S)[sl]
        rows_ref = ref_only.reshape(-1, Hkv * S)[sl]
        assert np.array_equal(rows_got, rows_ref), "store bytes differ"
    return out.float().cpu().numpy(), q.cpu().numpy().view(np.uint16), got_cache, bt, L, c


def test_tq4_batch32_ctx8192(dev):
    lens = np.full(32, 8192, np.int32)
    got, qb, cache, bt, L, c = _run(dev, "turboquant_4bit_nc", lens, 32, 8, 2, None)
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
    got, qb, cache, bt, L, c = _run(dev, "turboquant_3bit_nc", lens, 64, 8, 4, 65536)
    pick = np.array([0, 1, 17, 63])
    ref = O.f16_to_f32(O.tq_decode(qb[pick], cache, bt[pick], lens[pick], 8,
                                   np.float32(1 / np.sqrt(D)), BS, L, c))
    ok, err = close_report(got[pick], ref, ATOL, RTOL)
    assert ok, f"vs restatement: max err {err}"
    ex = O.tq_decode_exact(qb[pick], cache, bt[pick], lens[pick], 8, 1 / np.sqrt(D), BS, L, c)
    ok, err = close_report(got[pick], ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"
