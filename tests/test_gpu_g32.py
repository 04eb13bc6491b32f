"""GPU parity of the per-32-group TurboQuant variant ("turboquant_4bit_g32",
"turboquant_3bit_g32": seeded random-sign Walsh-Hadamard, codes with a
16-bit scale (+ minimum) per 32 values; no reference counterpart, the format
is defined in vmc_attn.h and restated by the oracle).

* store: every byte of the pool bit-exact against the oracle's store (fp16
  and bf16 inputs, skipped slots, untouched bytes outside the slots);
* decode: against the oracle's fp64 attention over the same pages, split-KV
  and per-sequence modes, ragged lengths, GQA 2..16;
* the benchmark shapes: batch 32 x 8192 (4-bit, seed 2) and the ragged
  32k batch (3-bit, seed 4): every pool byte bit-exact, every output row.
Tolerance: |got - ref| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, bits16, close_report, make_workload

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
METHODS = {"turboquant_4bit_g32": 4, "turboquant_3bit_g32": 3}


def _store(dev, w, method, seed, bf16=False, poison=0):
    import torch
    from vm_c_amd import capi
    bits = METHODS[method]
    cfg = capi.tq_config(128, method, sign_seed=seed)
    S = cfg.slot_size_aligned
    assert S == 2 * O.g32_part_bytes(bits)
    cache = torch.full((w.num_blocks * BS * w.Hkv * S,), poison, dtype=torch.uint8, device=dev)
    K, V = w.K, w.V
    if bf16:
        import kvgen
        Kb = kvgen.f32_to_bf16_bits(K.astype(np.float32))
        Vb = kvgen.f32_to_bf16_bits(V.astype(np.float32))
        kt = torch.from_numpy(Kb.view(np.int16)).to(dev).view(torch.bfloat16)
        vt = torch.from_numpy(Vb.view(np.int16)).to(dev).view(torch.bfloat16)
        kbits, vbits = Kb, Vb
    else:
        kt, vt = torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev)
        kbits, vbits = bits16(K), bits16(V)
    if K.shape[0]:
        capi.turboquant_store(kt, vt, cache, torch.from_numpy(w.slots).to(dev), BS, cfg)
    torch.cuda.synchronize()
    ref = np.full(cache.numel(), poison, np.uint8)
    if K.shape[0]:
        O.g32_store(kbits, vbits, w.slots, ref, BS, bits, seed, bf16=bf16)
    return cfg, cache, ref


@pytest.mark.parametrize("method", list(METHODS))
@pytest.mark.parametrize("seed", [0, 4])
@pytest.mark.parametrize("bf16", [False, True])
def test_g32_store_bitexact(dev, method, seed, bf16):
    w = make_workload([37, 300, 1, 64], Hq=16, Hkv=4, seed=seed + 3, pool_slack=3)
    w.slots[5] = -1            # skipped token: its slot stays untouched
    _, cache, ref = _store(dev, w, method, seed, bf16=bf16, poison=0xA5)
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
    "cfg3_small": dict(seq_lens=[1024, 1024], Hq=32, Hkv=8),
    "cfg5_small": dict(seq_lens=[1024, 4000, 32], Hq=64, Hkv=8),
    "ragged": dict(seq_lens=[1, 17, 0, 300], Hq=16, Hkv=4),
    "gqa16": dict(seq_lens=[300, 1024, 17, 33], Hq=32, Hkv=2),
    "gqa2": dict(seq_lens=[5, 129, 700], Hq=8, Hkv=4),
    # head shapes of the pipelined kernel (at most 8 query heads per KV head):
    # one query head per KV head, odd group sizes, one and three KV heads
    "mha": dict(seq_lens=[40, 257, 2], Hq=4, Hkv=4),
    "g3": dict(seq_lens=[700, 33], Hq=6, Hkv=2),
    "g5_one_kv_head": dict(seq_lens=[95, 1500, 16], Hq=5, Hkv=1),
    "g7_three_kv_heads": dict(seq_lens=[1, 600, 48, 31], Hq=21, Hkv=3),
}


@pytest.mark.parametrize("method", list(METHODS))
@pytest.mark.parametrize("case", list(CASES))
def test_g32_decode(dev, method, case):
    seed = 2 if METHODS[method] == 4 else 4
    w = make_workload(seed=len(case) * 5, **CASES[case])
    cfg, cache, ref = _store(dev, w, method, seed)
    got = _decode(dev, w, cfg, cache)
    ex = O.g32_decode_exact(bits16(w.Q), cache.cpu().numpy(), w.bt, w.seq_lens, w.Hkv, w.scale, BS,
                            METHODS[method], seed)
    ok, err = close_report(got, ex, ATOL, RTOL)
    assert ok, f"vs exact: max err {err}"


@pytest.mark.parametrize("method", list(METHODS))
def test_g32_decode_split_modes_agree(dev, method):
    """Per-sequence (1 split) and split-KV (up to 32) give the same rows."""
    w = make_workload([3000, 16, 513], Hq=32, Hkv=8, seed=17)
    cfg, cache, _ = _store(dev, w, method, 9)
    a = _decode(dev, w, cfg, cache, max_splits=1)
    b = _decode(dev, w, cfg, cache, max_splits=32)
    ex = O.g32_decode_exact(bits16(w.Q), cache.cpu().numpy(), w.bt, w.seq_lens, w.Hkv, w.scale, BS,
                            METHODS[method], 9)
    for got in (a, b):
        ok, err = close_report(got, ex, ATOL, RTOL)
        assert ok, f"max err {err}"


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


@pytest.mark.parametrize("method,shape", [("turboquant_4bit_g32", "cfg3"), ("turboquant_3bit_g32", "cfg5")])
def test_g32_benchmark_shapes(dev, method, shape):
    import torch
    from vm_c_amd import capi
    bits = METHODS[method]
    if shape == "cfg3":
        seed, Hq, Hkv = 2, 32, 8
        lens = np.full(32, 8192)
    else:
        seed, Hq, Hkv = 4, 64, 8
        rng = np.random.default_rng(seed)
        lens = np.exp(rng.uniform(np.log(1024), np.log(32768), 64)).astype(np.int64)
        lens[0] = 32768
    bt, slots, nblk = _layout(lens, seed)
    cfg = capi.tq_config(128, method, sign_seed=seed)
    S = cfg.slot_size_aligned
    cache = torch.zeros(nblk * BS * Hkv * S, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    T = slots.size
    chunk = 65536
    print(f"{method}: B={len(lens)} T={T} store", flush=True)
    ref = np.zeros(cache.numel(), np.uint8)
    for s0 in range(0, T, chunk):
        n = min(chunk, T - s0)
        k = torch.randn((n, Hkv, 128), generator=gen, device=dev).half()
        v = torch.randn((n, Hkv, 128), generator=gen, device=dev).half()
        sl = torch.from_numpy(slots[s0:s0 + n]).to(dev)
        capi.turboquant_store(k, v, cache, sl, BS, cfg)
        O.g32_store(bits16(k.cpu().numpy()), bits16(v.cpu().numpy()), slots[s0:s0 + n], ref, BS, bits, seed)
    torch.cuda.synchronize()
    # store: every byte of the pool, against the oracle storing the same chunks
    got = cache.cpu().numpy()
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"store differs at {bad.size} of {got.size} bytes"
    # decode of the whole batch, every row
    q = torch.randn((len(lens), Hq, 128), generator=gen, device=dev).half()
    out = torch.full_like(q, float("nan"))
    capi.turboquant_decode_attention(out, q, cache, torch.from_numpy(bt).to(dev),
                                     torch.from_numpy(lens.astype(np.int32)).to(dev), Hkv,
                                     1.0 / np.sqrt(128.0), cfg, block_size=BS)
    torch.cuda.synchronize()
    print(f"{method}: decode checked on all {len(lens)} sequences", flush=True)
    qn = q.cpu().numpy()
    ex = O.g32_decode_exact(bits16(qn), got, bt, lens.astype(np.int32), Hkv, 1.0 / np.sqrt(128.0), BS, bits, seed)
    ok, err = close_report(out.float().cpu().numpy(), ex, ATOL, RTOL)
    assert ok, f"max err {err}"
