"""Benchmark of the attention hot path on one MI355X.

Headline (one JSON line on stdout): the long-context ragged decode step --
batch 64, 64 query heads, 8 KV heads (GQA 8:1), head_dim 128, context lengths
log-uniform in [1024, 32768] (seed 4) with one sequence at 32768, 3-bit
TurboQuant KV (turboquant_3bit_nc, 102-byte slots), block size 16.  A step is
one single-layer decode: quantize-on-append of one new K/V token per sequence
into the paged cache, then split-KV paged decode attention over every
sequence's full context.  Inputs are resident in HBM before timing; the KV
page pool is replicated into >= 2 GiB of distinct copies and the steps rotate
through them so the 256 MB last-level cache cannot serve the pages.

Also measured in the same run (extra fields of the same line):
  * variant_g32: the same decode step with the configuration text's KV
    format, turboquant_3bit_g32 (random-sign Walsh-Hadamard, 3-bit codes and
    a 16-bit scale per 32 values, 112-byte slots);
  * decode_other_configs: the attention operator on batch 32 x 8192 with
    4-bit TurboQuant and with its per-32-group 4-bit variant, and on batch 16 (lengths in [512, 4096]) with q8_0
    K/V pages -> GB/s;
  * decode_other_configs also holds batch 1 x 2048 fp16 pages (the
    configuration the reference's CPU path runs);
  * causal prefill: batch 4 x 4096 tokens, 32/8 heads, bf16, fused q8_0
    quantize-on-append into the paged cache -> TFLOP/s;
  * fused_norm_rope: Q/K RMSNorm + RoPE + q8_0 append of the same prefill
    batch (16384 tokens, 32/8 heads, bf16) in one launch -> GB/s;
  * hbm_ceiling_measured: a 2 GiB copy and a 4 GiB read on the same GPU;
  * cpu_baseline: the CPU restatement of the TurboQuant decode (OpenMP over
    all host cores) on the headline workload (the reference has no CPU
    TurboQuant path), plus reference_ggml_cpu: the reference's own ggml CPU
    flash-attention (built from its sources into oracle/_ref) on the
    fp16 decode, q8_0 decode and bf16 prefill configurations.
Each timed loop records a HIP event per call on the kernels' stream: means
over the timed region (the headline step: exactly --steps calls) and the
median call are reported; the attention operator alone is timed over
max(50, --steps) calls.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
BS = 16
D = 128
HEAD_DIM = D


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ workloads

def decode_workload():
    rng = np.random.default_rng(4)
    B, Hq, Hkv = 64, 64, 8
    lens = np.exp(rng.uniform(np.log(1024), np.log(32768), B)).astype(np.int64)
    lens[0] = 32768
    lens = np.clip(lens, 1024, 32768).astype(np.int32)
    pages = (lens + BS - 1) // BS
    nblk = int(pages.sum())
    perm = rng.permutation(nblk).astype(np.int32)
    max_blocks = int(pages.max())
    bt = np.full((B, max_blocks), -1, np.int32)
    k = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[k:k + pages[b]]
        k += pages[b]
    return dict(B=B, Hq=Hq, Hkv=Hkv, lens=lens, bt=bt, nblk=nblk, max_blocks=max_blocks)


def time_loop(torch, fn, n, warm, stream):
    """Untimed warm-up (at least `warm` calls and at least 0.3 s, so the
    clocks have settled under the load), then `n` back-to-back timed calls
    between two HIP events on `stream` (the stream the kernels run on): the
    mean ms per call, the whole-job rate; then `n` more calls with an event
    after each, for the median ms of one call.  Returns (mean, median)."""
    import time
    t_end = time.perf_counter() + 0.3
    i = 0
    while i < warm or (time.perf_counter() < t_end and i < 4000):
        fn(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        fn(warm + i)
    e1.record(stream)
    e1.synchronize()
    mean = e0.elapsed_time(e1) / n
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    ev[0].record(stream)
    for i in range(n):
        fn(warm + n + i)
        ev[i + 1].record(stream)
    ev[n].synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]
    return mean, float(np.median(per))


def slots_for(bt, lens, positions_of):
    """slot of (sequence b, position p) = bt[b, p // 16] * 16 + p % 16."""
    b_idx, p_idx = positions_of
    return bt[b_idx, p_idx // BS].astype(np.int64) * BS + p_idx % BS


# ------------------------------------------------------------------ decode

def bench_decode(args, torch, capi, dev, method="turboquant_3bit_nc", sign_seed=0):
    w = decode_workload()
    B, Hq, Hkv, lens, bt = w["B"], w["Hq"], w["Hkv"], w["lens"], w["bt"]
    cfg = capi.tq_config(D, method, sign_seed=sign_seed)
    slot_bytes = cfg.slot_size_aligned
    pool_bytes = w["nblk"] * BS * Hkv * slot_bytes
    npool = max(2, math.ceil(2 * 1024 ** 3 / pool_bytes))
    log(f"decode {method}: B={B} Hq={Hq} Hkv={Hkv} sum(L)={int(lens.sum())} max(L)={int(lens.max())} "
        f"pool={pool_bytes / 1e6:.1f} MB x {npool} copies")
    pools = [torch.empty(pool_bytes, dtype=torch.uint8, device=dev) for _ in range(npool)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    # fill pool 0 with every token's K/V (N(0,1) fp16) through the store kernel
    b_all = np.repeat(np.arange(B), lens)
    p_all = np.concatenate([np.arange(n) for n in lens])
    slots_all = slots_for(bt, lens, (b_all, p_all))
    chunk = 65536
    for s in range(0, slots_all.size, chunk):
        n = min(chunk, slots_all.size - s)
        kk = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).half()
        vv = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).half()
        capi.turboquant_store(kk, vv, pools[0], torch.from_numpy(slots_all[s:s + n]).to(dev), BS, cfg)
    for i in range(1, npool):
        pools[i].copy_(pools[0])
    torch.cuda.synchronize()
    # per-step inputs: the new token of every sequence (position L-1) and q
    new_slots = torch.from_numpy(slots_for(bt, lens, (np.arange(B), lens - 1))).to(dev)
    k_new = torch.randn((B, Hkv, D), generator=gen, device=dev).half()
    v_new = torch.randn((B, Hkv, D), generator=gen, device=dev).half()
    q = torch.randn((B, Hq, D), generator=gen, device=dev).half()
    out = torch.empty_like(q)
    bt_d = torch.from_numpy(bt).to(dev)
    lens_d = torch.from_numpy(lens).to(dev)
    ws = torch.empty(capi.turboquant_decode_workspace_size(B, Hq, Hkv, D, bt.shape[1], BS),
                     dtype=torch.uint8, device=dev)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream()

    def step(i):
        pool = pools[i % npool]
        capi.turboquant_store(k_new, v_new, pool, new_slots, BS, cfg, stream=stream)
        capi.turboquant_decode_attention(out, q, pool, bt_d, lens_d, Hkv, scale, cfg, BS,
                                         workspace=ws, stream=stream)

    def attn_only(i):
        capi.turboquant_decode_attention(out, q, pools[i % npool], bt_d, lens_d, Hkv, scale, cfg,
                                         BS, workspace=ws, stream=stream)

    ms_step, med_step = time_loop(torch, step, args.steps, args.warmup, stream)
    n_attn = max(50, args.steps)
    ms_attn, med_attn = time_loop(torch, attn_only, n_attn, args.warmup, stream)
    assert torch.isfinite(out.float()).all().item(), "decode produced non-finite values"

    sum_l = int(lens.sum())
    kv_bytes = sum_l * Hkv * slot_bytes
    qo_bytes = 2 * B * Hq * D * 2
    table_bytes = int(((lens + BS - 1) // BS).sum()) * 4 + B * 4
    attn_bytes = kv_bytes + qo_bytes + table_bytes
    append_bytes = B * Hkv * (2 * D * 2 + slot_bytes) + B * 8
    step_bytes = attn_bytes + append_bytes
    res = dict(w=w, ms_step=ms_step, ms_attn=ms_attn, med_step=med_step, med_attn=med_attn, n_attn=n_attn,
               attn_bytes=attn_bytes, step_bytes=step_bytes, kv_bytes=kv_bytes, sum_l=sum_l, q=q,
               pools=pools, bt=bt, lens=lens, cfg=cfg)
    log(f"decode step {ms_step * 1e3:.1f} us, attention {ms_attn * 1e3:.1f} us, "
        f"{attn_bytes / ms_attn / 1e6:.0f} GB/s attention-only")
    return res


DECODE_CFGS = {
    # kind: (seed, batch, Hq, Hkv, lengths, KV format)
    "f16_single2048": (0, 1, 32, 8, "2048", "fp16"),
    "tq4_32x8192": (2, 32, 32, 8, "8192", "turboquant_4bit_nc"),
    "g32_4bit_32x8192": (2, 32, 32, 8, "8192", "turboquant_4bit_g32"),
    "q8_0_batch16": (1, 16, 32, 8, "u512_4096", "q8_0"),
    # (head_dim 256: the 16 / 2-head, 262-byte-slot deployment shape)
    "tq4_d256_32x32768": (3, 32, 16, 2, "32768", "turboquant_4bit_nc", 256),
}


def bench_decode_cfg(args, torch, capi, dev, kind):
    """The other decode configurations, attention operator only:
    "f16_single2048": batch 1, 2048 tokens, 32/8 heads, fp16 K/V pages, block
    table a permutation of 128 pages (seed 0) -- 8.4 MB, launch-bound;
    "tq4_32x8192": batch 32 x 8192 tokens, 32/8 heads, turboquant_4bit_nc
    (134 B slots), seed 2; "g32_4bit_32x8192": the same batch with the
    configuration text's 4-bit per-32-group variant (160 B slots, signs
    seed 2); "q8_0_batch16": batch 16, lengths uniform in [512, 4096]
    (seed 1), 32/8 heads, q8_0 K and V pages (136 B per token-head each);
    "tq4_d256_32x32768": batch 32 x 32768 tokens, head_dim 256, 16/2 heads,
    turboquant_4bit_nc (262 B slots), seed 3.  Pools replicated to >= 2 GiB
    and rotated."""
    seed, B, Hq, Hkv, lspec, fmt, *hd = DECODE_CFGS[kind]
    D = hd[0] if hd else HEAD_DIM
    if lspec == "u512_4096":
        lens = np.random.default_rng(seed).integers(512, 4097, B).astype(np.int32)
    else:
        lens = np.full(B, int(lspec), np.int32)
    rng = np.random.default_rng(seed)
    pages = (lens + BS - 1) // BS
    nblk = int(pages.sum())
    perm = rng.permutation(nblk).astype(np.int32)
    bt = np.full((B, int(pages.max())), -1, np.int32)
    k = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[k:k + pages[b]]
        k += pages[b]
    b_all = np.repeat(np.arange(B), lens)
    p_all = np.concatenate([np.arange(n) for n in lens])
    slots = torch.from_numpy(slots_for(bt, lens, (b_all, p_all))).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    tq = fmt.startswith("turboquant")
    if tq:
        cfg = capi.tq_config(D, fmt, sign_seed=2 if fmt.endswith("_g32") else 0)
        entry = cfg.slot_size_aligned
        pool_bytes = nblk * BS * Hkv * entry
    else:
        kvf = capi.KV_FORMATS[fmt]
        entry = capi.kv_entry_bytes(kvf, D)
        pool_bytes = 2 * nblk * BS * Hkv * entry
    npool = max(2, math.ceil(2 * 1024 ** 3 / pool_bytes))
    pools = [torch.empty(pool_bytes, dtype=torch.uint8, device=dev) for _ in range(npool)]
    T = int(lens.sum())
    half = pool_bytes // 2
    for s0 in range(0, T, 65536):
        n = min(65536, T - s0)
        kk = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        vv = torch.randn((n, Hkv, D), generator=gen, device=dev).half()
        if tq:
            capi.turboquant_store(kk, vv, pools[0], slots[s0:s0 + n], BS, cfg)
        else:
            capi.reshape_and_cache(kk, vv, pools[0][:half], pools[0][half:], slots[s0:s0 + n], BS,
                                   kv_format=kvf)
    for i in range(1, npool):
        pools[i].copy_(pools[0])
    q = torch.randn((B, Hq, D), generator=gen, device=dev).half()
    out = torch.empty_like(q)
    bt_d, lens_d = torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream()
    if tq:
        ws = torch.empty(capi.turboquant_decode_workspace_size(B, Hq, Hkv, D, bt.shape[1], BS),
                         dtype=torch.uint8, device=dev)
    else:
        ws = torch.empty(max(1, capi.paged_decode_workspace_size(B, Hq, Hkv, D, bt.shape[1], BS)),
                         dtype=torch.uint8, device=dev)

    def run(i):
        pool = pools[i % npool]
        if tq:
            capi.turboquant_decode_attention(out, q, pool, bt_d, lens_d, Hkv, scale, cfg, BS,
                                             workspace=ws, stream=stream)
        else:
            capi.paged_attention_decode(out, q, pool[:half], pool[half:], bt_d, lens_d, Hkv, scale,
                                        block_size=BS, kv_format=kvf, workspace=ws, stream=stream)

    ms, med = time_loop(torch, run, max(50, args.steps), args.warmup, stream)
    assert torch.isfinite(out.float()).all().item(), f"{kind} decode produced non-finite values"
    kv = T * Hkv * entry * (1 if tq else 2)
    nbytes = kv + 2 * B * Hq * D * 2 + nblk * 4 + B * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"decode {kind}: {ms * 1e3:.1f} us (median {med * 1e3:.1f}), {gbs:.0f} GB/s")
    del pools
    torch.cuda.empty_cache()
    return {"workload": kind, "kv": fmt, "batch": B, "num_heads": Hq, "num_kv_heads": Hkv, "head_dim": D,
            "sum_ctx": T, "ms": round(ms, 4), "ms_median": round(med, 4), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes,
            "tokens_per_s": round(B / (ms * 1e-3), 1)}


# ------------------------------------------------------------------ prefill

def bench_prefill(args, torch, capi, dev):
    """Causal prefill of 4 x 4096 tokens, 32/8 heads, bf16, the q8_0 pages
    written in the same launch (vmc_flash_attention_prefill_ws: the V^T
    tiles built by a first launch into a workspace, both launches timed).  Sets of q/k/v/out/pages (370 MB each) are
    replicated past 1 GiB and rotated, so the 256 MB last-level cache holds
    no set from one call to the next."""
    B, S, Hq, Hkv = 4, 4096, 32, 8
    T = B * S
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    E = capi.kv_entry_bytes(capi.KV_Q8_0, D)
    nblk = T // BS
    set_bytes = T * (2 * Hq + 2 * Hkv) * D * 2 + 2 * nblk * BS * Hkv * E
    nset = max(2, math.ceil(1024 ** 3 / set_bytes))
    sets = []
    for _ in range(nset):
        q = torch.randn((T, Hq, D), generator=gen, device=dev).bfloat16()
        k = torch.randn((T, Hkv, D), generator=gen, device=dev).bfloat16()
        v = torch.randn((T, Hkv, D), generator=gen, device=dev).bfloat16()
        kc = torch.empty(nblk * BS * Hkv * E, dtype=torch.uint8, device=dev)
        sets.append((q, k, v, torch.empty_like(q), kc, torch.empty_like(kc)))
    pos = torch.arange(S, dtype=torch.int32, device=dev).repeat(B)
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).to(dev)
    t = torch.arange(T, device=dev)
    slots = (perm[t // BS] * BS + t % BS).to(torch.int64)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream()
    # the call's V^T tiles (vmc_flash_attention_prefill_ws), allocated once
    ws = torch.empty(capi.flash_attention_prefill_workspace_size(T, Hkv, D), dtype=torch.uint8, device=dev)

    def run(i):
        q, k, v, out, kc, vc = sets[i % nset]
        capi.flash_attention_prefill(out, q, k, v, pos, Hkv, scale, key_cache=kc, value_cache=vc,
                                     slot_mapping=slots, block_size=BS, kv_format=capi.KV_Q8_0,
                                     stream=stream, workspace=ws)

    n = max(20, args.steps)
    ms, med = time_loop(torch, run, n, max(2, args.warmup // 2), stream)
    flops = 4.0 * B * Hq * D * S * (S + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    assert all(torch.isfinite(st[3].float()).all().item() for st in sets), "prefill produced non-finite values"
    log(f"prefill {ms * 1e3:.1f} us (median {med * 1e3:.1f}), {tflops:.1f} TFLOP/s, {nset} rotated sets")
    del sets
    torch.cuda.empty_cache()
    return dict(ms=ms, med=med, tflops=tflops, flops=flops, n=n)


def bench_paged_prefill(args, torch, capi, dev):
    """Chunked prefill over the paged cache: a 2048-token chunk of one
    sequence over a 30720-token cached prefix, 32/8 heads, fp16 q, q8_0
    pages (vmc_flash_attention_prefill_v2).  Four sets of pages + q + out
    (~105 MB each) rotate past the last-level cache.  The per-token path
    (vmc_paged_attention_prefill: one decode row per token) is timed on the
    same input for comparison."""
    prefix, new, Hq, Hkv = 30720, 2048, 32, 8
    L = prefix + new
    E = capi.kv_entry_bytes(capi.KV_Q8_0, D)
    nblk = L // BS
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    nset = 4
    sets = []
    for _ in range(nset):
        kc = torch.randint(-127, 128, (nblk * BS * Hkv * E,), generator=gen, device=dev,
                           dtype=torch.int8).view(torch.uint8)
        vc = torch.randint(-127, 128, (nblk * BS * Hkv * E,), generator=gen, device=dev,
                           dtype=torch.int8).view(torch.uint8)
        # every 34-byte block's fp16 scale := 1/64 (0x2400), so values are moderate
        for c in (kc, vc):
            c.view(-1, 34)[:, 0] = 0x00
            c.view(-1, 34)[:, 1] = 0x24
        q = torch.randn((new, Hq, D), generator=gen, device=dev).half()
        sets.append((q, torch.empty_like(q), kc, vc))
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(9)).to(torch.int32)
    bt = perm.view(1, -1).to(dev)
    tok_seq = torch.zeros(new, dtype=torch.int32, device=dev)
    tok_pos = torch.arange(prefix, L, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream()

    def run(i):
        q, out, kc, vc = sets[i % nset]
        capi.flash_attention_prefill_v2(out, q, kc, vc, bt, tok_seq, tok_pos, Hkv, scale, block_size=BS,
                                        kv_format=capi.KV_Q8_0, stream=stream)

    n = max(20, args.steps)
    ms, med = time_loop(torch, run, n, max(2, args.warmup // 2), stream)
    flops = 4.0 * Hq * D * (new * prefix + new * (new + 1) / 2)
    tflops = flops / (ms * 1e-3) / 1e12
    assert all(torch.isfinite(st[1].float()).all().item() for st in sets), "paged prefill produced non-finite values"
    ws = torch.empty(capi.paged_decode_workspace_size(new, Hq, Hkv, D, nblk, BS, 8), dtype=torch.uint8,
                     device=dev)

    def rows(i):
        q, out, kc, vc = sets[i % nset]
        capi.paged_attention_prefill(out, q, kc, vc, bt, tok_seq, tok_pos, Hkv, scale, block_size=BS,
                                     kv_format=capi.KV_Q8_0, workspace=ws, max_splits=8, stream=stream)

    ms_rows, _ = time_loop(torch, rows, 3, 1, stream)
    log(f"paged prefill {ms * 1e3:.1f} us (median {med * 1e3:.1f}), {tflops:.1f} TFLOP/s; "
        f"per-token path {ms_rows * 1e3:.1f} us")
    del sets
    torch.cuda.empty_cache()

    # the same chunk over 3-bit TurboQuant slots (vmc_turboquant_prefill_attention),
    # the pages stored from random K/V by the TurboQuant store
    cfg = capi.tq_config(D, "turboquant_3bit_nc")
    pos = torch.arange(L, device=dev)
    slots = (bt.view(-1).long()[pos // BS] * BS + pos % BS).contiguous()
    tq_sets = []
    for _ in range(nset):
        cache = torch.zeros(nblk * BS * Hkv * cfg.slot_size_aligned, dtype=torch.uint8, device=dev)
        k = torch.randn((L, Hkv, D), generator=gen, device=dev).half()
        v = torch.randn((L, Hkv, D), generator=gen, device=dev).half()
        capi.turboquant_store(k, v, cache, slots, BS, cfg)
        del k, v
        q = torch.randn((new, Hq, D), generator=gen, device=dev).half()
        tq_sets.append((q, torch.empty_like(q), cache))

    def run_tq(i):
        q, out, cache = tq_sets[i % nset]
        capi.turboquant_prefill_attention(out, q, cache, bt, tok_seq, tok_pos, Hkv, scale, cfg, block_size=BS,
                                          stream=stream)

    ms_tq, med_tq = time_loop(torch, run_tq, n, max(2, args.warmup // 2), stream)
    assert all(torch.isfinite(st[1].float()).all().item() for st in tq_sets), \
        "TurboQuant prefill produced non-finite values"
    tflops_tq = flops / (ms_tq * 1e-3) / 1e12
    log(f"TurboQuant 3-bit chunked prefill {ms_tq * 1e3:.1f} us (median {med_tq * 1e3:.1f}), "
        f"{tflops_tq:.1f} TFLOP/s")
    del tq_sets
    torch.cuda.empty_cache()
    return dict(ms=ms, med=med, tflops=tflops, flops=flops, n=n, ms_rows=ms_rows, tq3_ms=ms_tq, tq3_med=med_tq,
                tq3_tflops=tflops_tq)


# ------------------------------------------------------------------ fused norm + RoPE + append

def bench_fused_norm_rope(args, torch, capi, dev):
    """One launch over the prefill batch: q/k RMSNorm + neox RoPE in place,
    K (rotated) and V appended as q8_0 pages.  Algorithmic bytes: q and k read
    and written, v read, the page entries written, slots and positions read,
    the distinct cos/sin rows and the norm weights read once.  Sets of
    q/k/v/pages (~270 MB each) are replicated past 1 GiB and rotated."""
    B, S, Hq, Hkv = 4, 4096, 32, 8
    T = B * S
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    E = capi.kv_entry_bytes(capi.KV_Q8_0, D)
    nblk = T // BS
    set_bytes = T * (Hq + 2 * Hkv) * D * 2 + 2 * nblk * BS * Hkv * E
    nset = max(2, math.ceil(1024 ** 3 / set_bytes))
    sets = []
    for _ in range(nset):
        q = torch.randn((T, Hq, D), generator=gen, device=dev).bfloat16()
        k = torch.randn((T, Hkv, D), generator=gen, device=dev).bfloat16()
        v = torch.randn((T, Hkv, D), generator=gen, device=dev).bfloat16()
        kc = torch.empty(nblk * BS * Hkv * E, dtype=torch.uint8, device=dev)
        sets.append((q, k, v, kc, torch.empty_like(kc)))
    qw = (1.0 + 0.1 * torch.randn(Hq * D, generator=gen, device=dev)).bfloat16()
    kw = (1.0 + 0.1 * torch.randn(Hkv * D, generator=gen, device=dev)).bfloat16()
    theta = 10000.0 ** (-torch.arange(D // 2, device=dev, dtype=torch.float64) * 2.0 / D)
    ang = torch.arange(S, device=dev, dtype=torch.float64)[:, None] * theta[None, :]
    cs = torch.cat([ang.cos(), ang.sin()], dim=1).bfloat16().contiguous()
    pos = torch.arange(S, dtype=torch.int64, device=dev).repeat(B)
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(5)).to(dev)
    t = torch.arange(T, device=dev)
    slots = (perm[t // BS] * BS + t % BS).to(torch.int64)
    stream = torch.cuda.current_stream()

    def run(i):
        q, k, v, kc, vc = sets[i % nset]
        capi.fused_qk_norm_rope_store(q, k, v, qw, kw, cs, pos, kc, vc, slots, BS, eps=1e-6,
                                      is_neox=True, kv_format=capi.KV_Q8_0, stream=stream)

    n = max(20, args.steps)
    ms, med = time_loop(torch, run, n, max(2, args.warmup // 2), stream)
    per_token = 2 * 2 * (Hq + Hkv) * D + 2 * Hkv * D + 2 * Hkv * E + 16
    nbytes = T * per_token + S * D * 2 + (Hq + Hkv) * D * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    assert all(torch.isfinite(st[0].float()).all().item() for st in sets), "fused norm/RoPE produced non-finite values"
    log(f"fused norm+rope+append {ms * 1e3:.1f} us (median {med * 1e3:.1f}), {gbs:.0f} GB/s, {nset} rotated sets")
    del sets
    torch.cuda.empty_cache()
    return dict(ms=ms, med=med, gbs=gbs, bytes=nbytes)


def bench_hbm_ceiling(torch, capi, dev):
    """Measured HBM ceilings next to the 8 TB/s datasheet figure, median of 10
    each: a 2 GiB device-to-device copy (read + write bytes / time) and two
    4 GiB streaming reads (vmc_hbm_read_probe: 16-byte non-temporal loads into
    registers, and the decode's 16-byte non-temporal load-to-LDS transfers)."""
    stream = torch.cuda.current_stream()
    n = 2 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    _, med_copy = time_loop(torch, lambda i: dst.copy_(src), 10, 3, stream)
    del src, dst
    nr = 4 << 30
    x = torch.ones(nr, dtype=torch.uint8, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    meds = []
    for mode in (0, 1, 2):
        _, med = time_loop(torch, lambda i: capi.hbm_read_probe(x, mode, sink, stream), 10, 3, stream)
        meds.append(med)
    del x, sink
    torch.cuda.empty_cache()
    res = {"copy_gbs": round(2 * n / (med_copy * 1e-3) / 1e9, 1),
           "read_gbs": round(nr / (meds[0] * 1e-3) / 1e9, 1),
           "read_lds_dma_nt_gbs": round(nr / (meds[1] * 1e-3) / 1e9, 1),
           "read_lds_dma_gbs": round(nr / (meds[2] * 1e-3) / 1e9, 1),
           "method": "2 GiB torch copy_ (read+write); 4 GiB vmc_hbm_read_probe reads: mode 0 nt loads to "
                     "registers, mode 1 nt load-to-LDS, mode 2 load-to-LDS (the decode's transfers); "
                     "medians of 10"}
    log(f"HBM ceiling: copy {res['copy_gbs']} GB/s, read {res['read_gbs']} GB/s, load-to-LDS read "
        f"{res['read_lds_dma_gbs']} GB/s (nt {res['read_lds_dma_nt_gbs']})")
    return res


# ------------------------------------------------------------------ CPU baseline

def cpu_host_info(nthreads):
    """CPU model, SIMD extensions and the thread count the CPU legs use."""
    model, flags = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    simd = [f for f in ("sse4_2", "avx", "avx2", "fma", "f16c", "avx512f", "avx512_bf16", "amx_tile")
            if f in flags]
    return {"cpu_model": model, "simd": simd, "threads": nthreads, "logical_cpus": os.cpu_count()}


def cpu_baseline(dec, torch, nthreads):
    """The reference has no CPU path for TurboQuant (its ggml CPU op aborts),
    so the headline baseline is the CPU restatement of its two-stage decode
    (oracle, OpenMP over the host cores) on the same pages: the whole
    64-sequence batch, repeated until about 10 s of wall time."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    lens, bt = dec["lens"], dec["bt"]
    cache = dec["pools"][0].cpu().numpy()
    qb = dec["q"].cpu().numpy().view(np.uint16)
    L = O.tq_layout("turboquant_3bit_nc")
    c, _ = O.tq_tables(D, 3)
    reps, t0 = 0, time.time()
    while True:
        O.tq_decode(qb, cache, bt, lens, dec["w"]["Hkv"], np.float32(1 / math.sqrt(D)), BS, L, c,
                    num_splits=32, nthreads=nthreads)
        reps += 1
        if time.time() - t0 >= 10.0 or reps >= 16:
            break
    dt = (time.time() - t0) / reps
    return dict(value=round(dec["attn_bytes"] / dt / 1e9, 3), unit="GB/s", cores=nthreads, kind="port",
                tokens_per_s=round(len(lens) / dt, 1),
                sample=f"the full 64-sequence batch ({dec['sum_l']} tokens), {reps} passes, "
                       f"{dt:.2f} s each; two-stage TurboQuant decode restated in C (no CPU path "
                       f"exists in the reference for this format)")


def cpu_reference_ggml(nthreads):
    """The reference's own CPU path: ggml_flash_attn_ext of its vendored ggml
    (ggml-cpu/ops.cpp:8214-8957), compiled from its sources with vm_c's CPU
    flags into oracle/_ref, on the configurations it can run -- 1 (fp16
    decode, batch 1 x 2048), 2 (q8_0 decode, batch 16, lengths U[512, 4096],
    K/V rows from ggml's own q8_0 encoder) and 4 (bf16 causal prefill, a
    sample: the last 512 query rows of one 4096-token sequence, all 32
    heads).  K/V are contiguous per sequence (the CPU operator's input; the
    block-table gather is not timed); the timed region is ggml_graph_compute
    only, repeated to ~2-4 s per configuration.  Bytes and FLOPs are the
    GPU's algorithmic counts for the same work.  None without oracle/_ref."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    import kvgen
    if not O.ref_available():
        return None
    res = []
    scale = np.float32(1 / math.sqrt(D))

    def rows(fmt, x):  # [Hkv][n][D] fp32 values -> the reference's row encoding
        H, n, _ = x.shape
        if fmt == O.KV_F16:
            return x.astype(np.float16).view(np.uint8).reshape(H, n, 2 * D)
        if fmt == O.KV_BF16:
            return kvgen.f32_to_bf16_bits(x).view(np.uint8).reshape(H, n, 2 * D)
        return O.ref_quantize(fmt, np.ascontiguousarray(x).reshape(-1)).reshape(H, n, O.entry_bytes(fmt, D))

    def timed(q, K, V, fmt, n, Hkv, causal=False, budget=2.0):
        _, t1 = O.ref_flash_attn_timed(q, K, V, fmt, n, Hkv, scale, causal, nthreads, 1)
        reps = max(1, min(200, int(budget / max(t1, 1e-6))))
        _, t = O.ref_flash_attn_timed(q, K, V, fmt, n, Hkv, scale, causal, nthreads, reps)
        return t, reps

    # configuration 1
    w = kvgen.single_seq_fp16_workload()
    K = rows(O.KV_F16, np.ascontiguousarray(w.K.astype(np.float32).transpose(1, 0, 2)))
    V = rows(O.KV_F16, np.ascontiguousarray(w.V.astype(np.float32).transpose(1, 0, 2)))
    t, reps = timed(w.Q[0].astype(np.float32)[:, None, :], K, V, O.KV_F16, 2048, 8)
    nbytes = 8405508
    res.append({"config": 1, "workload": "fp16 decode, batch 1 x 2048 tokens, 32/8 heads", "kind": "reference",
                "ms": round(t * 1e3, 4), "gbs": round(nbytes / t / 1e9, 3), "tokens_per_s": round(1 / t, 1),
                "sample": f"whole workload, {reps} computes"})
    # configuration 2
    w = kvgen.batched_q8_0_workload()
    starts = np.concatenate([[0], np.cumsum(w.seq_lens)])
    tot, reps_min = 0.0, 10 ** 9
    for b in range(w.B):
        n = int(w.seq_lens[b])
        K = rows(O.KV_Q8_0, np.ascontiguousarray(w.K[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2)))
        V = rows(O.KV_Q8_0, np.ascontiguousarray(w.V[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2)))
        t, reps = timed(w.Q[b].astype(np.float32)[:, None, :], K, V, O.KV_Q8_0, n, 8, budget=0.2)
        tot += t
        reps_min = min(reps_min, reps)
    sum_l = int(w.seq_lens.sum())
    nbytes = sum_l * 2176 + 2 * w.B * 32 * D * 2 + int(((w.seq_lens + 15) // 16).sum()) * 4 + w.B * 4
    res.append({"config": 2, "workload": "q8_0 decode, batch 16, lengths U[512, 4096] seed 1, 32/8 heads",
                "kind": "reference", "ms": round(tot * 1e3, 4), "gbs": round(nbytes / tot / 1e9, 3),
                "tokens_per_s": round(w.B / tot, 1),
                "sample": f"whole batch (sum of the 16 sequences' compute times, >= {reps_min} computes each)"})
    # configuration 4 (sample)
    qb, kb, vb, _, _ = kvgen.prefill_inputs([4096], 32, 8, seed=3)
    n_q, n_kv = 512, 4096
    q = np.ascontiguousarray(O.bf16_to_f32(qb[n_kv - n_q:]).transpose(1, 0, 2))
    K = np.ascontiguousarray(kb.reshape(n_kv, 8, D).transpose(1, 0, 2)).view(np.uint8).reshape(8, n_kv, 2 * D)
    V = np.ascontiguousarray(vb.reshape(n_kv, 8, D).transpose(1, 0, 2)).view(np.uint8).reshape(8, n_kv, 2 * D)
    t, reps = timed(q, K, V, O.KV_BF16, n_kv, 8, causal=True, budget=4.0)
    keys = sum(n_kv - n_q + i + 1 for i in range(n_q))
    flops = 4.0 * 32 * D * keys
    res.append({"config": 4, "workload": "bf16 causal prefill, 32/8 heads", "kind": "reference",
                "ms": round(t * 1e3, 3), "tflops": round(flops / t / 1e12, 5),
                "sample": f"the last {n_q} query rows of one 4096-token sequence ({flops:.3g} FLOP), "
                          f"{reps} computes"})
    for r in res:
        log(f"reference ggml CPU, config {r['config']}: {r['ms']} ms")
    return res


# ------------------------------------------------------------------ traffic

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "tq_decode_tq3_ragged32k_traffic.md")


def measured_traffic():
    """HBM bytes per call of the decode operator, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (scaled by the copy calibration); None if
    that summary is absent."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-variant", action="store_true",
                    help="skip the per-32-group 3-bit variant's decode (turboquant_3bit_g32)")
    ap.add_argument("--only", choices=("decode", "prefill", "paged_prefill", "fused", "configs"),
                    help="profiling runs: only this part (decode: the headline operator; configs: "
                         "the other decode configurations), one JSON line of its numbers")
    ap.add_argument("--config", choices=tuple(DECODE_CFGS),
                    help="with --only configs: just this decode configuration")
    ap.add_argument("--read-calibration", action="store_true",
                    help="only run a 1 GiB load-to-LDS read (vmc_hbm_read_probe mode 2, the decode's "
                         "request type) 5 times (for scaling rocprofv3 FETCH_SIZE)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 5 times (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention hot path is single-device here "
              "(sharding by KV head / sequence is a design note, not a run). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from vm_c_amd import capi
    capi.load()
    dev = torch.device("cuda:0")
    if args.read_calibration:
        n = 1 << 30
        buf = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        torch.cuda.synchronize()
        for _ in range(5):
            capi.hbm_read_probe(buf, 2)
        torch.cuda.synchronize()
        print(json.dumps({"read_calibration_bytes": n, "launches": 5}), flush=True)
        return
    if args.copy_calibration:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return
    if args.only:
        if args.only == "decode":
            r = bench_decode(args, torch, capi, dev)
            r = {"ms_step": r["ms_step"], "ms_attn": r["ms_attn"], "ms_attn_median": r["med_attn"],
                 "attn_bytes": r["attn_bytes"]}
        elif args.only == "prefill":
            r = bench_prefill(args, torch, capi, dev)
        elif args.only == "paged_prefill":
            r = bench_paged_prefill(args, torch, capi, dev)
        elif args.only == "fused":
            r = bench_fused_norm_rope(args, torch, capi, dev)
        else:
            r = {"configs": [bench_decode_cfg(args, torch, capi, dev, k) for k in DECODE_CFGS
                             if args.config in (None, k)]}
        print(json.dumps({"only": args.only, **{k: v for k, v in r.items() if not hasattr(v, "shape")}}),
              flush=True)
        return
    dec = bench_decode(args, torch, capi, dev)
    var = None
    if not args.skip_variant:
        # the configuration text's format: random-sign WHT (seed 4) + 3-bit
        # codes with a scale per 32 values, same workload
        v = bench_decode(args, torch, capi, dev, method="turboquant_3bit_g32", sign_seed=4)
        var = {"kv": "turboquant_3bit_g32 (112 B slot, signs seed 4)",
               "ms_step": round(v["ms_step"], 4), "ms_attn": round(v["ms_attn"], 4),
               "attn_gbs": round(v["attn_bytes"] / (v["ms_attn"] * 1e-3) / 1e9, 1),
               "attn_frac_hbm": round(v["attn_bytes"] / (v["ms_attn"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "attn_bytes": v["attn_bytes"],
               "tokens_per_s": round(v["w"]["B"] / (v["ms_step"] * 1e-3), 1)}
        del v
        torch.cuda.empty_cache()
    kinds = ("f16_single2048",) + (() if args.skip_variant else
                                    ("tq4_32x8192", "g32_4bit_32x8192", "q8_0_batch16", "tq4_d256_32x32768"))
    others = [bench_decode_cfg(args, torch, capi, dev, k) for k in kinds]
    pre = None if args.skip_prefill else bench_prefill(args, torch, capi, dev)
    paged = None if args.skip_prefill else bench_paged_prefill(args, torch, capi, dev)
    fused = None if args.skip_prefill else bench_fused_norm_rope(args, torch, capi, dev)
    ceiling = bench_hbm_ceiling(torch, capi, dev)
    cpu = None
    if not args.no_cpu_baseline:
        nthreads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
        cpu = cpu_baseline(dec, torch, nthreads)
        cpu["host"] = cpu_host_info(nthreads)
        cpu["reference_ggml_cpu"] = cpu_reference_ggml(nthreads)

    ms_step = dec["ms_step"]
    gbs_step = dec["step_bytes"] / (ms_step * 1e-3) / 1e9
    gbs_attn = dec["attn_bytes"] / (dec["ms_attn"] * 1e-3) / 1e9
    line = {
        "metric": "decode attn HBM GB/s (% peak) + tokens/s at 32k ctx; prefill TFLOP/s",
        "value": round(gbs_step, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 codes + fp16",
        "data": "synthetic",
        "config": {"workload": "ragged 32k-context TurboQuant 3-bit paged decode step "
                               "(append 1 token/seq + split-KV attention)",
                   "batch": 64, "num_heads": 64, "num_kv_heads": 8, "head_dim": 128,
                   "block_size": 16, "kv": "turboquant_3bit_nc (102 B slot)",
                   "ctx": "log-uniform [1024, 32768] seed 4, one at 32768",
                   "sum_ctx": dec["sum_l"], "parallelism": "single GPU"},
        "pct_peak_hbm": round(100 * gbs_step / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(dec["w"]["B"] / (ms_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs_attn, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs_attn / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "turboquant_decode_attention: tq_stream_kernel + "
                               "decode_merge_kernel (one operator, two launches)",
                     "ms": round(dec["ms_attn"], 4), "ms_median": round(dec["med_attn"], 4),
                     "launches_timed": dec["n_attn"], "bytes": dec["attn_bytes"],
                     "frac_of_measured_read_ceiling": round(gbs_attn / ceiling["read_gbs"], 4)},
        "ms_per_step_median": round(dec["med_step"], 4),
        "hbm_ceiling_measured": ceiling,
        "cpu_baseline": cpu,
    }
    if var is not None:
        line["variant_g32"] = var
    if others:
        line["decode_other_configs"] = others
    if pre is not None:
        line["prefill"] = {"workload": "causal prefill B=4 S=4096 Hq=32 Hkv=8 bf16, fused q8_0 append "
                                       "(vmc_flash_attention_prefill_ws: vt_prep_kernel + prefill_kernel)",
                           "ms": round(pre["ms"], 4), "ms_median": round(pre["med"], 4),
                           "launches_timed": pre["n"], "tflops": round(pre["tflops"], 1),
                           "pct_peak_mfma_bf16": round(100 * pre["tflops"] / MFMA_BF16_PEAK_TFLOPS, 2)}
    if paged is not None:
        line["paged_prefill"] = {
            "workload": "chunked prefill: 2048-token chunk over a 30720-token cached prefix, Hq=32 Hkv=8, "
                        "fp16 q, q8_0 pages (flash_attention_prefill_v2)",
            "ms": round(paged["ms"], 4), "ms_median": round(paged["med"], 4), "launches_timed": paged["n"],
            "tflops": round(paged["tflops"], 1),
            "pct_peak_mfma_fp16": round(100 * paged["tflops"] / MFMA_BF16_PEAK_TFLOPS, 2),
            "ms_per_token_path": round(paged["ms_rows"], 3),
            "turboquant_3bit": {"ms": round(paged["tq3_ms"], 4), "ms_median": round(paged["tq3_med"], 4),
                                "tflops": round(paged["tq3_tflops"], 1)}}
    if fused is not None:
        line["fused_norm_rope"] = {
            "workload": "q/k RMSNorm + neox RoPE + q8_0 K/V append, 16384 tokens, Hq=32 Hkv=8 bf16",
            "ms": round(fused["ms"], 4), "ms_median": round(fused["med"], 4), "gbs": round(fused["gbs"], 1),
            "frac_hbm": round(fused["gbs"] / HBM_PEAK_GBS, 4), "bytes": fused["bytes"]}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
