"""Synthetic paged-KV workloads shared by the tests (numpy, seeded).

A workload is a batch of sequences with K/V rows N(0,1) rounded to fp16, a
block table that is a seeded permutation of a shared page pool, and the slot
mapping that appends every token (vm_c Engine semantics: slot =
block_id * block_size + pos % block_size, src/core/engine.cpp:701-714).
"""
import numpy as np

BS = 16


class Workload:
    pass


def make_workload(seq_lens, Hq, Hkv, D=128, seed=0, holes=0, pool_slack=0, dtype=np.float16):
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    B = len(seq_lens)
    pages = [(int(L) + BS - 1) // BS for L in seq_lens]
    max_blocks = max(1, max(pages) if pages else 1)
    total_pages = sum(pages) + pool_slack
    perm = rng.permutation(max(total_pages, 1)).astype(np.int32)
    bt = np.full((B, max_blocks), -1, dtype=np.int32)
    k = 0
    for b in range(B):
        for p in range(pages[b]):
            bt[b, p] = perm[k]
            k += 1
    # optional holes: drop some block-table entries (tokens there are skipped)
    hole_list = []
    for _ in range(holes):
        b = int(rng.integers(0, B))
        if pages[b] > 1:
            p = int(rng.integers(0, pages[b] - 1))
            hole_list.append((b, p))
    T = int(seq_lens.sum())
    tok_seq = np.repeat(np.arange(B), seq_lens)
    tok_pos = np.concatenate([np.arange(L) for L in seq_lens]) if T else np.zeros(0, np.int64)
    slots = (bt[tok_seq, tok_pos // BS].astype(np.int64) * BS + tok_pos % BS) if T else np.zeros(0, np.int64)
    K = rng.standard_normal((T, Hkv, D)).astype(dtype)
    V = rng.standard_normal((T, Hkv, D)).astype(dtype)
    Q = rng.standard_normal((B, Hq, D)).astype(dtype)
    for (b, p) in hole_list:
        bt[b, p] = -1
    w = Workload()
    w.B, w.Hq, w.Hkv, w.D = B, Hq, Hkv, D
    w.seq_lens, w.bt, w.slots, w.K, w.V, w.Q = seq_lens, bt, slots, K, V, Q
    w.num_blocks = max(total_pages, 1)
    w.max_blocks = max_blocks
    w.scale = 1.0 / np.sqrt(D)
    return w


def f32_to_bf16_bits(x):
    """float32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bits16(a):
    return np.ascontiguousarray(a).view(np.uint16)


def close_report(got, ref, atol=2e-3, rtol=1e-2):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    return bool(ok.all()), float(err.max()) if err.size else 0.0


# ------------------------------------------------------------ named workloads
# The decode / prefill shapes the benchmarks and golden fixtures are quoted on.

def single_seq_fp16_workload():
    """Batch 1, 32/8 heads, 2048-token context, fp16 KV, block table a seeded
    permutation of 128 pages, seed 0."""
    return make_workload([2048], Hq=32, Hkv=8, seed=0)


def batched_q8_0_lens():
    """16 context lengths uniform in [512, 4096], seed 1."""
    return np.random.default_rng(1).integers(512, 4097, 16).astype(np.int32)


def batched_q8_0_workload():
    """Batch 16, 32/8 heads, lengths from batched_q8_0_lens(), seed 1."""
    return make_workload(batched_q8_0_lens(), Hq=32, Hkv=8, seed=1)


def prefill_inputs(seq_lens, Hq, Hkv, D=128, seed=0, bf16=True):
    """Q [T][Hq][D], K/V [T][Hkv][D] as bf16 (or fp16) bits, N(0,1) from
    `seed`; positions restart at 0 per sequence; cu_seqlens [B+1]."""
    rng = np.random.default_rng(seed)
    T = int(sum(seq_lens))
    mk = lambda *s: rng.standard_normal(s).astype(np.float32)
    q, k, v = mk(T, Hq, D), mk(T, Hkv, D), mk(T, Hkv, D)
    if bf16:
        qb, kb, vb = (f32_to_bf16_bits(x) for x in (q, k, v))
    else:
        qb, kb, vb = (x.astype(np.float16).view(np.uint16) for x in (q, k, v))
    pos = np.concatenate([np.arange(n) for n in seq_lens]).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(seq_lens)]).astype(np.int32)
    return qb, kb, vb, pos, cu


def crc(a):
    """crc32 of an array's bytes (fixtures record it for their inputs)."""
    import zlib
    return zlib.crc32(np.ascontiguousarray(a).tobytes()) & 0xFFFFFFFF
