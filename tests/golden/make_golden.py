"""Writes the golden fixtures in this folder from the reference's own code.

The reference's ggml CPU backend (vendored ggml 0.12.0 + vm_c's op patch,
third_party/vm_c_official/ggml) is compiled from its sources by
`make -C oracle ref` into oracle/_ref/ (never committed, never shipped).  This
script feeds it seeded inputs and stores the inputs' crc32 and the
reference's outputs as small .npz files; the tests regenerate the inputs
from the same seeds (tests/kvgen.py), check the crc32, and compare.

    python tests/golden/make_golden.py      # needs oracle/_ref built

Fixtures
  quant_q8_0.npz, quant_q4_0.npz
      quantize_row_q8_0_ref / quantize_row_q4_0_ref (ggml-quants.c:234-257,
      :71-104) and the CPU from_float trait set_rows uses
      (ggml-cpu/ops.cpp:4950-4998), on edge-case and random rows.
  fa_decode_f16.npz, fa_decode_bf16.npz
      ggml_flash_attn_ext on the CPU backend (ggml-cpu/ops.cpp:8214-8957,
      GGML_PREC_F32): batch 1, 32 query / 8 KV heads, head_dim 128, 2048
      tokens, scale 1/sqrt(128), n_threads 1 and 4 (the f16 path splits the
      context over the threads, ops.cpp:8862-8893).
  fa_decode_q8_0.npz, fa_decode_q4_0.npz
      same operator over q8_0 / q4_0 K/V rows encoded by the reference's own
      quantizer: batch 16, 32/8 heads, lengths uniform in [512, 4096]
      (seed 1); outputs of all 16 sequences.
  fa_prefill_bf16.npz
      causal prefill rows of the bf16 batch-4 x 4096-token workload (32/8
      heads, seed 3): every head of the first and last 4 rows of each
      sequence, rows at 64-key tile and page edges, random (token, head)
      pairs (1,280 rows); each row is the operator on that token's causal
      prefix (the bf16 K/V path evaluates every query row independently,
      ops.cpp:8895-8934 -> one_chunk).
  tq_tables_d128.json
      TurboQuant codebooks of the restated Lloyd-Max solver (not a reference
      run: the reference computes them in its CUDA host code).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
sys.path.insert(0, TESTS)

import oracle_lib as O  # noqa: E402
import kvgen  # noqa: E402

D = 128


def quant_rows(seed=11):
    """Edge cases for the GGUF block encoders, 32 values per block."""
    rng = np.random.default_rng(seed)
    blocks = []
    z = np.zeros(32, np.float32)
    blocks.append(z.copy())                                   # all zero
    b = z.copy(); b[5] = 1.0; blocks.append(b)                # one nonzero
    b = z.copy(); b[3] = -2.0; b[10] = 1.5; blocks.append(b)  # negative signed max
    b = z.copy(); b[0] = -3.0; b[1] = 3.0; blocks.append(b)   # |max| tie, first wins
    b = z.copy(); b[0] = 3.0; b[1] = -3.0; blocks.append(b)
    b = (np.arange(32) - 15.5).astype(np.float32); b[0] = 127.0; blocks.append(b)  # x*id ties
    b = (np.arange(32) - 16).astype(np.float32) * 0.5; b[0] = -8.0; blocks.append(b)
    b = np.full(32, -0.0, np.float32); blocks.append(b)       # negative zeros
    b = np.full(32, 1e-40, np.float32); b[::2] *= -1; blocks.append(b)  # subnormals
    b = rng.uniform(-6e4, 6e4, 32).astype(np.float32); blocks.append(b)  # near fp16 max
    b = np.full(32, 7.0, np.float32); blocks.append(b)        # constant
    for s in (1e-3, 1.0, 37.0):
        for _ in range(8):
            blocks.append((rng.standard_normal(32) * s).astype(np.float32))
    for _ in range(16):
        blocks.append(rng.standard_normal(32).astype(np.float16).astype(np.float32))
    return np.concatenate(blocks)


def gen_quant(fmt, name):
    x = quant_rows()
    ref = O.ref_quantize(fmt, x)
    ff = O.ref_from_float(fmt, x)
    np.savez(os.path.join(HERE, name), x=x, ref=ref, from_float=ff)
    print(f"{name}: {x.size // 32} blocks, from_float == ref: {np.array_equal(ff, ref)}")


def _rows(fmt, x):
    """rows [Hkv][n][D] fp32-valued -> reference row encoding [Hkv][n][row]."""
    H, n, _ = x.shape
    if fmt == O.KV_F16:
        return x.astype(np.float16).view(np.uint8).reshape(H, n, 2 * D)
    if fmt == O.KV_BF16:
        return kvgen.f32_to_bf16_bits(x).view(np.uint8).reshape(H, n, 2 * D)
    E = O.entry_bytes(fmt, D)
    return O.ref_quantize(fmt, x.reshape(-1)).reshape(H, n, E)


def _ref_decode(w, fmt, seqs, n_threads):
    """Reference operator, one sequence at a time, K/V gathered in token order."""
    out = np.zeros((len(seqs), w.Hq, D), np.float32)
    starts = np.concatenate([[0], np.cumsum(w.seq_lens)])
    for i, b in enumerate(seqs):
        n = int(w.seq_lens[b])
        K = w.K[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2)
        V = w.V[starts[b]:starts[b] + n].astype(np.float32).transpose(1, 0, 2)
        q = w.Q[b].astype(np.float32)
        if fmt == O.KV_BF16:
            q = O.bf16_to_f32(kvgen.f32_to_bf16_bits(q))
        out[i] = O.ref_flash_attn(q[:, None, :], _rows(fmt, np.ascontiguousarray(K)),
                                  _rows(fmt, np.ascontiguousarray(V)), fmt, n, w.Hkv,
                                  np.float32(w.scale), n_threads=n_threads)[0]
    return out


def gen_decode_single(fmt, name):
    w = kvgen.single_seq_fp16_workload()
    crcs = dict(crc_k=kvgen.crc(w.K), crc_v=kvgen.crc(w.V), crc_q=kvgen.crc(w.Q))
    if fmt == O.KV_BF16:
        # same N(0,1) draws, rounded to bf16 instead of fp16
        w.K, w.V, w.Q = (O.bf16_to_f32(kvgen.f32_to_bf16_bits(a.astype(np.float32)))
                         for a in (w.K, w.V, w.Q))
    o1 = _ref_decode(w, fmt, [0], 1)
    o4 = _ref_decode(w, fmt, [0], 4)
    np.savez(os.path.join(HERE, name), out_nth1=o1, out_nth4=o4, seq_lens=w.seq_lens, **crcs)
    print(f"{name}: |nth1 - nth4| max {np.abs(o1 - o4).max():.3e}")


def gen_decode_batched(fmt, name, nseq=16):
    w = kvgen.batched_q8_0_workload()
    o = _ref_decode(w, fmt, list(range(nseq)), 8)
    np.savez(os.path.join(HERE, name), out=o, seqs=np.arange(nseq), seq_lens=w.seq_lens,
             crc_k=kvgen.crc(w.K), crc_v=kvgen.crc(w.V), crc_q=kvgen.crc(w.Q))
    print(f"{name}: lens {w.seq_lens[:nseq].tolist()}")


PREFILL = dict(seq_lens=[4096] * 4, Hq=32, Hkv=8, seed=3)


def prefill_rows():
    """(token, head) pairs of the batch-4 x 4096 prefill: every head of the
    first and last 4 rows of each sequence, rows on both sides of 64-key tile
    edges and page edges (4 heads each), and 64 random pairs."""
    rng = np.random.default_rng(5)
    S, Hq = 4096, 32
    toks, heads = [], []
    for b in range(4):
        for p in list(range(4)) + list(range(S - 4, S)):
            toks += [b * S + p] * Hq
            heads += list(range(Hq))
        for p in (15, 16, 63, 64, 65, 127, 128, 1023, 1024, 2047, 2048, 3071):
            hs = rng.choice(Hq, 4, replace=False)
            toks += [b * S + p] * 4
            heads += hs.tolist()
    toks += rng.integers(0, 4 * S, 64).tolist()
    heads += rng.integers(0, Hq, 64).tolist()
    return np.array(toks, np.int64), np.array(heads, np.int32)


def gen_prefill(name):
    qb, kb, vb, pos, cu = kvgen.prefill_inputs(**PREFILL)
    toks, heads = prefill_rows()
    G = PREFILL["Hq"] // PREFILL["Hkv"]
    out = np.zeros((toks.size, D), np.float32)
    for i, (t, h) in enumerate(zip(toks, heads)):
        s0 = int(t) - int(pos[t])
        n = int(pos[t]) + 1
        kv = h // G
        K = np.ascontiguousarray(kb[s0:s0 + n, kv][None]).view(np.uint8).reshape(1, n, 2 * D)
        V = np.ascontiguousarray(vb[s0:s0 + n, kv][None]).view(np.uint8).reshape(1, n, 2 * D)
        q = O.bf16_to_f32(qb[t, h])[None, None, :]
        out[i] = O.ref_flash_attn(q, K, V, O.KV_BF16, n, 1, np.float32(1 / np.sqrt(D)),
                                  n_threads=4)[0, 0]
    np.savez(os.path.join(HERE, name), out=out, tokens=toks, heads=heads,
             crc_q=kvgen.crc(qb), crc_k=kvgen.crc(kb), crc_v=kvgen.crc(vb))
    print(f"{name}: {toks.size} rows")


def gen_tq_tables(name):
    """Lloyd-Max centroids / midpoints of the restated solver
    (turboquant_kernels.cu:578-623, :662-664) as fp32 bit patterns: the
    reference computes them on the host at start-up, so their last bits
    depend on the host libm; these are the values every test here uses."""
    import json
    res = {}
    for bits in (3, 4):
        c, m = O.tq_tables(D, bits)
        res[f"centroids_{bits}bit"] = [f"{v:08x}" for v in c.view(np.uint32)]
        res[f"midpoints_{bits}bit"] = [f"{v:08x}" for v in m.view(np.uint32)]
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(res, f, indent=1)
    print(f"{name}: written")


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref not built: run `make -C oracle ref` (needs the reference sources)")
    gen_quant(O.KV_Q8_0, "quant_q8_0.npz")
    gen_quant(O.KV_Q4_0, "quant_q4_0.npz")
    gen_decode_single(O.KV_F16, "fa_decode_f16.npz")
    gen_decode_single(O.KV_BF16, "fa_decode_bf16.npz")
    gen_decode_batched(O.KV_Q8_0, "fa_decode_q8_0.npz")
    gen_decode_batched(O.KV_Q4_0, "fa_decode_q4_0.npz")
    gen_prefill("fa_prefill_bf16.npz")
    gen_tq_tables("tq_tables_d128.json")


if __name__ == "__main__":
    main()
