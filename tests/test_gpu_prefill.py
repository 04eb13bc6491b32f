"""Causal prefill parity on the GPU: HIP MFMA prefill vs exact fp64 causal
attention (oracle), tolerance |got - ref| <= 2e-3 + 1e-2 |ref|; the fused
quantize-on-append must write the same bytes as the standalone append.  Each
case runs through vmc_flash_attention_prefill and, with a workspace of
prebuilt V^T tiles, through vmc_flash_attention_prefill_ws, whose outputs
must equal the first's bit for bit wherever neither runs the exact mode."""
import os

import numpy as np
import pytest

import oracle_lib as O
from kvgen import BS, close_report, crc, prefill_inputs

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _inputs(seq_lens, Hq, Hkv, D=128, seed=0, bf16=True):
    return prefill_inputs(seq_lens, Hq, Hkv, D=D, seed=seed, bf16=bf16)


def _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=True, append=None, ws=False):
    import torch
    from vm_c_amd import capi
    tdt = torch.bfloat16 if bf16 else torch.float16
    to = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(tdt)
    q, k, v = to(qb), to(kb), to(vb)
    out = torch.full_like(q, float("nan"))
    kw = {}
    if ws:
        n = capi.flash_attention_prefill_workspace_size(q.shape[0], Hkv, q.shape[2])
        # stale bytes from an earlier use must not matter
        kw["workspace"] = torch.full((n,), 0xA5, dtype=torch.uint8, device=dev)
    if append is not None:
        fmt, slots, nbytes = append
        kc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        vc = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        kw.update(key_cache=kc, value_cache=vc, slot_mapping=torch.from_numpy(slots).to(dev),
                  block_size=BS, kv_format=fmt)
    capi.flash_attention_prefill(out, q, k, v, torch.from_numpy(pos).to(dev), Hkv, scale, **kw)
    torch.cuda.synchronize()
    res = out.float().cpu().numpy()
    if append is not None:
        return res, kw["key_cache"].cpu().numpy(), kw["value_cache"].cpu().numpy()
    return res


@pytest.mark.parametrize("ws", [False, True])
@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("seq_lens,Hq,Hkv", [([300, 77], 8, 2), ([1, 2, 129, 64, 200], 4, 4),
                                              ([513], 8, 1), ([256, 64, 192], 8, 2)])
def test_prefill_all_rows_vs_exact(dev, bf16, seq_lens, Hq, Hkv, ws):
    qb, kb, vb, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=len(seq_lens), bf16=bf16)
    T = qb.shape[0]
    scale = 1.0 / np.sqrt(128)
    got = _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=bf16, ws=ws)
    toks = np.repeat(np.arange(T), Hq)
    heads = np.tile(np.arange(Hq), T)
    ex = O.prefill_exact_rows(qb, kb, vb, cu, Hkv, scale, toks, heads, is_bf16=bf16)
    ok, err = close_report(got.reshape(T * Hq, 128), ex, ATOL, RTOL)
    assert ok, f"max err {err}"


def _slots_for(T, seed):
    rng = np.random.default_rng(seed)
    nblk = (T + BS - 1) // BS
    perm = rng.permutation(nblk).astype(np.int64)
    t = np.arange(T)
    return perm[t // BS] * BS + t % BS, nblk


@pytest.mark.parametrize("ws", [False, True])
@pytest.mark.parametrize("fmt", [O.KV_Q8_0, O.KV_Q4_0, O.KV_F16, O.KV_BF16])
def test_prefill_fused_append_bitexact(dev, fmt, ws):
    seq_lens, Hq, Hkv = [333, 190], 8, 2
    qb, kb, vb, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=13)
    T = qb.shape[0]
    slots, nblk = _slots_for(T, 3)
    slots[7] = -1
    E = O.entry_bytes(fmt, 128)
    nbytes = nblk * BS * Hkv * E
    got, kc, vc = _run(dev, qb, kb, vb, pos, Hkv, 1.0 / np.sqrt(128), append=(fmt, slots, nbytes), ws=ws)
    kr = np.zeros(nbytes, np.uint8)
    vr = np.zeros(nbytes, np.uint8)
    O.kv_append(kb, vb, slots, kr, vr, BS, fmt, src_bf16=True)
    assert np.array_equal(kc, kr) and np.array_equal(vc, vr)


def test_prefill_config4_full_size(dev):
    """B=4, S=4096, Hq=32, Hkv=8, bf16, causal, fused q8_0 append (seed 3):
    1,280 rows vs the reference's output (golden fixture: every head of the
    first and last 4 rows of each sequence, tile and page edges), 8,256 rows
    vs exact fp64, every page byte vs the oracle's append."""
    seq_lens, Hq, Hkv = [4096] * 4, 32, 8
    qb, kb, vb, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=3)
    T = qb.shape[0]
    slots, nblk = _slots_for(T, 4)
    E = O.entry_bytes(O.KV_Q8_0, 128)
    nbytes = nblk * BS * Hkv * E
    scale = 1.0 / np.sqrt(128)
    got, kc, vc = _run(dev, qb, kb, vb, pos, Hkv, scale, append=(O.KV_Q8_0, slots, nbytes), ws=True)
    # the workspace path (prebuilt V^T tiles, the benchmark's) equals the
    # in-kernel one bit for bit on this input
    got0 = _run(dev, qb, kb, vb, pos, Hkv, scale)
    assert np.array_equal(got.view(np.uint32), got0.view(np.uint32))
    # 8,256 rows against fp64 attention: every head of 256 random tokens and
    # of the first and last token of each sequence
    rng = np.random.default_rng(0)
    pick = np.concatenate([rng.integers(0, T, 256), [0, 4095, 4096, 8191, 8192, 12287, 12288, T - 1]])
    toks = np.repeat(pick, Hq)
    heads = np.tile(np.arange(Hq), pick.size)
    ex = O.prefill_exact_rows(qb, kb, vb, cu, Hkv, scale, toks, heads)
    ok, err = close_report(got[toks, heads], ex, ATOL, RTOL)
    assert ok, f"max err {err}"
    assert np.isfinite(got).all()
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "fa_prefill_bf16.npz"))
    assert (crc(qb), crc(kb), crc(vb)) == (g["crc_q"], g["crc_k"], g["crc_v"])
    ok, err = close_report(got[g["tokens"], g["heads"]], g["out"], ATOL, RTOL)
    assert ok, f"vs reference rows: max err {err}"
    kr = np.zeros(nbytes, np.uint8)
    vr = np.zeros(nbytes, np.uint8)
    O.kv_append(kb, vb, slots, kr, vr, BS, O.KV_Q8_0, src_bf16=True)
    assert np.array_equal(kc, kr) and np.array_equal(vc, vr)


@pytest.mark.parametrize("ws", [False, True])
def test_prefill_bf16_v_outside_fp16_range(dev, ws):
    """bf16 V that fp16 cannot hold: one sequence at 2^100 scale (fp16
    overflows), one at 2^-20 (fp16 subnormals keep 4 bits) with bf16
    subnormals mixed in, one N(0,1) with sparse +-1e30 and +-1e-38 spikes
    (these three take the kernel's exact mode), and one N(0,1) with sparse
    2^-20 and +-1e-38 values only (the fp16 path, whose rounding of them is
    below 2^-25).  Each sequence's rows are compared with exact fp64
    attention after dividing both by the sequence's magnitude, so the usual
    tolerance is relative to that scale."""
    from kvgen import f32_to_bf16_bits
    seq_lens, Hq, Hkv = [300, 77, 129, 200], 8, 2
    qb, kb, _, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=21)
    T = qb.shape[0]
    rng = np.random.default_rng(22)
    v = rng.standard_normal((T, Hkv, 128)).astype(np.float64)
    mag = np.ones(T)
    mag[cu[0]:cu[1]] = 2.0 ** 100
    mag[cu[1]:cu[2]] = 2.0 ** -20
    v *= mag[:, None, None]
    tiny = rng.random(v[cu[1]:cu[2]].shape) < 0.05
    v[cu[1]:cu[2]][tiny] = 2.0 ** -130 * rng.choice([-1, 1], int(tiny.sum()))
    for b, vals in ((2, [-1e30, 1e30, -1e-38, 1e-38]), (3, [-2.0 ** -20, 2.0 ** -20, -1e-38, 1e-38])):
        seg = v[cu[b]:cu[b + 1]].reshape(-1)
        spikes = np.flatnonzero(rng.random(seg.size) < 2e-3)
        seg[spikes] = rng.choice(vals, spikes.size)
        v[cu[b]:cu[b + 1]] = seg.reshape(v[cu[b]:cu[b + 1]].shape)
    vb = f32_to_bf16_bits(v.astype(np.float32))
    scale = 1.0 / np.sqrt(128)
    got = _run(dev, qb, kb, vb, pos, Hkv, scale, ws=ws).reshape(T * Hq, 128)
    assert np.isfinite(got).all()
    toks = np.repeat(np.arange(T), Hq)
    heads = np.tile(np.arange(Hq), T)
    ex = O.prefill_exact_rows(qb, kb, vb, cu, Hkv, scale, toks, heads)
    rs = mag[toks][:, None]
    for b in range(len(seq_lens)):
        sel = (toks >= cu[b]) & (toks < cu[b + 1])
        ok, err = close_report(got[sel] / rs[sel], ex[sel] / rs[sel], ATOL, RTOL)
        assert ok, f"sequence {b}: max scaled err {err}"


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("seq_lens,Hq,Hkv", [([256, 512, 64, 128], 8, 2), ([300, 77, 129], 4, 1),
                                              ([1000, 24], 32, 8)])
def test_prefill_ws_equals_in_kernel_transpose(dev, bf16, seq_lens, Hq, Hkv):
    """Prebuilt V^T tiles (sequences starting on 64-key boundaries) and the
    in-kernel pass (the others) give the same bits."""
    qb, kb, vb, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=31, bf16=bf16)
    scale = 1.0 / np.sqrt(128)
    a = _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=bf16)
    b = _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=bf16, ws=True)
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_prefill_ws_fp16_inf_in_a_shared_tile(dev):
    """fp16 V with an inf in the second sequence, which shares a 64-key tile
    with the first: the tile's flag sends the workgroups that read it to
    the in-kernel pass, so the two paths agree bit for bit; the first
    sequence's rows of other tiles and the third sequence (no shared tile)
    stay finite.  (Rows whose tile holds the inf, masked or not, are not
    finite on either path: 0 * inf in the P . V product.)"""
    seq_lens, Hq, Hkv = [100, 28, 64], 8, 2
    qb, kb, vb, pos, cu = _inputs(seq_lens, Hq, Hkv, seed=33, bf16=False)
    vb = vb.copy()
    vb[cu[1] + 3, 1, 17] = 0x7C00  # +inf, second sequence, KV head 1
    scale = 1.0 / np.sqrt(128)
    a = _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=False)
    b = _run(dev, qb, kb, vb, pos, Hkv, scale, bf16=False, ws=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.isfinite(b[:64]).all() and np.isfinite(b[cu[2]:cu[3]]).all()
    assert np.isfinite(b[cu[0]:cu[1], :4]).all()  # query heads of KV head 0
