"""ctypes bindings to the CPU checker (oracle/) and to the vendored-ggml
reference build (oracle/_ref/).

Test infrastructure: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py only.  numpy in, numpy out.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "libvmc_oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libggml_ref_harness.so")

KV_F16, KV_BF16, KV_Q8_0, KV_Q4_0 = 0, 1, 2, 3

_P = C.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


class TQLayout(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "head_dim", "key_quant_bits", "value_quant_bits", "norm_correction",
        "mse_bytes", "key_packed_size", "val_data_bytes", "value_packed_size",
        "slot_size", "slot_size_aligned", "n_centroids", "key_fp8", "fp8_e4b15")]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        L = C.CDLL(ORACLE_SO)
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        for n in ("orc_f32_to_f16_n", "orc_f16_to_f32_n"):
            getattr(L, n).argtypes = [_P, _P, C.c_int64]
        for n in ("orc_quantize_row_q8_0", "orc_dequantize_row_q8_0",
                  "orc_quantize_row_q4_0", "orc_dequantize_row_q4_0"):
            getattr(L, n).argtypes = [_P, _P, C.c_int64]
        L.orc_kv_entry_bytes.restype = C.c_int64
        L.orc_kv_entry_bytes.argtypes = [C.c_int, C.c_int]
        L.orc_kv_append.argtypes = [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int,
                                    C.c_int64, C.c_int, C.c_int]
        L.orc_kv_dequant_entry.argtypes = [_P, C.c_int, C.c_int, _P]
        L.orc_tq_layout_from_method.restype = C.c_int
        L.orc_tq_layout_from_method.argtypes = [C.c_int, C.c_char_p, C.POINTER(TQLayout)]
        L.orc_tq_hadamard.argtypes = [_P, C.c_int]
        L.orc_tq_lloyd_max.argtypes = [_P, C.c_int, C.c_int]
        L.orc_tq_midpoints.argtypes = [_P, C.c_int, _P]
        L.orc_tq_rotate.argtypes = [_P, _P, _P, C.c_int]
        L.orc_tq_store.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int64,
                                   C.POINTER(TQLayout), _P, C.c_int]
        L.orc_tq_dequant_slot.argtypes = [_P, C.POINTER(TQLayout), _P, C.c_int, _P, _P]
        L.orc_tq_decode.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                    C.c_float, C.c_int64, C.c_int64, C.POINTER(TQLayout), _P,
                                    C.c_int, C.c_int, C.c_int]
        L.orc_tq_decode_exact.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int,
                                          C.c_int, C.c_double, C.c_int64, C.c_int64,
                                          C.POINTER(TQLayout), _P, C.c_int, C.c_int]
        L.orc_g32_signs.argtypes = [C.c_uint64, _P, C.c_int]
        L.orc_g32_part_bytes.restype = C.c_int
        L.orc_g32_part_bytes.argtypes = [C.c_int]
        L.orc_g32_quantize_part.argtypes = [_P, C.c_int, _P]
        L.orc_g32_dequant_part.argtypes = [_P, C.c_int, _P]
        L.orc_g32_store.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int64, C.c_int,
                                    C.c_uint64, C.c_int]
        L.orc_g32_decode_exact.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_double, C.c_int64, C.c_int64, C.c_int, C.c_uint64,
                                           C.c_int, C.c_int]
        L.orc_f32_to_ofp8_n.argtypes = [_P, _P, C.c_int64, C.c_int]
        L.orc_ofp8_to_f32.argtypes = [C.c_uint8, C.c_int]
        L.orc_ofp8_to_f32.restype = C.c_float
        L.orc_reshape_and_cache_fp8.argtypes = [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int,
                                                C.c_int64, C.c_int64, C.c_float, C.c_float, C.c_int]
        L.orc_convert_fp8.argtypes = [_P, _P, C.c_int, C.c_float, C.c_int64, C.c_int]
        L.orc_f32_to_fp8.argtypes = [C.c_float, C.c_int]
        L.orc_f32_to_fp8.restype = C.c_uint8
        L.orc_fp8_to_f32.argtypes = [C.c_uint8, C.c_int]
        L.orc_fp8_to_f32.restype = C.c_float
        L.orc_qk_norm_rope.argtypes = [_P, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_float, C.c_int, C.c_int]
        L.orc_paged_decode_exact.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, _P, _P,
                                             C.c_int, C.c_int, C.c_int, C.c_int, C.c_double,
                                             C.c_int64, C.c_int64, C.c_int]
        L.orc_decode_ggml.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, _P, _P, C.c_int,
                                      C.c_int, C.c_int, C.c_int, C.c_float, C.c_int64,
                                      C.c_int64, C.c_int, C.c_int]
        L.orc_prefill_exact_rows.argtypes = [_P, _P, _P, _P, C.c_int, _P, C.c_int, C.c_int,
                                             C.c_int, C.c_int, C.c_double, _P, _P, C.c_int64,
                                             C.c_int]
        L.orc_randn.restype = C.c_double
        L.orc_randn.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.orc_rand_u64.restype = C.c_uint64
        L.orc_rand_u64.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.orc_randn_f16.argtypes = [_P, C.c_int64, C.c_uint64, C.c_uint64]
        L.orc_randn_bf16.argtypes = [_P, C.c_int64, C.c_uint64, C.c_uint64]
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError("reference build absent: run `make -C oracle ref`")
        R = C.CDLL(REF_SO)
        R.ref_from_float.restype = C.c_int
        R.ref_from_float.argtypes = [C.c_int, _P, _P, C.c_int64]
        R.ref_quantize_q8_0_ref.argtypes = [_P, _P, C.c_int64]
        R.ref_quantize_q4_0_ref.argtypes = [_P, _P, C.c_int64]
        R.ref_flash_attn.restype = C.c_int
        R.ref_flash_attn.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_float, C.c_int, C.c_int]
        R.ref_flash_attn_timed.restype = C.c_int
        R.ref_flash_attn_timed.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_int, C.c_float, C.c_int, C.c_int, C.c_int,
                                           C.POINTER(C.c_double)]
        _ref = R
    return _ref


# ---------------------------------------------------------------- helpers

def f16_bits(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32)).astype(np.float16).view(np.uint16)


def entry_bytes(fmt, d):
    return int(lib().orc_kv_entry_bytes(fmt, d))


def quantize_rows(fmt, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    out = np.zeros(n // 32 * (34 if fmt == KV_Q8_0 else 18), dtype=np.uint8)
    fn = lib().orc_quantize_row_q8_0 if fmt == KV_Q8_0 else lib().orc_quantize_row_q4_0
    fn(_ptr(x), _ptr(out), n)
    return out


def dequantize_rows(fmt, q, n):
    out = np.zeros(n, dtype=np.float32)
    fn = lib().orc_dequantize_row_q8_0 if fmt == KV_Q8_0 else lib().orc_dequantize_row_q4_0
    fn(_ptr(np.ascontiguousarray(q)), _ptr(out), n)
    return out


def tq_layout(method, head_dim=128):
    L = TQLayout()
    rc = lib().orc_tq_layout_from_method(head_dim, method.encode(), C.byref(L))
    if rc != 0:
        raise ValueError(method)
    return L


def tq_tables(head_dim, bits):
    n = 1 << bits
    c = np.zeros(n, dtype=np.float32)
    lib().orc_tq_lloyd_max(_ptr(c), head_dim, bits)
    m = np.zeros(n - 1, dtype=np.float32)
    lib().orc_tq_midpoints(_ptr(c), n, _ptr(m))
    return c, m


def tq_rotate(x, signs=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().orc_tq_rotate(_ptr(x), _ptr(signs), _ptr(y), x.size)
    return y


def kv_append(key_bits, value_bits, slot_mapping, kcache, vcache, block_size, fmt,
              hnd=False, src_bf16=False):
    T, H, D = key_bits.shape
    lib().orc_kv_append(_ptr(np.ascontiguousarray(key_bits)), _ptr(np.ascontiguousarray(value_bits)),
                        int(src_bf16), _ptr(kcache), _ptr(vcache),
                        _ptr(np.ascontiguousarray(slot_mapping, dtype=np.int64)), T, H, D,
                        block_size, fmt, int(hnd))


def tq_store(key_bits, value_bits, slot_mapping, cache, block_size, L, midpoints, bf16=False):
    T, H, D = key_bits.shape
    lib().orc_tq_store(_ptr(np.ascontiguousarray(key_bits)), _ptr(np.ascontiguousarray(value_bits)),
                       _ptr(cache), _ptr(np.ascontiguousarray(slot_mapping, dtype=np.int64)),
                       T, H, D, block_size, C.byref(L), _ptr(midpoints), int(bf16))


def tq_decode(q_bits, cache, block_tables, seq_lens, Hkv, scale, block_size, L, centroids,
              num_splits=32, bf16=False, nthreads=0):
    B, Hq, D = q_bits.shape
    out = np.zeros((B, Hq, D), dtype=np.uint16)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    lib().orc_tq_decode(_ptr(out), _ptr(np.ascontiguousarray(q_bits)), _ptr(cache), _ptr(bt),
                        _ptr(np.ascontiguousarray(seq_lens, dtype=np.int32)), B, Hq, Hkv, D,
                        scale, block_size, bt.shape[1], C.byref(L), _ptr(centroids), num_splits,
                        int(bf16), nthreads)
    return out


def tq_decode_exact(q_bits, cache, block_tables, seq_lens, Hkv, scale, block_size, L, centroids,
                    bf16=False, nthreads=0):
    B, Hq, D = q_bits.shape
    out = np.zeros((B, Hq, D), dtype=np.float64)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    lib().orc_tq_decode_exact(_ptr(out), _ptr(np.ascontiguousarray(q_bits)), _ptr(cache),
                              _ptr(bt), _ptr(np.ascontiguousarray(seq_lens, dtype=np.int32)),
                              B, Hq, Hkv, D, scale, block_size, bt.shape[1], C.byref(L),
                              _ptr(centroids), int(bf16), nthreads)
    return out


def g32_signs(seed, d=128):
    out = np.zeros(d, dtype=np.float32)
    lib().orc_g32_signs(seed, _ptr(out), d)
    return out


def g32_part_bytes(bits):
    return int(lib().orc_g32_part_bytes(bits))


def g32_quantize_part(y, bits):
    y = np.ascontiguousarray(y, dtype=np.float32)
    assert y.size == 128
    out = np.zeros(g32_part_bytes(bits), dtype=np.uint8)
    lib().orc_g32_quantize_part(_ptr(y), bits, _ptr(out))
    return out


def g32_dequant_part(part, bits):
    part = np.ascontiguousarray(part, dtype=np.uint8)
    out = np.zeros(128, dtype=np.float32)
    lib().orc_g32_dequant_part(_ptr(part), bits, _ptr(out))
    return out


def g32_store(key_bits, value_bits, slot_mapping, cache, block_size, bits, seed, bf16=False):
    T, H, D = key_bits.shape
    lib().orc_g32_store(_ptr(np.ascontiguousarray(key_bits)), _ptr(np.ascontiguousarray(value_bits)),
                        _ptr(cache), _ptr(np.ascontiguousarray(slot_mapping, dtype=np.int64)),
                        T, H, D, block_size, bits, seed, int(bf16))


def g32_decode_exact(q_bits, cache, block_tables, seq_lens, Hkv, scale, block_size, bits, seed,
                     bf16=False, nthreads=0):
    B, Hq, D = q_bits.shape
    out = np.zeros((B, Hq, D), dtype=np.float64)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    lib().orc_g32_decode_exact(_ptr(out), _ptr(np.ascontiguousarray(q_bits)), _ptr(cache), _ptr(bt),
                               _ptr(np.ascontiguousarray(seq_lens, dtype=np.int32)), B, Hq, Hkv, D,
                               scale, block_size, bt.shape[1], bits, seed, int(bf16), nthreads)
    return out


def ofp8_encode(x, e5m2=False):
    """OCP E4M3 / E5M2 bytes of fp32 values (round to nearest even, saturated)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(x.shape, np.uint8)
    lib().orc_f32_to_ofp8_n(_ptr(x), _ptr(y), x.size, int(e5m2))
    return y


def ofp8_decode(b, e5m2=False):
    b = np.asarray(b, np.uint8)
    return np.array([lib().orc_ofp8_to_f32(int(v), int(e5m2)) for v in b.ravel()],
                    np.float32).reshape(b.shape)


def reshape_and_cache_fp8(key_bits, value_bits, slot_mapping, kcache, vcache, block_size, k_scale=1.0,
                          v_scale=1.0, hnd=False, src_bf16=False, stride=0):
    T, H, D = key_bits.shape
    lib().orc_reshape_and_cache_fp8(_ptr(np.ascontiguousarray(key_bits)), _ptr(np.ascontiguousarray(value_bits)),
                                    int(src_bf16), _ptr(kcache), _ptr(vcache),
                                    _ptr(np.ascontiguousarray(slot_mapping, dtype=np.int64)), T, H, D,
                                    block_size, stride, float(k_scale), float(v_scale), int(hnd))


def convert_fp8(src_bits, scale, e5m2=False, src_bf16=False):
    src = np.ascontiguousarray(src_bits, np.uint16)
    dst = np.zeros(src.shape, np.uint8)
    lib().orc_convert_fp8(_ptr(dst), _ptr(src), int(src_bf16), float(scale), src.size, int(e5m2))
    return dst


def fp8_encode(x, e4b15=False):
    x = np.asarray(x, np.float32)
    return np.array([lib().orc_f32_to_fp8(float(v), int(e4b15)) for v in x.ravel()],
                    np.uint8).reshape(x.shape)


def fp8_decode(b, e4b15=False):
    b = np.asarray(b, np.uint8)
    return np.array([lib().orc_fp8_to_f32(int(v), int(e4b15)) for v in b.ravel()],
                    np.float32).reshape(b.shape)


def qk_norm_rope(q_bits, k_bits, q_weight, k_weight, cos_sin, pos, eps, is_neox, bf16=False):
    """In-place restatement on copies; returns (q, k) as uint16 bit arrays."""
    q = np.ascontiguousarray(q_bits, dtype=np.uint16).copy()
    k = np.ascontiguousarray(k_bits, dtype=np.uint16).copy()
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    qw = None if q_weight is None else np.ascontiguousarray(q_weight, dtype=np.uint16)
    kw = None if k_weight is None else np.ascontiguousarray(k_weight, dtype=np.uint16)
    lib().orc_qk_norm_rope(_ptr(q), _ptr(k), _ptr(qw), _ptr(kw),
                           _ptr(np.ascontiguousarray(cos_sin, dtype=np.uint16)),
                           _ptr(np.ascontiguousarray(pos, dtype=np.int64)), T, Hq, Hkv, D, eps,
                           int(is_neox), int(bf16))
    return q, k


def paged_decode_exact(q, kcache, vcache, fmt, block_tables, seq_lens, Hkv, scale, block_size,
                       hnd=False, nthreads=0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, D = q.shape
    out = np.zeros((B, Hq, D), dtype=np.float64)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    lib().orc_paged_decode_exact(_ptr(out), _ptr(q), _ptr(kcache), _ptr(vcache), fmt, int(hnd),
                                 _ptr(bt), _ptr(np.ascontiguousarray(seq_lens, dtype=np.int32)),
                                 B, Hq, Hkv, D, scale, block_size, bt.shape[1], nthreads)
    return out


def decode_ggml(q, kcache, vcache, fmt, block_tables, seq_lens, Hkv, scale, block_size,
                hnd=False, nth=1, nthreads=0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, D = q.shape
    out = np.zeros((B, Hq, D), dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    lib().orc_decode_ggml(_ptr(out), _ptr(q), _ptr(kcache), _ptr(vcache), fmt, int(hnd),
                          _ptr(bt), _ptr(np.ascontiguousarray(seq_lens, dtype=np.int32)),
                          B, Hq, Hkv, D, scale, block_size, bt.shape[1], nth, nthreads)
    return out


def prefill_exact_rows(q, k, v, cu_seqlens, Hkv, scale, tokens, heads, is_bf16=True, nthreads=0):
    T, Hq, D = q.shape
    tokens = np.ascontiguousarray(tokens, dtype=np.int64)
    heads = np.ascontiguousarray(heads, dtype=np.int32)
    out = np.zeros((tokens.size, D), dtype=np.float64)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    lib().orc_prefill_exact_rows(_ptr(out), _ptr(np.ascontiguousarray(q)), _ptr(np.ascontiguousarray(k)),
                                 _ptr(np.ascontiguousarray(v)), int(is_bf16), _ptr(cu),
                                 cu.size - 1, Hq, Hkv, D, scale, _ptr(tokens), _ptr(heads),
                                 tokens.size, nthreads)
    return out


def randn_f16(n, seed, stream):
    out = np.zeros(n, dtype=np.uint16)
    lib().orc_randn_f16(_ptr(out), n, seed, stream)
    return out


def randn_bf16(n, seed, stream):
    out = np.zeros(n, dtype=np.uint16)
    lib().orc_randn_bf16(_ptr(out), n, seed, stream)
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------ reference side

def ref_quantize(fmt, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * (34 if fmt == KV_Q8_0 else 18), dtype=np.uint8)
    fn = ref().ref_quantize_q8_0_ref if fmt == KV_Q8_0 else ref().ref_quantize_q4_0_ref
    fn(_ptr(x), _ptr(out), x.size)
    return out


def ref_from_float(fmt, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * (34 if fmt == KV_Q8_0 else 18), dtype=np.uint8)
    rc = ref().ref_from_float(fmt, _ptr(x), _ptr(out), x.size)
    assert rc == 0
    return out


def ref_flash_attn(q, k_rows, v_rows, fmt, n_kv, Hkv, scale, causal=False, n_threads=1):
    """q: fp32 [Hq][n_q][D]; k_rows/v_rows: uint8 [Hkv][n_kv][row] -> out fp32 [n_q][Hq][D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    Hq, n_q, D = q.shape
    out = np.zeros((n_q, Hq, D), dtype=np.float32)
    rc = ref().ref_flash_attn(_ptr(out), _ptr(q), _ptr(np.ascontiguousarray(k_rows)),
                              _ptr(np.ascontiguousarray(v_rows)), fmt, n_q, n_kv, Hq, Hkv, D,
                              scale, int(causal), n_threads)
    assert rc == 0, rc
    return out


def ref_flash_attn_timed(q, k_rows, v_rows, fmt, n_kv, Hkv, scale, causal=False, n_threads=1, reps=1):
    """ref_flash_attn computed `reps` times on one built graph; returns
    (out fp32 [n_q][Hq][D], mean seconds of one graph compute)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    Hq, n_q, D = q.shape
    out = np.zeros((n_q, Hq, D), dtype=np.float32)
    secs = C.c_double(0.0)
    rc = ref().ref_flash_attn_timed(_ptr(out), _ptr(q), _ptr(np.ascontiguousarray(k_rows)),
                                    _ptr(np.ascontiguousarray(v_rows)), fmt, n_q, n_kv, Hq, Hkv, D,
                                    scale, int(causal), n_threads, reps, C.byref(secs))
    assert rc == 0, rc
    return out, secs.value
