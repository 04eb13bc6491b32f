"""ctypes binding of the C ABI in include/vmc_attn.h (libvmc_attn.so).

Thin: torch tensors are used only as device memory and for the current HIP
stream; every call goes straight to the gfx950 kernels.  There is no fallback:
if the library is missing or a call fails, this raises.
"""
import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libvmc_attn.so")

VMC_OK, VMC_EINVAL, VMC_ENOMEM, VMC_EIO = 0, -22, -12, -5
DTYPE_F16, DTYPE_BF16 = 0, 1
KV_F16, KV_BF16, KV_Q8_0, KV_Q4_0 = 0, 1, 2, 3
LAYOUT_NHD, LAYOUT_HND = 0, 1
KV_FORMATS = {"fp16": KV_F16, "bf16": KV_BF16, "q8_0": KV_Q8_0, "q4_0": KV_Q4_0}

EXPORTS = [
    "vmc_kv_entry_bytes", "vmc_reshape_and_cache", "vmc_paged_decode_workspace_size",
    "vmc_paged_attention_decode", "vmc_tq_config_from_method", "vmc_tq_host_tables",
    "vmc_turboquant_store", "vmc_turboquant_decode_workspace_size",
    "vmc_turboquant_decode_attention", "vmc_flash_attention_prefill",
    "vmc_flash_attention_prefill_v2", "vmc_selftest",
    "vmc_version",
]


class TQConfig(C.Structure):
    """Mirror of vmc_tq_config (vm_c::TQConfig)."""
    _fields_ = [(n, C.c_int) for n in (
        "head_dim", "key_quant_bits", "value_quant_bits", "norm_correction", "key_fp8",
        "fp8_e4b15", "mse_bytes", "key_packed_size", "val_data_bytes", "value_packed_size",
        "slot_size", "slot_size_aligned", "n_centroids", "max_num_kv_splits",
        "group_size")] + [("sign_seed", C.c_ulonglong)]


class VmcError(RuntimeError):
    pass


_lib = None
_P = C.c_void_p
_I, _I64, _F, _SZ = C.c_int, C.c_int64, C.c_float, C.c_size_t


def load():
    """Load libvmc_attn.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VmcError(f"{LIB_PATH} not built: run `python -m vm_c_amd.build`")
    L = C.CDLL(LIB_PATH)
    L.vmc_kv_entry_bytes.restype = _I64
    L.vmc_kv_entry_bytes.argtypes = [_I, _I]
    L.vmc_reshape_and_cache.restype = _I
    L.vmc_reshape_and_cache.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I64, _I64, _I, _I, _I, _P]
    L.vmc_reshape_and_cache_fp8.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I64, _I64, _P, _P, _I, _I, _P]
    L.vmc_convert_fp8.argtypes = [_P, _P, C.c_double, _I64, _I, _I, _P]
    L.vmc_paged_decode_workspace_size.restype = _SZ
    L.vmc_paged_decode_workspace_size.argtypes = [_I, _I, _I, _I, _I, _I, _I]
    L.vmc_paged_attention_decode.restype = _I
    L.vmc_paged_attention_decode.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F,
                                             _I, _I, _I, _I, _P, _SZ, _P]
    L.vmc_paged_attention_prefill.restype = _I
    L.vmc_paged_attention_prefill.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P,
                                              _I, _I, _I, _I, _P, _SZ, _P]
    L.vmc_flash_attention_prefill_v2.restype = _I
    L.vmc_flash_attention_prefill_v2.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P,
                                                 _P, _I, _I, _I, _I, _P]
    L.vmc_turboquant_prefill_attention.restype = _I
    L.vmc_turboquant_prefill_attention.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I64,
                                                   _I64, C.POINTER(TQConfig), _I, _I, _P, _SZ, _P]
    L.vmc_batch_token_rows.restype = _I
    L.vmc_batch_token_rows.argtypes = [_P, _P, _P, _P, _P, _I, _I, _P]
    L.vmc_tq_config_from_method.restype = _I
    L.vmc_tq_config_from_method.argtypes = [_I, C.c_char_p, C.POINTER(TQConfig)]
    L.vmc_tq_host_tables.restype = _I
    L.vmc_tq_host_tables.argtypes = [_I, _I, _P, _P]
    L.vmc_turboquant_store.restype = _I
    L.vmc_turboquant_store.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I64, C.POINTER(TQConfig), _I, _P]
    L.vmc_turboquant_decode_workspace_size.restype = _SZ
    L.vmc_turboquant_decode_workspace_size.argtypes = [_I, _I, _I, _I, _I64, _I64, _I]
    L.vmc_turboquant_decode_attention.restype = _I
    L.vmc_turboquant_decode_attention.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I64,
                                                  _I64, C.POINTER(TQConfig), _I, _I, _P, _SZ, _P]
    L.vmc_noalloc_scratch_bytes.restype = _SZ
    L.vmc_noalloc_scratch_bytes.argtypes = []
    L.vmc_turboquant_decode_attention_noalloc.restype = _I
    L.vmc_turboquant_decode_attention_noalloc.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I64,
                                                          _I64, C.POINTER(TQConfig), _I, _I, _P]
    L.vmc_fused_qk_norm_rope_store.restype = _I
    L.vmc_fused_qk_norm_rope_store.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                               _F, _I, _I64, _I64, _I, _I, C.POINTER(TQConfig), _I,
                                               _P]
    L.vmc_flash_attention_prefill.restype = _I
    L.vmc_flash_attention_prefill.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P, _P,
                                              _P, _I64, _I, _I, _P]
    L.vmc_flash_attention_prefill_workspace_size.restype = _SZ
    L.vmc_flash_attention_prefill_workspace_size.argtypes = [_I, _I, _I]
    L.vmc_flash_attention_prefill_ws.restype = _I
    L.vmc_flash_attention_prefill_ws.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P, _P,
                                                 _P, _I64, _I, _I, _P, _SZ, _P]
    L.vmc_hbm_read_probe.restype = _I
    L.vmc_hbm_read_probe.argtypes = [_P, _SZ, _I, _P, _P]
    L.vmc_selftest.restype = _I
    L.vmc_selftest.argtypes = []
    L.vmc_version.restype = C.c_char_p
    L.vmc_version.argtypes = []
    _lib = L
    return L


def _check(rc, what):
    if rc != VMC_OK:
        raise VmcError(f"{what} failed with status {rc}")


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dtype_code(t):
    import torch
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise VmcError(f"unsupported dtype {t.dtype}")


SELFTEST_CHECKS = {1: "sum over rows", 2: "max over rows", 4: "LDS gather",
                   8: "mfma 16x16x32 f16", 16: "mfma 16x16x16 f16", 32: "mfma 32x32x16 f16",
                   64: "mfma 16x16x32 bf16", 128: "mfma 32x32x16 bf16",
                   256: "mfma 16x16x16 f16 subnormal operands", 512: "LDS gather from the diagonal",
                   1024: "mfma 16x16x32 f16 subnormal operands",
                   2048: "bf16 conversion instruction vs the integer rounding rule",
                   4096: "16-lane DPP xor exchanges", 8192: "16-lane DPP row sum"}


def selftest():
    """Run the device self-check; raises VmcError naming the failed checks."""
    rc = load().vmc_selftest()
    if rc < 0:
        raise VmcError(f"vmc_selftest failed with status {rc}")
    if rc:
        raise VmcError("device self-check failed: " +
                       ", ".join(n for b, n in SELFTEST_CHECKS.items() if rc & b))


def version():
    return load().vmc_version().decode()


def kv_entry_bytes(kv_format, head_dim):
    return int(load().vmc_kv_entry_bytes(kv_format, head_dim))


def tq_config(head_dim=128, method="turboquant_4bit_nc", sign_seed=0):
    """vmc_tq_config_from_method; sign_seed sets the rotation signs of the
    per-32-group methods ("turboquant_4bit_g32", "turboquant_3bit_g32")."""
    cfg = TQConfig()
    _check(load().vmc_tq_config_from_method(head_dim, method.encode(), C.byref(cfg)),
           f"vmc_tq_config_from_method({method})")
    cfg.sign_seed = int(sign_seed)
    return cfg


def tq_host_tables(head_dim, bits):
    import numpy as np
    n = 1 << bits
    c = np.zeros(n, dtype=np.float32)
    m = np.zeros(n - 1, dtype=np.float32)
    _check(load().vmc_tq_host_tables(head_dim, bits, c.ctypes.data_as(_P), m.ctypes.data_as(_P)),
           "vmc_tq_host_tables")
    return c, m


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, block_size,
                      kv_format=KV_F16, layout=LAYOUT_NHD, cache_stride=0, stream=None):
    T, H, D = key.shape
    rc = load().vmc_reshape_and_cache(_ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
                                      _ptr(slot_mapping), T, H, D, block_size, cache_stride,
                                      kv_format, _dtype_code(key), layout, _stream(stream))
    _check(rc, "vmc_reshape_and_cache")


def reshape_and_cache_fp8(key, value, key_cache, value_cache, slot_mapping, block_size, k_scale=None,
                          v_scale=None, layout=LAYOUT_NHD, cache_stride=0, stream=None):
    """vmc_reshape_and_cache_fp8: E4M3 pages of key / k_scale and value / v_scale
    (scales are host floats, None = 1)."""
    T, H, D = key.shape
    ks = C.c_float(k_scale) if k_scale is not None else None
    vs = C.c_float(v_scale) if v_scale is not None else None
    rc = load().vmc_reshape_and_cache_fp8(_ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
                                          _ptr(slot_mapping), T, H, D, block_size, cache_stride,
                                          C.byref(ks) if ks is not None else None,
                                          C.byref(vs) if vs is not None else None,
                                          _dtype_code(key), layout, _stream(stream))
    _check(rc, "vmc_reshape_and_cache_fp8")


def convert_fp8(dst, src, scale, e5m2=False, stream=None):
    """vmc_convert_fp8: dst (uint8, src.numel() bytes) = fp8(src * scale)."""
    rc = load().vmc_convert_fp8(_ptr(dst), _ptr(src), float(scale), src.numel(), int(bool(e5m2)),
                                _dtype_code(src), _stream(stream))
    _check(rc, "vmc_convert_fp8")


def paged_decode_workspace_size(batch, num_heads, num_kv_heads, head_dim=128, max_blocks=0,
                                block_size=16, max_splits=0):
    return int(load().vmc_paged_decode_workspace_size(batch, num_heads, num_kv_heads, head_dim,
                                                      max_blocks, block_size, max_splits))


def paged_attention_decode(out, query, key_cache, value_cache, block_tables, seq_lens,
                           num_kv_heads, scale, block_size=16, kv_format=KV_F16,
                           layout=LAYOUT_NHD, workspace=None, max_splits=0, stream=None):
    import torch
    B, Hq, D = query.shape
    max_blocks = block_tables.shape[1]
    ws_bytes = paged_decode_workspace_size(B, Hq, num_kv_heads, D, max_blocks, block_size, max_splits)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=query.device)
    rc = load().vmc_paged_attention_decode(
        _ptr(out), _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
        _ptr(seq_lens), B, Hq, num_kv_heads, D, block_size, max_blocks, scale,
        _dtype_code(query), kv_format, layout, max_splits, _ptr(workspace),
        workspace.numel() * workspace.element_size(), _stream(stream))
    _check(rc, "vmc_paged_attention_decode")
    return out


def turboquant_store(key, value, kv_cache, slot_mapping, block_size, cfg, stream=None):
    T, H, D = key.shape
    rc = load().vmc_turboquant_store(_ptr(key), _ptr(value), _ptr(kv_cache), _ptr(slot_mapping),
                                     T, H, D, block_size, C.byref(cfg), _dtype_code(key),
                                     _stream(stream))
    _check(rc, "vmc_turboquant_store")


def turboquant_decode_workspace_size(batch, num_heads, num_kv_heads, head_dim=128, max_blocks=0,
                                     block_size=16, max_splits=0):
    return int(load().vmc_turboquant_decode_workspace_size(batch, num_heads, num_kv_heads, head_dim,
                                                           max_blocks, block_size, max_splits))


def turboquant_decode_attention(out, query, kv_cache, block_tables, seq_lens, num_kv_heads, scale,
                                cfg, block_size=16, workspace=None, max_splits=0, stream=None):
    import torch
    B, Hq, D = query.shape
    max_blocks = block_tables.shape[1]
    ws_bytes = turboquant_decode_workspace_size(B, Hq, num_kv_heads, D, max_blocks, block_size,
                                                max_splits)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=query.device)
    rc = load().vmc_turboquant_decode_attention(
        _ptr(out), _ptr(query), _ptr(kv_cache), _ptr(block_tables), _ptr(seq_lens), B, Hq,
        num_kv_heads, D, scale, block_size, max_blocks, C.byref(cfg), _dtype_code(query),
        max_splits, _ptr(workspace), workspace.numel() * workspace.element_size(),
        _stream(stream))
    _check(rc, "vmc_turboquant_decode_attention")
    return out


def turboquant_decode_attention_noalloc(out, query, kv_cache, block_tables, seq_lens, num_kv_heads,
                                        scale, cfg, block_size=16, max_splits=0, stream=None):
    """vmc_turboquant_decode_attention_noalloc: the split partials go to the
    library's own device array (nothing is allocated by the call)."""
    B, Hq, D = query.shape
    rc = load().vmc_turboquant_decode_attention_noalloc(
        _ptr(out), _ptr(query), _ptr(kv_cache), _ptr(block_tables), _ptr(seq_lens), B, Hq,
        num_kv_heads, D, scale, block_size, block_tables.shape[1], C.byref(cfg), _dtype_code(query),
        max_splits, _stream(stream))
    _check(rc, "vmc_turboquant_decode_attention_noalloc")
    return out


def flash_attention_prefill_workspace_size(num_tokens, num_kv_heads, head_dim=128):
    return load().vmc_flash_attention_prefill_workspace_size(num_tokens, num_kv_heads, head_dim)


def flash_attention_prefill(out, query, key, value, token_positions, num_kv_heads, scale,
                            key_cache=None, value_cache=None, slot_mapping=None, block_size=16,
                            kv_format=KV_Q8_0, layout=LAYOUT_NHD, stream=None, workspace=None):
    """vmc_flash_attention_prefill; with a workspace (a uint8 device tensor of
    at least flash_attention_prefill_workspace_size bytes),
    vmc_flash_attention_prefill_ws (V^T tiles built once per call)."""
    T, Hq, D = query.shape
    args = (_ptr(out), _ptr(query), _ptr(key), _ptr(value), T, Hq, num_kv_heads, D, scale,
            _ptr(token_positions), _dtype_code(query), _ptr(key_cache), _ptr(value_cache),
            _ptr(slot_mapping), block_size, kv_format, layout)
    if workspace is None:
        rc = load().vmc_flash_attention_prefill(*args, _stream(stream))
        _check(rc, "vmc_flash_attention_prefill")
    else:
        rc = load().vmc_flash_attention_prefill_ws(*args, _ptr(workspace), workspace.numel() * workspace.element_size(),
                                                   _stream(stream))
        _check(rc, "vmc_flash_attention_prefill_ws")
    return out


def hbm_read_probe(buf, mode, sink=None, stream=None):
    """One streaming read of the whole buffer (measurement): mode 0 vector
    loads into registers, mode 1 non-temporal load-to-LDS transfers, mode 2
    the decode's load-to-LDS transfers."""
    rc = load().vmc_hbm_read_probe(_ptr(buf), buf.numel() * buf.element_size(), mode, _ptr(sink),
                                   _stream(stream))
    _check(rc, "vmc_hbm_read_probe")


def fused_qk_norm_rope_store(q, k, v, q_norm_weight, k_norm_weight, cos_sin_cache, position_ids,
                             key_cache=None, value_cache=None, slot_mapping=None, block_size=16,
                             eps=1e-6, is_neox=True, kv_format=KV_F16, layout=LAYOUT_NHD,
                             cache_stride=0, tq_cfg=None, stream=None):
    """q [T][Hq][D], k, v [T][Hkv][D] (q, k updated in place); key_cache None:
    norm + RoPE only; tq_cfg given: TurboQuant slots in key_cache."""
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    rc = load().vmc_fused_qk_norm_rope_store(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_weight), _ptr(k_norm_weight), _ptr(cos_sin_cache),
        _ptr(position_ids), _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), T, Hq, Hkv, D,
        eps, int(bool(is_neox)), block_size, cache_stride, kv_format, layout,
        None if tq_cfg is None else C.byref(tq_cfg), _dtype_code(q), _stream(stream))
    _check(rc, "vmc_fused_qk_norm_rope_store")


def paged_attention_prefill(out, query, key_cache, value_cache, block_tables, token_to_seq,
                            token_positions, num_kv_heads, scale, block_size=16, kv_format=KV_F16,
                            layout=LAYOUT_NHD, workspace=None, max_splits=1, stream=None):
    """query/out [T][Hq][D]: token t attends positions 0 .. token_positions[t] of
    sequence token_to_seq[t] in the paged cache."""
    import torch
    T, Hq, D = query.shape
    max_blocks = block_tables.shape[1]
    ws_bytes = paged_decode_workspace_size(T, Hq, num_kv_heads, D, max_blocks, block_size, max_splits)
    if workspace is None and ws_bytes > 0:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
    rc = load().vmc_paged_attention_prefill(
        _ptr(out), _ptr(query), _ptr(key_cache), _ptr(value_cache), T, Hq, num_kv_heads, D, scale,
        block_size, max_blocks, _ptr(block_tables), _ptr(token_to_seq), _ptr(token_positions),
        _dtype_code(query), kv_format, layout, max_splits, _ptr(workspace),
        0 if workspace is None else workspace.numel() * workspace.element_size(), _stream(stream))
    _check(rc, "vmc_paged_attention_prefill")
    return out


def flash_attention_prefill_v2(out, query, key_cache, value_cache, block_tables, token_to_seq,
                               token_positions, num_kv_heads, scale, block_size=16, kv_format=KV_F16,
                               layout=LAYOUT_NHD, seq_lens=None, stream=None):
    """Tiled MFMA prefill over the paged cache: token t attends positions
    0 .. token_positions[t] of sequence token_to_seq[t] (block_tables
    [num_reqs][max_blocks]); query/out [T][Hq][D]."""
    T, Hq, D = query.shape
    num_reqs, max_blocks = block_tables.shape
    rc = load().vmc_flash_attention_prefill_v2(
        _ptr(out), _ptr(query), _ptr(key_cache), _ptr(value_cache), T, Hq, num_kv_heads, D, scale,
        block_size, max_blocks, _ptr(block_tables), _ptr(seq_lens), _ptr(token_to_seq),
        _ptr(token_positions), num_reqs, _dtype_code(query), kv_format, layout, _stream(stream))
    _check(rc, "vmc_flash_attention_prefill_v2")
    return out


def turboquant_prefill_attention(out, query, kv_cache, block_tables, token_to_seq, token_positions,
                                 num_kv_heads, scale, cfg, block_size=16, stream=None):
    """Token t attends positions 0 .. token_positions[t] of its sequence over
    the packed slots (cached prefix + appended step): steps of 16 tokens or
    more over codebook slots (head_dim 128) take the tiled prefill, others
    one decode row per token."""
    T, Hq, D = query.shape
    rc = load().vmc_turboquant_prefill_attention(
        _ptr(out), _ptr(query), _ptr(kv_cache), _ptr(block_tables), _ptr(token_to_seq),
        _ptr(token_positions), T, Hq, num_kv_heads, D, scale, block_size, block_tables.shape[1],
        C.byref(cfg), _dtype_code(query), 1, None, 0, _stream(stream))
    _check(rc, "vmc_turboquant_prefill_attention")
    return out


def batch_token_rows(row_seq, row_pos, token_to_seq, token_positions, seq_lens, stream=None):
    """Per-token (sequence, position) rows of an Engine step whose
    token_to_seq / token_positions hold only the prefill tokens' entries
    (decode tokens 0 / 0); seq_lens is per request."""
    rc = load().vmc_batch_token_rows(_ptr(row_seq), _ptr(row_pos), _ptr(token_to_seq), _ptr(token_positions),
                                     _ptr(seq_lens), token_to_seq.numel(), seq_lens.numel(), _stream(stream))
    _check(rc, "vmc_batch_token_rows")
