"""CPU checks of the C ABI library: it loads, exports every symbol the header
declares, and its host-only entry points behave (no GPU calls here)."""
import ctypes as C
import os
import re

import numpy as np

import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "vmc_attn.h")).read()
    return sorted(set(re.findall(r"\b(vmc_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from vm_c_amd import capi
    lib = capi.load()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(capi.EXPORTS) <= set(_declared())


def test_version():
    from vm_c_amd import capi
    assert "gfx950" in capi.version()


def test_entry_bytes():
    from vm_c_amd import capi
    assert capi.kv_entry_bytes(capi.KV_F16, 128) == 256
    assert capi.kv_entry_bytes(capi.KV_Q8_0, 128) == 136
    assert capi.kv_entry_bytes(capi.KV_Q4_0, 128) == 72
    assert capi.kv_entry_bytes(7, 128) < 0


def test_tq_config_layouts():
    """Slot sizes held by the reference: 134 / 102 / 118 B for head_dim 128
    (src/distributed/tp_runtime.cpp:257-261, kernels_turboquant.h:29-42)."""
    from vm_c_amd import capi
    exp = {"turboquant_4bit_nc": (64, 66, 64, 68, 134), "turboquant_3bit_nc": (48, 50, 48, 52, 102),
           "turboquant_k3v4_nc": (48, 50, 64, 68, 118)}
    for m, (mse, kp, vd, vp, slot) in exp.items():
        c = capi.tq_config(128, m)
        assert (c.mse_bytes, c.key_packed_size, c.val_data_bytes, c.value_packed_size,
                c.slot_size_aligned) == (mse, kp, vd, vp, slot)
        L = O.tq_layout(m)
        assert L.slot_size_aligned == slot
    assert capi.tq_config(256, "turboquant_4bit_nc").slot_size_aligned == 262
    # fp8 keys (turboquant_k8v4): 128 key bytes, no norm, 4-bit values
    c8 = capi.tq_config(128, "turboquant_k8v4")
    L8 = O.tq_layout("turboquant_k8v4")
    assert c8.slot_size_aligned == L8.slot_size_aligned == 196
    assert c8.key_fp8 == L8.key_fp8 == 1 and c8.fp8_e4b15 == 0 and c8.key_packed_size == 128


def test_g32_config_layouts():
    """The per-32-group variant (no reference counterpart): K and V parts of
    four blocks, 2 x 80 B (4-bit: fp16 scale + fp16 min + 16 B) and 2 x 56 B
    (3-bit: fp16 scale + 12 B), matching the oracle's part sizes."""
    from vm_c_amd import capi
    for m, bits, part in (("turboquant_4bit_g32", 4, 80), ("turboquant_3bit_g32", 3, 56)):
        c = capi.tq_config(128, m, sign_seed=7)
        assert (c.group_size, c.key_quant_bits, c.value_quant_bits) == (32, bits, bits)
        assert (c.key_packed_size, c.value_packed_size, c.slot_size_aligned) == (part, part, 2 * part)
        assert c.sign_seed == 7 and c.n_centroids == 0
        assert O.g32_part_bytes(bits) == part
    import pytest
    with pytest.raises(capi.VmcError):
        capi.tq_config(64, "turboquant_4bit_g32")


def test_tq_host_tables_match_oracle():
    from vm_c_amd import capi
    for bits in (3, 4):
        c, m = capi.tq_host_tables(128, bits)
        oc, om = O.tq_tables(128, bits)
        assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(m.view(np.uint32), om.view(np.uint32))


def test_argument_validation_without_gpu():
    """Invalid shapes are rejected before any device work."""
    from vm_c_amd import capi
    L = capi.load()
    # head_dim not a multiple of 32
    assert L.vmc_reshape_and_cache(None, None, None, None, None, 1, 1, 100, 16, 0, 0, 0, 0, None) == capi.VMC_EINVAL
    # zero tokens is a no-op
    assert L.vmc_reshape_and_cache(None, None, None, None, None, 0, 1, 128, 16, 0, 0, 0, 0, None) == capi.VMC_OK
    # decode: GQA group > 16 rejected
    assert L.vmc_paged_attention_decode(None, None, None, None, None, None, 1, 64, 2, 128, 16, 4,
                                        C.c_float(0.1), 0, 0, 0, 0, None, 0, None) == capi.VMC_EINVAL
    # decode: workspace too small
    assert L.vmc_paged_attention_decode(C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), C.c_void_p(16),
                                        C.c_void_p(16), C.c_void_p(16), 1, 8, 8, 128, 16, 4,
                                        C.c_float(0.1), 0, 0, 0, 0, C.c_void_p(16), 8, None) == capi.VMC_ENOMEM


def test_null_and_stride_validation_without_gpu():
    """Null buffers and too-small page strides are rejected before any launch:
    the fp8-key TurboQuant store checks its pointers like every other method,
    and the fused norm/RoPE append checks the page stride and the 16-byte
    alignment of f16/bf16 pages as vmc_reshape_and_cache does."""
    from vm_c_amd import capi
    L = capi.load()
    c8 = capi.tq_config(128, "turboquant_k8v4")
    p = C.c_void_p(256)
    for key, val, cache, slots in ((None, p, p, p), (p, None, p, p), (p, p, None, p), (p, p, p, None)):
        assert L.vmc_turboquant_store(key, val, cache, slots, 4, 8, 128, 16, C.byref(c8), 0,
                                      None) == capi.VMC_EINVAL
    fused = L.vmc_fused_qk_norm_rope_store
    args = lambda stride, fmt: (p, p, p, None, None, p, p, p, p, p, 4, 32, 8, 128, C.c_float(1e-6), 1,
                                16, stride, fmt, 0, None, 0, None)
    # one page of 16 tokens x 8 heads of 136-byte q8_0 entries needs 17408 bytes
    assert fused(*args(17407, capi.KV_Q8_0)) == capi.VMC_EINVAL
    # f16 pages are written 16 bytes at a time
    assert fused(*args(16 * 8 * 256 + 8, capi.KV_F16)) == capi.VMC_EINVAL


def test_tq_configs_other_head_dims():
    """head_dim 64 and 256 (TQConfig::kMaxSupportedHeadDim = 256,
    kernels_turboquant.h:11): slot sizes from compute_layout, the reference's
    262-byte 4-bit slot at 256 (tp_runtime.cpp:257-261), fp8-key slots of
    head_dim + head_dim / 2 + 4 bytes, and the host codebooks equal to the
    oracle's."""
    from vm_c_amd import capi
    assert capi.tq_config(256, "turboquant_4bit_nc").slot_size_aligned == 262
    for d in (64, 256):
        for m in ("turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc", "turboquant_k8v4"):
            c = capi.tq_config(d, m)
            L = O.tq_layout(m, d)
            assert (c.mse_bytes, c.key_packed_size, c.val_data_bytes, c.slot_size_aligned) == \
                   (L.mse_bytes, L.key_packed_size, L.val_data_bytes, L.slot_size_aligned)
        assert capi.tq_config(d, "turboquant_k8v4").slot_size_aligned == d + d // 2 + 4
        for bits in (3, 4):
            c, m = capi.tq_host_tables(d, bits)
            oc, om = O.tq_tables(d, bits)
            assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
            assert np.array_equal(m.view(np.uint32), om.view(np.uint32))
