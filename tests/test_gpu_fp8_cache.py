"""fp8 pages on the GPU: vmc_reshape_and_cache_fp8 (reshape_and_cache with
kv_cache_dtype "fp8_e4m3" / "fp8_e5m2", cache_kernels.cu:101-131) and
vmc_convert_fp8 (convert_fp8, cache_kernels.cu:175-212), every byte equal
to the oracle's restatement of the OCP FP8 conversion (which
tests/test_oracle_ofp8.py pins by exhaustive search).  Inputs hold values
past the saturation limits, below the smallest subnormal and at exact
rounding midpoints; a negative slot, NHD and HND, a padded block stride,
fp16 and bf16 sources."""
import numpy as np
import pytest

import oracle_lib as O
from kvgen import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _bits(x, bf16):
    with np.errstate(over="ignore"):  # values past fp16's range become inf on purpose
        return f32_to_bf16_bits(x) if bf16 else np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _dev(dev, bits, bf16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(
        torch.bfloat16 if bf16 else torch.float16)


def _values(rng, shape):
    x = (rng.standard_normal(shape) * 40).astype(np.float32)
    flat = x.reshape(-1)
    special = np.array([1e5, -1e5, 448.0, 464.0, 480.0, 1e-7, -1e-7, 2.0 ** -10, 3 * 2.0 ** -10,
                        0.0, -0.0, 60000.0, 57344.0, 2.0 ** -17], np.float32)
    flat[:special.size] = special
    return x


@pytest.mark.parametrize("hnd", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("scales", [(None, None), (0.5, 3.0)])
def test_reshape_and_cache_fp8(dev, hnd, bf16, scales):
    import torch
    from vm_c_amd import capi
    T, H, D, bs, nblk = 301, 8, 128, 16, 24
    rng = np.random.default_rng(7 + hnd + 2 * bf16)
    kb, vb = _bits(_values(rng, (T, H, D)), bf16), _bits(_values(rng, (T, H, D)), bf16)
    stride = bs * H * D + 256
    slots = rng.permutation(nblk * bs)[:T].astype(np.int64)
    slots[9] = -1
    kc = torch.full((nblk * stride,), 0x5A, dtype=torch.uint8, device=dev)
    vc = torch.full_like(kc, 0x5A)
    print(f"fp8 append hnd={hnd} bf16={bf16} scales={scales}", flush=True)
    capi.reshape_and_cache_fp8(_dev(dev, kb, bf16), _dev(dev, vb, bf16), kc, vc, torch.from_numpy(slots).to(dev),
                               bs, k_scale=scales[0], v_scale=scales[1],
                               layout=capi.LAYOUT_HND if hnd else capi.LAYOUT_NHD, cache_stride=stride)
    torch.cuda.synchronize()
    ek = np.full(nblk * stride, 0x5A, np.uint8)
    ev = np.full(nblk * stride, 0x5A, np.uint8)
    O.reshape_and_cache_fp8(kb, vb, slots, ek, ev, bs, k_scale=scales[0] or 1.0, v_scale=scales[1] or 1.0,
                            hnd=hnd, src_bf16=bf16, stride=stride)
    gk, gv = kc.cpu().numpy(), vc.cpu().numpy()
    for name, g, e in (("K", gk, ek), ("V", gv, ev)):
        bad = np.flatnonzero(g != e)
        assert bad.size == 0, f"{name} pages differ at {bad.size} bytes (first {bad[:4]}: {g[bad[:4]]} vs {e[bad[:4]]})"


@pytest.mark.parametrize("e5m2", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("n,offset", [(1 << 16, 0), (1003, 0), (4097, 1)])
def test_convert_fp8(dev, e5m2, bf16, n, offset):
    """A whole run (16 values per thread), a ragged one, and an unaligned one
    (one value per thread)."""
    import torch
    from vm_c_amd import capi
    rng = np.random.default_rng(n + e5m2)
    x = (rng.standard_normal(n + offset) * (3e4 if e5m2 else 300)).astype(np.float32)
    x[offset:offset + 6] = [np.inf, -np.inf, 1e9, 2.0 ** -20, 0.0, -0.0]
    bits = _bits(x, bf16)
    src = _dev(dev, bits, bf16)[offset:]
    dst = torch.zeros(n + offset, dtype=torch.uint8, device=dev)[offset:]
    print(f"convert_fp8 e5m2={e5m2} bf16={bf16} n={n} offset={offset}", flush=True)
    capi.convert_fp8(dst, src, 0.75, e5m2=e5m2)
    torch.cuda.synchronize()
    exp = O.convert_fp8(bits[offset:], 0.75, e5m2=e5m2, src_bf16=bf16)
    got = dst.cpu().numpy()
    bad = np.flatnonzero(got != exp)
    assert bad.size == 0, f"{bad.size} bytes differ (first {bad[:4]}: {got[bad[:4]]} vs {exp[bad[:4]]})"
