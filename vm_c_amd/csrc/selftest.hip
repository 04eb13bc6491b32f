// selftest.hip -- device check of the lane-level assumptions the kernels rely
// on: cross-row reductions, the wave-private LDS gathers, the operand /
// result layouts of the MFMA shapes used (16x16x32 f16/bf16, 16x16x16 f16,
// 32x32x16 f16/bf16), exact fp16 subnormal operands in the 16x16x16 MFMA,
// the bf16 conversion instruction and the 16-lane DPP exchanges.  One wave,
// fixed inputs (small integers where arithmetic is checked), every lane
// compares its own results with the expected values.
#include "vmc_common.hpp"

namespace vmc {
namespace {

enum {
    kSumGroups = 1, kMaxGroups = 2, kGather = 4, kMfma16x32 = 8, kMfma16x16 = 16,
    kMfma32x16 = 32, kMfma16x32bf = 64, kMfma32x16bf = 128, kMfma16x16Subnormal = 256,
    kGatherDiag = 512, kMfma16x32Subnormal = 1024, kBf16Convert = 2048, kRowXor = 4096,
    kRowSum = 8192
};

// bf16 rounding cases: ties to even (both ways), a carry into the exponent,
// overflow to infinity, subnormals, signed zeros, NaN payloads, infinities
__constant__ uint32_t kBf16Cases[16] = {
    0x3f808000u, 0x3f818000u, 0x3f80ffffu, 0x7f7fffffu, 0x7f7f7fffu, 0x00018000u,
    0x80028000u, 0x007fffffu, 0x80000000u, 0x00000000u, 0x7fa00001u, 0xffc12345u,
    0x7f800001u, 0xff800000u, 0xc0490fdbu, 0x3eaaaaabu};

// A[i][k] = (i + 2k) % 5 - 2, B[k][j] = (3k + j) % 7 - 3 (all exact)
__device__ __forceinline__ float Aval(int i, int k) { return (float)((i + 2 * k) % 5 - 2); }
__device__ __forceinline__ float Bval(int k, int j) { return (float)((3 * k + j) % 7 - 3); }

__global__ void __launch_bounds__(64) selftest_kernel(int* fail) {
    __shared__ __attribute__((aligned(16))) float sc[16];
    const int l = threadIdx.x, r16 = l & 15, grp = l >> 4;
    int bad = 0;
    // cross-row reductions
    {
        const float s = sum_over_groups((float)l);
        if (s != (float)(4 * r16 + 96)) bad |= kSumGroups;
        const float m = max_over_groups((float)l);
        if (m != (float)(48 + r16)) bad |= kMaxGroups;
        const f32x4 g = gather4_from_row0((float)(100 + l), sc, r16, grp);
        for (int i = 0; i < 4; ++i)
            if (g[i] != (float)(100 + 4 * grp + i)) bad |= kGather;
        // diagonal lanes (grp == r16 / 4) publish row r16
        const f32x4 gd = gather4_from_diag((float)(200 + 16 * grp + r16), sc, r16, grp);
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * grp + i;
            if (gd[i] != (float)(200 + 16 * (row >> 2) + row)) bad |= kGatherDiag;
        }
    }
    // bf16 conversion instruction against the integer rule; 16-lane DPP
    // exchanges and the row sum against their definitions
    {
        const uint32_t c = kBf16Cases[r16];
        for (int v = 0; v < 2; ++v) {
            const float f = __builtin_bit_cast(float, v ? c ^ (uint32_t)(grp * 0x00011001u) : c);
            if (f32_to_bf16_bits(f) != f32_to_bf16_bits_int(f)) bad |= kBf16Convert;
        }
        const float x = (float)(1000 + l);
        if (row_xor<1>(x, l) != (float)(1000 + (l ^ 1)) || row_xor<2>(x, l) != (float)(1000 + (l ^ 2)) ||
            row_xor<4>(x, l) != (float)(1000 + (l ^ 4)) || row_xor<8>(x, l) != (float)(1000 + (l ^ 8)) ||
            row_xor<4>(l, l) != (l ^ 4))
            bad |= kRowXor;
        float ref = 0.0f;
        for (int i = 0; i < 16; ++i) ref += (float)(3 * (16 * grp + i) + 1);
        if (row_sum16((float)(3 * l + 1)) != ref) bad |= kRowSum;
    }
    // 16x16x32 f16: A lane (row l%16, k = 8*(l/16) + e), D rows 4*(l/16)+i, col l%16
    {
        f16x8 a, b;
        bf16x8 ab, bb;
        for (int e = 0; e < 8; ++e) {
            const int k = 8 * grp + e;
            a[e] = (_Float16)Aval(r16, k);
            b[e] = (_Float16)Bval(k, r16);
            ab[e] = (__bf16)Aval(r16, k);
            bb[e] = (__bf16)Bval(k, r16);
        }
        const f32x4 d = mfma16x16x32(a, b, f32x4{0.f, 0.f, 0.f, 0.f});
        const f32x4 db = mfma16x16x32(ab, bb, f32x4{0.f, 0.f, 0.f, 0.f});
        for (int i = 0; i < 4; ++i) {
            float ref = 0.0f;
            for (int k = 0; k < 32; ++k) ref += Aval(4 * grp + i, k) * Bval(k, r16);
            if (d[i] != ref) bad |= kMfma16x32;
            if (db[i] != ref) bad |= kMfma16x32bf;
        }
        // B as fp16 subnormals holding a 3-bit code shifted left by 0..7
        // (column r16 uses shift r16 % 8, so bit 9 is the highest set): the
        // value is code * 2^(shift - 24), products and sums exact
        f16x8 bs;
        const int sh = r16 & 7;
        for (int e = 0; e < 8; ++e) {
            const int k = 8 * grp + e;
            bs[e] = __builtin_bit_cast(_Float16, (uint16_t)(((3 * k + r16) % 8) << sh));
        }
        const f32x4 ds = mfma16x16x32(a, bs, f32x4{0.f, 0.f, 0.f, 0.f});
        for (int i = 0; i < 4; ++i) {
            float ref = 0.0f;
            for (int k = 0; k < 32; ++k) ref += Aval(4 * grp + i, k) * (float)((3 * k + r16) % 8);
            if (ds[i] * (float)(1 << (24 - sh)) != ref) bad |= kMfma16x32Subnormal;
        }
    }
    // 16x16x16 f16: k = 4*(l/16) + e
    {
        f16x4 a, b;
        for (int e = 0; e < 4; ++e) {
            const int k = 4 * grp + e;
            a[e] = (_Float16)Aval(r16, k);
            b[e] = (_Float16)Bval(k, r16);
        }
        const f32x4 d = mfma16x16x16(a, b, f32x4{0.f, 0.f, 0.f, 0.f});
        for (int i = 0; i < 4; ++i) {
            float ref = 0.0f;
            for (int k = 0; k < 16; ++k) ref += Aval(4 * grp + i, k) * Bval(k, r16);
            if (d[i] != ref) bad |= kMfma16x16;
        }
        // B given as fp16 subnormals (integer codes c as c * 2^-24): the
        // products and sums must stay exact, i.e. the unit does not flush them
        f16x4 bs;
        for (int e = 0; e < 4; ++e) {
            const int k = 4 * grp + e;
            bs[e] = __builtin_bit_cast(_Float16, (uint16_t)((3 * k + r16) % 8));
        }
        const f32x4 ds = mfma16x16x16(a, bs, f32x4{0.f, 0.f, 0.f, 0.f});
        for (int i = 0; i < 4; ++i) {
            float ref = 0.0f;
            for (int k = 0; k < 16; ++k) ref += Aval(4 * grp + i, k) * (float)((3 * k + r16) % 8);
            if (ds[i] * 16777216.0f != ref) bad |= kMfma16x16Subnormal;
        }
    }
    // 32x32x16: A lane (row l%32, k = 8*(l/32) + e), D col l%32, rows 8*(v/4) + 4*(l/32) + v%4
    {
        const int c32 = l & 31, h = l >> 5;
        f16x8 a, b;
        bf16x8 ab, bb;
        for (int e = 0; e < 8; ++e) {
            const int k = 8 * h + e;
            a[e] = (_Float16)Aval(c32, k);
            b[e] = (_Float16)Bval(k, c32);
            ab[e] = (__bf16)Aval(c32, k);
            bb[e] = (__bf16)Bval(k, c32);
        }
        f32x16 z;
        for (int v = 0; v < 16; ++v) z[v] = 0.0f;
        const f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, z, 0, 0, 0);
        const f32x16 db = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, bb, z, 0, 0, 0);
        for (int v = 0; v < 16; ++v) {
            const int row = 8 * (v >> 2) + 4 * h + (v & 3);
            float ref = 0.0f;
            for (int k = 0; k < 16; ++k) ref += Aval(row, k) * Bval(k, c32);
            if (d[v] != ref) bad |= kMfma32x16;
            if (db[v] != ref) bad |= kMfma32x16bf;
        }
    }
    atomicOr(fail, bad);
}

}  // namespace
}  // namespace vmc

// Returns 0 when every check passes, a bitmask of failed checks (> 0), or a
// negative status on a HIP error.  Synchronous; allocates 4 bytes.
extern "C" int vmc_selftest(void) {
    int* d = nullptr;
    if (hipMalloc(&d, sizeof(int)) != hipSuccess) return VMC_EIO;
    int h = 0;
    int rc = VMC_OK;
    if (hipMemset(d, 0, sizeof(int)) != hipSuccess) rc = VMC_EIO;
    if (rc == VMC_OK) {
        hipLaunchKernelGGL(vmc::selftest_kernel, dim3(1), dim3(64), 0, 0, d);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
            hipMemcpy(&h, d, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
            rc = VMC_EIO;
    }
    (void)hipFree(d);
    return rc == VMC_OK ? h : rc;
}
