/*
 * vmc_oracle.c -- CPU restatement of vm_c's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product path.  Built with -ffp-contract=off so every a*b+c below is two
 * roundings unless written as fmaf(): the CUDA reference was compiled by nvcc
 * with its default --fmad=true, so the places where nvcc contracted are
 * written as explicit fmaf() and cited.
 *
 * Parity status per function is recorded beside its declaration in vmc_oracle.h.
 */
#include "vmc_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                       */
/* ------------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const int shift = 14 - e;
        uint32_t hm = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            mant &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp + 127u - 15u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    const uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_n(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

static inline float half_to_f32(uint16_t h, int bf16) {
    return bf16 ? orc_bf16_to_f32(h) : orc_f16_to_f32(h);
}
static inline uint16_t f32_to_half(float f, int bf16) {
    return bf16 ? orc_f32_to_bf16(f) : orc_f32_to_f16(f);
}

/* ------------------------------------------------------------------------ */
/* GGUF q8_0 / q4_0                                                         */
/* ------------------------------------------------------------------------ */

enum { QK = 32, Q8_0_BYTES = 34, Q4_0_BYTES = 18 };

/* ggml/src/ggml-quants.c:234-257 (quantize_row_q8_0_ref): d = amax/127,
 * id = d ? 1/d : 0, qs = roundf(x*id) (half away from zero), d stored fp16. */
void orc_quantize_row_q8_0(const float* x, void* yv, int64_t k) {
    uint8_t* y = (uint8_t*)yv;
    for (int64_t i = 0; i < k / QK; ++i) {
        const float* xb = x + i * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        uint8_t* blk = y + i * Q8_0_BYTES;
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < QK; ++j) blk[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
    }
}

/* ggml/src/ggml-quants.c:491-503 */
void orc_dequantize_row_q8_0(const void* xv, float* y, int64_t k) {
    const uint8_t* x = (const uint8_t*)xv;
    for (int64_t i = 0; i < k / QK; ++i) {
        const uint8_t* blk = x + i * Q8_0_BYTES;
        const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < QK; ++j) y[i * QK + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* ggml/src/ggml-quants.c:71-104 (quantize_row_q4_0_ref): max = signed value of
 * largest |x| (first wins), d = max/-8, q = min(15, (int8_t)(x*id + 8.5f)),
 * qs[j] = q[j] | q[j+16] << 4.  x*id and +8.5f are separate roundings (the
 * ggml CPU build has no FMA). */
void orc_quantize_row_q4_0(const float* x, void* yv, int64_t k) {
    uint8_t* y = (uint8_t*)yv;
    for (int64_t i = 0; i < k / QK; ++i) {
        const float* xb = x + i * QK;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float v = xb[j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        uint8_t* blk = y + i * Q4_0_BYTES;
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < QK / 2; ++j) {
            volatile float x0 = xb[j] * id;
            volatile float x1 = xb[QK / 2 + j] * id;
            const int8_t t0 = (int8_t)(x0 + 8.5f);
            const int8_t t1 = (int8_t)(x1 + 8.5f);
            const uint8_t q0 = (uint8_t)(t0 < 15 ? t0 : 15);
            const uint8_t q1 = (uint8_t)(t1 < 15 ? t1 : 15);
            blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* ggml/src/ggml-quants.c:397-414 */
void orc_dequantize_row_q4_0(const void* xv, float* y, int64_t k) {
    const uint8_t* x = (const uint8_t*)xv;
    for (int64_t i = 0; i < k / QK; ++i) {
        const uint8_t* blk = x + i * Q4_0_BYTES;
        const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < QK / 2; ++j) {
            y[i * QK + j] = (float)((blk[2 + j] & 0x0f) - 8) * d;
            y[i * QK + QK / 2 + j] = (float)((blk[2 + j] >> 4) - 8) * d;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* paged KV (src/cuda/cache_kernels.cu:14-54 addressing; q8_0/q4_0 rows as  */
/* written by ggml_set_rows, ggml/src/ggml-cpu/ops.cpp:4950-5020)           */
/* ------------------------------------------------------------------------ */

int64_t orc_kv_entry_bytes(int fmt, int head_dim) {
    switch (fmt) {
        case ORC_KV_F16:
        case ORC_KV_BF16: return (int64_t)head_dim * 2;
        case ORC_KV_Q8_0: return (int64_t)(head_dim / QK) * Q8_0_BYTES;
        case ORC_KV_Q4_0: return (int64_t)(head_dim / QK) * Q4_0_BYTES;
        default: return -1;
    }
}

static inline int64_t kv_entry_offset(int64_t slot, int h, int64_t bs, int Hkv,
                                      int64_t E, int hnd) {
    const int64_t blk = slot / bs, off = slot % bs;
    const int64_t stride = bs * Hkv * E;
    return hnd ? blk * stride + (int64_t)h * bs * E + off * E
               : blk * stride + off * Hkv * E + (int64_t)h * E;
}

static void encode_entry(const uint16_t* src, int src_bf16, uint8_t* dst, int fmt,
                         int D, float* tmp) {
    if (fmt == ORC_KV_F16 || fmt == ORC_KV_BF16) {
        uint16_t* d16 = (uint16_t*)dst;
        for (int d = 0; d < D; ++d) {
            const float v = half_to_f32(src[d], src_bf16);
            /* same-type copy is a bit copy (cache_kernels.cu:49-50) */
            d16[d] = ((fmt == ORC_KV_BF16) == (src_bf16 != 0)) ? src[d]
                                                               : f32_to_half(v, fmt == ORC_KV_BF16);
        }
        return;
    }
    for (int d = 0; d < D; ++d) tmp[d] = half_to_f32(src[d], src_bf16);
    if (fmt == ORC_KV_Q8_0) orc_quantize_row_q8_0(tmp, dst, D);
    else orc_quantize_row_q4_0(tmp, dst, D);
}

void orc_kv_append(const uint16_t* key, const uint16_t* value, int src_bf16,
                   uint8_t* key_cache, uint8_t* value_cache,
                   const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                   int head_dim, int64_t block_size, int fmt, int hnd) {
    const int64_t E = orc_kv_entry_bytes(fmt, head_dim);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
    for (int t = 0; t < num_tokens; ++t) {
        const int64_t slot = slot_mapping[t];
        if (slot < 0) continue; /* cache_kernels.cu:26 */
        for (int h = 0; h < num_kv_heads; ++h) {
            const int64_t src = ((int64_t)t * num_kv_heads + h) * head_dim;
            const int64_t off = kv_entry_offset(slot, h, block_size, num_kv_heads, E, hnd);
            encode_entry(key + src, src_bf16, key_cache + off, fmt, head_dim, tmp);
            encode_entry(value + src, src_bf16, value_cache + off, fmt, head_dim, tmp);
        }
    }
    free(tmp);
}

/* OCP OFP8 v1.0 (E4M3: 3 mantissa bits, bias 7, max 448 = 0x7e; E5M2: 2
 * mantissa bits, bias 15, max 57344 = 0x7b), round to nearest even with
 * saturation to the largest finite value; see the header. */
uint8_t orc_f32_to_ofp8(float x, int e5m2) {
    const int M = e5m2 ? 2 : 3, B = e5m2 ? 15 : 7;
    const float maxv = e5m2 ? 57344.0f : 448.0f;
    const uint8_t maxc = e5m2 ? 0x7b : 0x7e;
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint8_t s = (uint8_t)((u >> 31) << 7);
    if (isnan(x)) return 0x7f;
    if (fabsf(x) >= maxv) return (uint8_t)(s | maxc);
    const uint32_t a = u & 0x7fffffffu;
    const int E = (int)(a >> 23) - 127;
    const uint32_t man = a & 0x7fffffu;
    if (E >= 1 - B) { /* normal: keep M mantissa bits, a carry moves into the exponent */
        const int sh = 23 - M;
        const uint32_t q = man >> sh, rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
        const uint32_t up = rem > half || (rem == half && (q & 1u));
        return (uint8_t)(s | ((((uint32_t)(E + B)) << M) + q + up));
    }
    if (a < 0x00800000u) return s; /* zero and fp32 subnormals (far below the fp8 quantum) */
    /* subnormal: multiples of 2^(1 - B - M) */
    const uint32_t sig = man | 0x800000u;
    const int sh = 24 - B - M - E; /* value / quantum = sig >> sh */
    if (sh >= 32) return s;
    const uint32_t q = sig >> sh, rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
    const uint32_t up = rem > half || (rem == half && (q & 1u));
    return (uint8_t)(s | (q + up));
}

void orc_f32_to_ofp8_n(const float* x, uint8_t* y, int64_t n, int e5m2) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_ofp8(x[i], e5m2);
}

float orc_ofp8_to_f32(uint8_t b, int e5m2) {
    const int M = e5m2 ? 2 : 3, B = e5m2 ? 15 : 7;
    const float sg = (b & 0x80) ? -1.0f : 1.0f;
    const int e = (b & 0x7f) >> M, m = b & ((1 << M) - 1);
    if (e5m2 && e == 31) return m ? NAN : sg * INFINITY;
    if (!e5m2 && e == 15 && m == 7) return NAN;
    if (e == 0) return sg * ldexpf((float)m, 1 - B - M);
    return sg * ldexpf((float)((1 << M) + m), e - B - M);
}

void orc_reshape_and_cache_fp8(const uint16_t* key, const uint16_t* value, int src_bf16,
                               uint8_t* key_cache, uint8_t* value_cache,
                               const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                               int head_dim, int64_t block_size, int64_t stride, float k_scale,
                               float v_scale, int hnd) {
    const int64_t E = head_dim;
    if (stride <= 0) stride = block_size * num_kv_heads * E;
    for (int t = 0; t < num_tokens; ++t) {
        const int64_t slot = slot_mapping[t];
        if (slot < 0) continue; /* cache_kernels.cu:26 */
        const int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < num_kv_heads; ++h) {
            const int64_t src = ((int64_t)t * num_kv_heads + h) * head_dim;
            /* cache_kernels.cu:36-40 */
            const int64_t dst = hnd ? blk * stride + (int64_t)h * block_size * E + off * E
                                    : blk * stride + off * num_kv_heads * E + (int64_t)h * E;
            for (int d = 0; d < head_dim; ++d) { /* cache_kernels.cu:42-46 */
                key_cache[dst + d] = orc_f32_to_ofp8(half_to_f32(key[src + d], src_bf16) / k_scale, 0);
                value_cache[dst + d] = orc_f32_to_ofp8(half_to_f32(value[src + d], src_bf16) / v_scale, 0);
            }
        }
    }
}

void orc_convert_fp8(uint8_t* dst, const uint16_t* src, int src_bf16, float scale, int64_t n, int e5m2) {
    for (int64_t i = 0; i < n; ++i) /* cache_kernels.cu:181-184 */
        dst[i] = orc_f32_to_ofp8(half_to_f32(src[i], src_bf16) * scale, e5m2);
}

void orc_kv_dequant_entry(const uint8_t* e, int fmt, int D, float* out) {
    if (fmt == ORC_KV_F16 || fmt == ORC_KV_BF16) {
        for (int d = 0; d < D; ++d) {
            const uint16_t h = (uint16_t)(e[2 * d] | (e[2 * d + 1] << 8));
            out[d] = half_to_f32(h, fmt == ORC_KV_BF16);
        }
    } else if (fmt == ORC_KV_Q8_0) {
        orc_dequantize_row_q8_0(e, out, D);
    } else {
        orc_dequantize_row_q4_0(e, out, D);
    }
}

/* ------------------------------------------------------------------------ */
/* TurboQuant                                                               */
/* ------------------------------------------------------------------------ */

/* include/vm_c/cuda/kernels_turboquant.h:29-74 (compute_layout/from_method);
 * include/vm_c/memory/kv_cache_manager.hpp:121-162.  Only the codebook
 * methods are restated here (k8v4 stores fp8 keys). */
int orc_tq_layout_from_method(int head_dim, const char* method, orc_tq_layout* L) {
    memset(L, 0, sizeof(*L));
    L->head_dim = head_dim;
    L->norm_correction = 1;
    if (method && strcmp(method, "turboquant_k8v4") == 0) {
        /* kernels_turboquant.h:47-55: fp8 keys, 4-bit values, no norm
         * correction; e4m3 on devices with fp8 support (the flag is the
         * caller's to change) */
        L->key_quant_bits = 8; L->value_quant_bits = 4;
        L->norm_correction = 0;
        L->key_fp8 = 1;
    } else if (method && strcmp(method, "turboquant_k3v4_nc") == 0) {
        L->key_quant_bits = 3; L->value_quant_bits = 4;
    } else if (method && strcmp(method, "turboquant_3bit_nc") == 0) {
        L->key_quant_bits = 3; L->value_quant_bits = 3;
    } else if (!method || strcmp(method, "turboquant_4bit_nc") == 0 ||
               strcmp(method, "") == 0) {
        L->key_quant_bits = 4; L->value_quant_bits = 4;
    } else {
        return -1;
    }
    /* compute_layout, kernels_turboquant.h:29-42 */
    L->n_centroids = 1 << L->key_quant_bits;
    L->mse_bytes = L->key_fp8 ? head_dim : (head_dim * L->key_quant_bits + 7) / 8;
    L->key_packed_size = L->key_fp8 ? head_dim : L->mse_bytes + 2;
    L->val_data_bytes = (head_dim * L->value_quant_bits + 7) / 8;
    L->value_packed_size = L->val_data_bytes + 4;
    L->slot_size = L->key_packed_size + L->value_packed_size;
    L->slot_size_aligned = L->slot_size + (L->slot_size % 2);
    return 0;
}

/* src/cuda/turboquant_kernels.cu:551-570 (build_hadamard_on_host): Sylvester
 * doubling, then every entry times 1.0f/sqrtf(d). */
void orc_tq_hadamard(float* out, int d) {
    const float inv_sqrt_d = 1.0f / sqrtf((float)d);
    for (int i = 0; i < d; ++i)
        for (int j = 0; j < d; ++j)
            out[i * d + j] = (__builtin_popcount((unsigned)(i & j)) & 1) ? -inv_sqrt_d : inv_sqrt_d;
}

/* src/cuda/turboquant_kernels.cu:572-576 */
static float gaussian_pdf(float x, float sigma2) {
    return (1.0f / sqrtf(2.0f * 3.14159265358979f * sigma2)) * expf(-x * x / (2.0f * sigma2));
}

/* src/cuda/turboquant_kernels.cu:578-623 (solve_lloyd_max_centroids): N(0,1/d)
 * Lloyd-Max, init uniform centres on [-3.5s, 3.5s], outer edges +-10.5s,
 * 201-point trapezoid per cell, <= 200 iterations, tolerance 1e-10, sorted. */
void orc_tq_lloyd_max(float* centroids_out, int d, int bits) {
    const int n = 1 << bits;
    const float sigma2 = 1.0f / (float)d;
    const float sigma = sqrtf(sigma2);
    const float lo = -3.5f * sigma, hi = 3.5f * sigma;
    float c[256], nc[256], edges[257];
    for (int i = 0; i < n; ++i) c[i] = lo + (hi - lo) * ((float)i + 0.5f) / (float)n;
    for (int iter = 0; iter < 200; ++iter) {
        edges[0] = lo * 3.0f;
        for (int i = 0; i < n - 1; ++i) edges[i + 1] = (c[i] + c[i + 1]) * 0.5f;
        edges[n] = hi * 3.0f;
        int converged = 1;
        for (int i = 0; i < n; ++i) {
            const int n_trap = 200;
            const float a = edges[i], b = edges[i + 1];
            const float step = (b - a) / (float)n_trap;
            float num = 0.0f, den = 0.0f;
            for (int j = 0; j <= n_trap; ++j) {
                const float x = a + (float)j * step;
                const float p = gaussian_pdf(x, sigma2);
                const float w = (j == 0 || j == n_trap) ? 0.5f : 1.0f;
                den += w * p;
                num += w * x * p;
            }
            num *= step;
            den *= step;
            nc[i] = (den > 1e-15f) ? num / den : c[i];
            if (fabsf(nc[i] - c[i]) > 1e-10f) converged = 0;
        }
        memcpy(c, nc, sizeof(float) * (size_t)n);
        if (converged) break;
    }
    /* std::sort ascending (:621) */
    for (int i = 1; i < n; ++i) {
        const float v = c[i];
        int j = i - 1;
        while (j >= 0 && c[j] > v) { c[j + 1] = c[j]; --j; }
        c[j + 1] = v;
    }
    memcpy(centroids_out, c, sizeof(float) * (size_t)n);
}

/* src/cuda/turboquant_kernels.cu:662-664 */
void orc_tq_midpoints(const float* c, int n, float* mid) {
    for (int i = 0; i < n - 1; ++i) mid[i] = (c[i] + c[i + 1]) * 0.5f;
}

/* Declared order for y = H x (the reference used cublasSgemm, :841-848, whose
 * summation order is unspecified): butterflies of half-width 1, 2, ..., d/2
 * on (a, b) -> (a + b, a - b), then a single multiply by 1.0f/sqrtf(d), the
 * same fp32 constant build_hadamard_on_host scales H by (:568). */
void orc_tq_rotate(const float* x, const float* signs, float* y, int d) {
    for (int i = 0; i < d; ++i) y[i] = signs ? x[i] * signs[i] : x[i];
    for (int h = 1; h < d; h <<= 1) {
        for (int i = 0; i < d; i += 2 * h) {
            for (int j = i; j < i + h; ++j) {
                const float a = y[j], b = y[j + h];
                y[j] = a + b;
                y[j + h] = a - b;
            }
        }
    }
    const float c = 1.0f / sqrtf((float)d);
    for (int i = 0; i < d; ++i) y[i] = y[i] * c;
}

/* float_to_fp8_e4m3 / _e4b15 (turboquant_kernels.cu:47-83, :98-134): the
 * same code with exponent bias B = 7 or 15 and the exponent-255 code 0x7C
 * (e4m3) or 0x78 (e4b15); values below the smallest normal keep exponent
 * field 1 with a rounded, clamped mantissa; overflow saturates to 0x7F. */
uint8_t orc_f32_to_fp8(float v, int e4b15) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    const uint32_t sign = (bits >> 31) & 1;
    const int32_t exp_f32 = (int32_t)((bits >> 23) & 0xFF);
    const uint32_t mant_f32 = bits & 0x7FFFFF;
    const int32_t bias = e4b15 ? 15 : 7;
    if (exp_f32 == 0 && mant_f32 == 0) return (uint8_t)(sign << 7);
    if (exp_f32 == 255) return (uint8_t)((sign << 7) | (e4b15 ? 0x78 : 0x7C));
    int32_t e = exp_f32 - 127 + bias;
    if (e < 1) {
        const int32_t shift = 1 - e;
        if (shift > 24) return (uint8_t)(sign << 7);
        const uint32_t mant = (0x800000u | mant_f32) >> shift;
        uint32_t m8 = (mant + 4) >> 4;
        if (m8 > 7) m8 = 7;
        return (uint8_t)((sign << 7) | (1 << 3) | m8);
    }
    if (e > 15) return (uint8_t)((sign << 7) | 0x7F);
    uint32_t m8 = (mant_f32 + 0x40000) >> 19;
    if (m8 > 7) {
        m8 = 0;
        e++;
        if (e > 15) return (uint8_t)((sign << 7) | 0x7F);
    }
    return (uint8_t)((sign << 7) | ((e & 0xF) << 3) | (m8 & 0x7));
}

/* fp8_e4m3_to_float / fp8_e4b15_to_float (:85-96, :136-143) */
float orc_fp8_to_f32(uint8_t b, int e4b15) {
    const uint32_t sign = (b >> 7) & 1, e = (b >> 3) & 0xF, m = b & 0x7;
    if (e == 0 && m == 0) return sign ? -0.0f : 0.0f;
    const float v = ldexpf(1.0f + (float)m / 8.0f, (int)e - (e4b15 ? 15 : 7));
    return sign ? -v : v;
}

static inline void put_half(uint8_t* p, float v, int bf16) {
    const uint16_t b = f32_to_half(v, bf16);
    p[0] = (uint8_t)(b & 0xff);
    p[1] = (uint8_t)(b >> 8);
}
static inline float get_half(const uint8_t* p, int bf16) {
    return half_to_f32((uint16_t)(p[0] | (p[1] << 8)), bf16);
}

/* pack codes: 4-bit -> even d low nibble (:278-292); 3-bit -> 8 codes per 3
 * bytes little-endian, code i at bits 3i (:293-310, :335-347). */
static void pack_codes(const int* q, int D, int bits, uint8_t* dst) {
    if (bits == 4) {
        for (int d = 0; d < D; d += 2) dst[d / 2] = (uint8_t)((q[d] & 0xf) | ((q[d + 1] & 0xf) << 4));
    } else {
        for (int g = 0; g < D / 8; ++g) {
            int packed = 0;
            for (int i = 0; i < 8; ++i) packed |= (q[g * 8 + i] & 0x7) << (i * 3);
            dst[g * 3] = (uint8_t)(packed & 0xff);
            dst[g * 3 + 1] = (uint8_t)((packed >> 8) & 0xff);
            dst[g * 3 + 2] = (uint8_t)((packed >> 16) & 0xff);
        }
    }
}

static void unpack_codes(const uint8_t* src, int D, int bits, int* q) {
    if (bits == 4) {
        for (int d = 0; d < D; d += 2) { q[d] = src[d / 2] & 0xf; q[d + 1] = src[d / 2] >> 4; }
    } else {
        for (int g = 0; g < D / 8; ++g) {
            const int packed = src[g * 3] | (src[g * 3 + 1] << 8) | (src[g * 3 + 2] << 16);
            for (int i = 0; i < 8; ++i) q[g * 8 + i] = (packed >> (i * 3)) & 0x7;
        }
    }
}

/* src/cuda/turboquant_kernels.cu:792-860 (turboquant_store) ->
 *   half_to_float_norm_kernel :145-161  norm = sqrtf(sum k*k), the sum a
 *                                       sequential fmaf chain (nvcc contracts);
 *   normalize_kernel :163-175           x = k * (1/(norm + 1e-8f));
 *   cublasSgemm :841-848                y = H x (declared order, orc_tq_rotate);
 *   tq_store_mse_kernel :247-351        codes = #midpoints <= y (scan :283-304),
 *                                       norm fp16 at +mse_bytes (:312);
 *                                       V min/max asymmetric codes (:314-347),
 *                                       scale, zero at +val_data(+2) (:349-350). */
void orc_tq_store(const uint16_t* key, const uint16_t* value, uint8_t* kv_cache,
                  const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                  int head_dim, int64_t block_size, const orc_tq_layout* L,
                  const float* midpoints, int bf16) {
    const int D = head_dim;
    /* tokens are independent (distinct slots): parallel over tokens */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < num_tokens; ++t) {
        float kf[256], xh[256], y[256], vf[256];
        int q[256];
        const int64_t slot = slot_mapping[t];
        if (slot < 0) continue; /* :266-267 */
        const int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < num_kv_heads; ++h) {
            const int64_t pid = (int64_t)t * num_kv_heads + h;
            /* compute_slot_byte_offset :39-45 */
            uint8_t* sp = kv_cache + blk * block_size * num_kv_heads * L->slot_size_aligned +
                          off * num_kv_heads * L->slot_size_aligned +
                          (int64_t)h * L->slot_size_aligned;
            if (L->key_fp8) {
                /* half_to_fp8_store_kernel :188-245: K byte d = fp8(k[d]) */
                for (int d = 0; d < D; ++d)
                    sp[d] = orc_f32_to_fp8(half_to_f32(key[pid * D + d], bf16), L->fp8_e4b15);
            } else {
            float norm_sq = 0.0f;
            for (int d = 0; d < D; ++d) {
                kf[d] = half_to_f32(key[pid * D + d], bf16);
                norm_sq = fmaf(kf[d], kf[d], norm_sq);
            }
            const float norm = sqrtf(norm_sq);
            const float inv_norm = 1.0f / (norm + 1e-8f);
            for (int d = 0; d < D; ++d) xh[d] = kf[d] * inv_norm;
            orc_tq_rotate(xh, NULL, y, D);
            const int nc = L->n_centroids;
            for (int d = 0; d < D; ++d) {
                int idx = 0;
                for (int c = nc - 2; c >= 0; --c) {
                    if (y[d] >= midpoints[c]) { idx = c + 1; break; }
                }
                q[d] = idx < nc - 1 ? idx : nc - 1;
            }
            pack_codes(q, D, L->key_quant_bits, sp);
            put_half(sp + L->mse_bytes, norm, bf16);
            }

            float vmin = FLT_MAX, vmax = -FLT_MAX;
            for (int d = 0; d < D; ++d) {
                vf[d] = half_to_f32(value[pid * D + d], bf16);
                vmin = fminf(vmin, vf[d]);
                vmax = fmaxf(vmax, vf[d]);
            }
            const int vmaxq = L->value_quant_bits == 4 ? 15 : 7;
            float vscale = (vmax - vmin) / (float)vmaxq;
            vscale = fmaxf(vscale, 1e-8f);
            for (int d = 0; d < D; ++d) {
                int qq = (int)roundf((vf[d] - vmin) / vscale);
                qq = qq < 0 ? 0 : (qq > vmaxq ? vmaxq : qq);
                q[d] = qq;
            }
            uint8_t* vp = sp + L->key_packed_size;
            pack_codes(q, D, L->value_quant_bits, vp);
            put_half(vp + L->val_data_bytes, vscale, bf16);
            put_half(vp + L->val_data_bytes + 2, vmin, bf16);
        }
    }
}

/* Dequantisation of tq_decode_stage1_kernel :416-483.  fp8 keys (:407-415)
 * carry no norm: the reference also multiplies them by the fp16 read at
 * +mse_bytes (:444-450), which for k8v4 is the first two bytes of the V
 * codes -- a defect, not restated. */
void orc_tq_dequant_slot(const uint8_t* sp, const orc_tq_layout* L, const float* C,
                         int bf16, float* k_out, float* v_out) {
    const int D = L->head_dim;
    int q[256];
    if (L->key_fp8) {
        for (int d = 0; d < D; ++d) k_out[d] = orc_fp8_to_f32(sp[d], L->fp8_e4b15);
        const uint8_t* vp = sp + L->key_packed_size;
        const float vs = get_half(vp + L->val_data_bytes, bf16);
        const float vz = get_half(vp + L->val_data_bytes + 2, bf16);
        unpack_codes(vp, D, L->value_quant_bits, q);
        for (int d = 0; d < D; ++d) v_out[d] = fmaf((float)q[d], vs, vz);
        return;
    }
    unpack_codes(sp, D, L->key_quant_bits, q);
    for (int d = 0; d < D; ++d) k_out[d] = C[q[d]];
    if (L->norm_correction) {
        float c_norm_sq = 0.0f;
        for (int d = 0; d < D; ++d) c_norm_sq = fmaf(k_out[d], k_out[d], c_norm_sq);
        const float c_inv = 1.0f / sqrtf(c_norm_sq + 1e-16f);
        for (int d = 0; d < D; ++d) k_out[d] *= c_inv;
    }
    const float vec_norm = get_half(sp + L->mse_bytes, bf16);
    for (int d = 0; d < D; ++d) k_out[d] *= vec_norm;
    const uint8_t* vp = sp + L->key_packed_size;
    const float vs = get_half(vp + L->val_data_bytes, bf16);
    const float vz = get_half(vp + L->val_data_bytes + 2, bf16);
    unpack_codes(vp, D, L->value_quant_bits, q);
    for (int d = 0; d < D; ++d) v_out[d] = fmaf((float)q[d], vs, vz);
}

static inline const uint8_t* tq_slot_ptr(const uint8_t* cache, int64_t blk, int64_t off,
                                         int h, int64_t bs, int Hkv, int S) {
    return cache + blk * bs * Hkv * S + off * Hkv * S + (int64_t)h * S;
}

/* src/cuda/turboquant_kernels.cu:939-1007 (turboquant_decode_attention):
 * q -> fp32 (:968), q_rot = H q (:975-982, declared order), stage 1 per
 * (b, h, split) (:353-506) executed once, stage 2 LSE merge (:508-547).
 * A split with no tokens has zero weight (the reference leaves it unwritten,
 * :380).  seq_len <= 0 writes zeros (the reference writes nothing, :375).
 * Tokens whose block-table entry is < 0 contribute nothing (:402). */
void orc_tq_decode(uint16_t* out, const uint16_t* query, const uint8_t* kv_cache,
                   const int32_t* block_tables, const int32_t* seq_lens,
                   int B, int Hq, int Hkv, int D, float scale, int64_t bs,
                   int64_t max_blocks, const orc_tq_layout* L, const float* C,
                   int ns, int bf16, int nthreads) {
    const int kv_group = Hq / Hkv;
    const int BLOCK_KV = 4;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq;
        const int kv_head = h / kv_group;
        const int seq_len = seq_lens[b];
        uint16_t* o = out + (int64_t)bh * D;
        if (seq_len <= 0) {
            for (int d = 0; d < D; ++d) o[d] = f32_to_half(0.0f, bf16);
            continue;
        }
        float qf[256], qr[256], acc[256], kr[256], vr[4][256], s[4], merge[256];
        float* mid = (float*)malloc(sizeof(float) * (size_t)ns * (size_t)(D + 1));
        int* valid = (int*)malloc(sizeof(int) * (size_t)ns);
        for (int d = 0; d < D; ++d) qf[d] = half_to_f32(query[(int64_t)bh * D + d], bf16);
        /* fp8 keys: q is not rotated (the reference copies it, :984) */
        if (L->key_fp8) memcpy(qr, qf, sizeof(float) * (size_t)D);
        else orc_tq_rotate(qf, NULL, qr, D);
        const int split_len = (seq_len + ns - 1) / ns;
        for (int sid = 0; sid < ns; ++sid) {
            const int start = split_len * sid;
            const int end = start + split_len < seq_len ? start + split_len : seq_len;
            valid[sid] = start < end;
            if (!valid[sid]) continue;
            for (int d = 0; d < D; ++d) acc[d] = 0.0f;
            float m_prev = -FLT_MAX, l_prev = 0.0f;
            for (int sn = start; sn < end; sn += BLOCK_KV) {
                const int en = sn + BLOCK_KV < end ? sn + BLOCK_KV : end;
                int cnt = 0;
                for (int pos = sn; pos < en; ++pos) {
                    const int32_t blk = block_tables[(int64_t)b * max_blocks + pos / bs];
                    if (blk < 0) continue;
                    const uint8_t* sp = tq_slot_ptr(kv_cache, blk, pos % bs, kv_head, bs, Hkv,
                                                    L->slot_size_aligned);
                    orc_tq_dequant_slot(sp, L, C, bf16, kr, vr[cnt]);
                    float dot = 0.0f;
                    for (int d = 0; d < D; ++d) dot = fmaf(qr[d], kr[d], dot);
                    s[cnt] = dot * scale;
                    cnt++;
                }
                if (cnt == 0) continue;
                float bmax = -FLT_MAX;
                for (int n = 0; n < cnt; ++n) bmax = fmaxf(bmax, s[n]);
                const float new_max = fmaxf(m_prev, bmax);
                const float re = expf(m_prev - new_max);
                for (int d = 0; d < D; ++d) acc[d] *= re;
                l_prev *= re;
                for (int n = 0; n < cnt; ++n) {
                    const float p = expf(s[n] - new_max);
                    l_prev += p;
                    for (int d = 0; d < D; ++d) acc[d] = fmaf(p, vr[n][d], acc[d]);
                }
                m_prev = new_max;
            }
            float* mo = mid + (int64_t)sid * (D + 1);
            const float safe_l = l_prev > 0.0f ? l_prev : 1.0f;
            for (int d = 0; d < D; ++d) mo[d] = acc[d] / safe_l;
            mo[D] = m_prev + logf(safe_l);
        }
        float max_lse = -FLT_MAX;
        for (int sid = 0; sid < ns; ++sid)
            if (valid[sid]) max_lse = fmaxf(max_lse, mid[(int64_t)sid * (D + 1) + D]);
        for (int d = 0; d < D; ++d) merge[d] = 0.0f;
        float sum_exp = 0.0f;
        for (int sid = 0; sid < ns; ++sid) {
            if (!valid[sid]) continue;
            const float* mo = mid + (int64_t)sid * (D + 1);
            const float w = expf(mo[D] - max_lse);
            sum_exp += w;
            for (int d = 0; d < D; ++d) merge[d] = fmaf(w, mo[d], merge[d]);
        }
        const float inv_sum = 1.0f / (sum_exp + 1e-8f);
        for (int d = 0; d < D; ++d) o[d] = f32_to_half(merge[d] * inv_sum, bf16);
        free(mid);
        free(valid);
    }
}

/* exact fp64 softmax(q k^T * scale) v over rows k[n][D], v[n][D] */
static void softmax_av_exact(const double* qd, const double* K, const double* V, int n,
                             int D, double scale, double* out) {
    double m = -INFINITY;
    double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    for (int i = 0; i < n; ++i) {
        double dot = 0.0;
        for (int d = 0; d < D; ++d) dot += qd[d] * K[(int64_t)i * D + d];
        s[i] = dot * scale;
        if (s[i] > m) m = s[i];
    }
    double l = 0.0;
    for (int d = 0; d < D; ++d) out[d] = 0.0;
    for (int i = 0; i < n; ++i) {
        const double p = exp(s[i] - m);
        l += p;
        for (int d = 0; d < D; ++d) out[d] += p * V[(int64_t)i * D + d];
    }
    for (int d = 0; d < D; ++d) out[d] = n > 0 ? out[d] / l : 0.0;
    free(s);
}

void orc_tq_decode_exact(double* out, const uint16_t* query, const uint8_t* kv_cache,
                         const int32_t* block_tables, const int32_t* seq_lens,
                         int B, int Hq, int Hkv, int D, double scale, int64_t bs,
                         int64_t max_blocks, const orc_tq_layout* L, const float* C,
                         int bf16, int nthreads) {
    const int kv_group = Hq / Hkv;
    const double c = 1.0 / sqrt((double)D);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq, kvh = h / kv_group;
        const int n = seq_lens[b] > 0 ? seq_lens[b] : 0;
        double* K = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        double* V = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        double qd[256], qr[256];
        float kr[256], vr[256];
        int cnt = 0;
        for (int pos = 0; pos < n; ++pos) {
            const int32_t blk = block_tables[(int64_t)b * max_blocks + pos / bs];
            if (blk < 0) continue;
            const uint8_t* sp = tq_slot_ptr(kv_cache, blk, pos % bs, kvh, bs, Hkv,
                                            L->slot_size_aligned);
            /* exact dequant: centroid / ||centroids|| * norm (fp8 keys: the
             * decoded byte), code*scale + zero */
            int qc[256];
            if (L->key_fp8) {
                for (int d = 0; d < D; ++d) K[(int64_t)cnt * D + d] = orc_fp8_to_f32(sp[d], L->fp8_e4b15);
            } else {
            unpack_codes(sp, D, L->key_quant_bits, qc);
            double cn = 0.0;
            for (int d = 0; d < D; ++d) cn += (double)C[qc[d]] * (double)C[qc[d]];
            const double ci = L->norm_correction ? 1.0 / sqrt(cn + 1e-16) : 1.0;
            const double nrm = get_half(sp + L->mse_bytes, bf16);
            for (int d = 0; d < D; ++d) K[(int64_t)cnt * D + d] = (double)C[qc[d]] * ci * nrm;
            }
            const uint8_t* vp = sp + L->key_packed_size;
            const double vs = get_half(vp + L->val_data_bytes, bf16);
            const double vz = get_half(vp + L->val_data_bytes + 2, bf16);
            unpack_codes(vp, D, L->value_quant_bits, qc);
            for (int d = 0; d < D; ++d) V[(int64_t)cnt * D + d] = qc[d] * vs + vz;
            cnt++;
        }
        (void)kr; (void)vr;
        for (int d = 0; d < D; ++d) qd[d] = half_to_f32(query[(int64_t)bh * D + d], bf16);
        for (int i = 0; i < D; ++i) {
            double acc = 0.0;
            for (int j = 0; j < D; ++j)
                acc += ((__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c) * qd[j];
            qr[i] = L->key_fp8 ? qd[i] : acc;
        }
        softmax_av_exact(qr, K, V, cnt, D, scale, out + (int64_t)bh * D);
        free(K);
        free(V);
    }
}

/* ------------------------------------------------------------------------ */
/* TurboQuant per-32-group variant (configuration text; no reference code)  */
/* ------------------------------------------------------------------------ */
/* Defined here (the configuration asks for "seeded random-sign Walsh-Hadamard
 * + 4-bit / 3-bit codes with a 16-bit scale (+zero) per 32-value group"):
 *   y = H (s * x) / sqrt(d), in orc_tq_rotate's declared order, for K and V;
 *   s[i] = -1 where bit i % 64 of orc_rand_u64(seed, ORC_G32_SIGN_STREAM,
 *   i / 64) is set (seed 0: all +1);
 *   slot = K part then V part, each four 32-value blocks of y:
 *     4-bit: {fp16 d, fp16 m, qs[16]}, qs[j] = q[j] | q[j+16] << 4, y ~ q d + m,
 *            d = (max - min) / 15, q = min(15, (int)((y - min) / d + 0.5));
 *     3-bit: {fp16 d, qs[12]}, codes 8k .. 8k+7 in bytes 3k .. 3k+2 little
 *            endian (code i at bits 3i), y ~ (q - 4) d, d = v / -4 with v the
 *            first value of largest magnitude, q = min(7, (int)(y / d + 4.5));
 *   the divisions are y * (1/d) (0 when d = 0) in fp32, no contraction. */
#define ORC_G32_SIGN_STREAM 0x5349474eULL

void orc_g32_signs(uint64_t seed, float* s, int d) {
    for (int i = 0; i < d; ++i) {
        const uint64_t w = seed ? orc_rand_u64(seed, ORC_G32_SIGN_STREAM, (uint64_t)(i / 64)) : 0;
        s[i] = ((w >> (i % 64)) & 1) ? -1.0f : 1.0f;
    }
}

int orc_g32_part_bytes(int bits) { return bits == 4 ? 80 : 56; }

static void g32_put_f16(uint8_t* p, float v) {
    const uint16_t b = orc_f32_to_f16(v);
    p[0] = (uint8_t)(b & 0xff);
    p[1] = (uint8_t)(b >> 8);
}
static float g32_get_f16(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

void orc_g32_quantize_part(const float* y, int bits, uint8_t* dst) {
    for (int g = 0; g < 4; ++g) {
        const float* x = y + 32 * g;
        int q[32];
        if (bits == 4) {
            uint8_t* blk = dst + 20 * g;
            float mn = x[0], mx = x[0];
            for (int j = 1; j < 32; ++j) {
                mn = fminf(mn, x[j]);
                mx = fmaxf(mx, x[j]);
            }
            const float d = (mx - mn) / 15.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            g32_put_f16(blk, d);
            g32_put_f16(blk + 2, mn);
            for (int j = 0; j < 32; ++j) {
                float t = x[j] - mn;
                t = t * id;
                t = t + 0.5f;
                const int c = (int)t;
                q[j] = c > 15 ? 15 : c;
            }
            for (int j = 0; j < 16; ++j) blk[4 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
        } else {
            uint8_t* blk = dst + 14 * g;
            float amax = 0.0f, v = 0.0f;
            for (int j = 0; j < 32; ++j) {
                const float a = fabsf(x[j]);
                if (a > amax) {
                    amax = a;
                    v = x[j];
                }
            }
            const float d = v / -4.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            g32_put_f16(blk, d);
            for (int j = 0; j < 32; ++j) {
                float t = x[j] * id;
                t = t + 4.5f;
                const int c = (int)t;
                q[j] = c > 7 ? 7 : c;
            }
            for (int k = 0; k < 4; ++k) {
                uint32_t w = 0;
                for (int i = 0; i < 8; ++i) w |= (uint32_t)q[8 * k + i] << (3 * i);
                blk[2 + 3 * k] = (uint8_t)(w & 0xff);
                blk[3 + 3 * k] = (uint8_t)((w >> 8) & 0xff);
                blk[4 + 3 * k] = (uint8_t)((w >> 16) & 0xff);
            }
        }
    }
}

void orc_g32_dequant_part(const uint8_t* src, int bits, float* y) {
    for (int g = 0; g < 4; ++g) {
        if (bits == 4) {
            const uint8_t* blk = src + 20 * g;
            const float d = g32_get_f16(blk), m = g32_get_f16(blk + 2);
            for (int j = 0; j < 16; ++j) {
                y[32 * g + j] = (float)(blk[4 + j] & 0xf) * d + m;
                y[32 * g + j + 16] = (float)(blk[4 + j] >> 4) * d + m;
            }
        } else {
            const uint8_t* blk = src + 14 * g;
            const float d = g32_get_f16(blk);
            for (int k = 0; k < 4; ++k) {
                const uint32_t w = blk[2 + 3 * k] | (blk[3 + 3 * k] << 8) | (blk[4 + 3 * k] << 16);
                for (int i = 0; i < 8; ++i) y[32 * g + 8 * k + i] = (float)((int)((w >> (3 * i)) & 7) - 4) * d;
            }
        }
    }
}

void orc_g32_store(const uint16_t* key, const uint16_t* value, uint8_t* kv_cache,
                   const int64_t* slot_mapping, int T, int Hkv, int D, int64_t bs, int bits,
                   uint64_t seed, int bf16) {
    const int P = orc_g32_part_bytes(bits), S = 2 * P;
    float sg[128];
    orc_g32_signs(seed, sg, D);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        const int64_t slot = slot_mapping[t];
        if (slot < 0) continue;
        float x[128], y[128];
        for (int h = 0; h < Hkv; ++h) {
            const int64_t pid = (int64_t)t * Hkv + h;
            uint8_t* sp = kv_cache + (slot / bs) * bs * Hkv * S + (slot % bs) * Hkv * S + (int64_t)h * S;
            for (int part = 0; part < 2; ++part) {
                const uint16_t* src = (part ? value : key) + pid * D;
                for (int d = 0; d < D; ++d) x[d] = half_to_f32(src[d], bf16);
                orc_tq_rotate(x, sg, y, D);
                orc_g32_quantize_part(y, bits, sp + part * P);
            }
        }
    }
}

/* Exact fp64 attention over the dequantized pages, in the rotated domain:
 * q_r = H (s q) / sqrt(d), O = s (H O_r) / sqrt(d) (exact H, fp64). */
void orc_g32_decode_exact(double* out, const uint16_t* query, const uint8_t* kv_cache,
                          const int32_t* block_tables, const int32_t* seq_lens, int B, int Hq,
                          int Hkv, int D, double scale, int64_t bs, int64_t max_blocks, int bits,
                          uint64_t seed, int q_bf16, int nthreads) {
    const int kv_group = Hq / Hkv;
    const int P = orc_g32_part_bytes(bits), S = 2 * P;
    const double c = 1.0 / sqrt((double)D);
    float sg[128];
    orc_g32_signs(seed, sg, D);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq, kvh = h / kv_group;
        const int n = seq_lens[b] > 0 ? seq_lens[b] : 0;
        double* K = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        double* V = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        double qs[128], qr[128], orr[128];
        float y[128];
        int cnt = 0;
        for (int pos = 0; pos < n; ++pos) {
            const int32_t blk = block_tables[(int64_t)b * max_blocks + pos / bs];
            if (blk < 0) continue;
            const uint8_t* sp = kv_cache + (int64_t)blk * bs * Hkv * S + (pos % bs) * Hkv * S +
                                (int64_t)kvh * S;
            orc_g32_dequant_part(sp, bits, y);
            for (int d = 0; d < D; ++d) K[(int64_t)cnt * D + d] = y[d];
            orc_g32_dequant_part(sp + P, bits, y);
            for (int d = 0; d < D; ++d) V[(int64_t)cnt * D + d] = y[d];
            cnt++;
        }
        for (int d = 0; d < D; ++d) qs[d] = half_to_f32(query[(int64_t)bh * D + d], q_bf16) * sg[d];
        for (int i = 0; i < D; ++i) {
            double acc = 0.0;
            for (int j = 0; j < D; ++j) acc += ((__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c) * qs[j];
            qr[i] = acc;
        }
        softmax_av_exact(qr, K, V, cnt, D, scale, orr);
        for (int i = 0; i < D; ++i) {
            double acc = 0.0;
            for (int j = 0; j < D; ++j) acc += ((__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c) * orr[j];
            out[(int64_t)bh * D + i] = acc * sg[i];
        }
        free(K);
        free(V);
    }
}

/* ------------------------------------------------------------------------ */
/* fused Q/K RMSNorm + RoPE (src/cuda/fused_attn_kernels.cu:39-313)         */
/* ------------------------------------------------------------------------ */
/* Intended semantics of fused_qk_norm_rope_store_kernel, in place on q
 * [T][Hq][D] and k [T][Hkv][D] (fp16 or bf16 bits):
 *   RMSNorm (:72-124, when the weight is given): S = sum of x^2 over the
 *     head's D values, inv = 1 / sqrtf(S / D + eps), y = (x * inv) * w[h*D+d],
 *     rounded to the element type (the reference writes the buffer back);
 *   RoPE (:128-178): cos = cache[pos][0 .. D/2), sin = cache[pos][D/2 .. D);
 *     neox pairs (d, d + D/2), GPT-J pairs (2d, 2d+1), pair index d:
 *     a' = a*cos[d] - b*sin[d], b' = b*cos[d] + a*sin[d], rounded.
 * The reference's reduction shuffles across warps of a 128-thread block and
 * its GPT-J branch reads the neox pairs; those are defects, not semantics.
 * Declared order of S (shared with the kernel): 16 partial sums, partial j
 * = fmaf chain over dims 8j .. 8j+7 from 0, then a butterfly over j with
 * lane distances 1, 2, 4, 8 (s_j += s_{j^m}).  No other contraction. */
static float norm_sum_sq(const float* x, int D) {
    float p[32];
    const int L = D / 8;
    for (int j = 0; j < L; ++j) {
        float a = 0.0f;
        for (int e = 0; e < 8; ++e) a = fmaf(x[8 * j + e], x[8 * j + e], a);
        p[j] = a;
    }
    for (int m = 1; m < L; m <<= 1) {
        float t[32];
        for (int j = 0; j < L; ++j) t[j] = p[j] + p[j ^ m];
        for (int j = 0; j < L; ++j) p[j] = t[j];
    }
    return p[0];
}

static void norm_rope_row(uint16_t* row, const uint16_t* w, const uint16_t* cs, int D, float eps,
                          int is_neox, int bf16) {
    float x[256];
    for (int d = 0; d < D; ++d) x[d] = half_to_f32(row[d], bf16);
    if (w) {
        const float S = norm_sum_sq(x, D);
        const float inv = 1.0f / sqrtf(S / (float)D + eps);
        for (int d = 0; d < D; ++d) {
            float t = x[d] * inv;
            t = t * half_to_f32(w[d], bf16);
            x[d] = half_to_f32(f32_to_half(t, bf16), bf16);
        }
    }
    const int half = D / 2;
    for (int d = 0; d < half; ++d) {
        const int ia = is_neox ? d : 2 * d, ib = is_neox ? d + half : 2 * d + 1;
        const float a = x[ia], b = x[ib];
        const float c = half_to_f32(cs[d], bf16), s = half_to_f32(cs[half + d], bf16);
        float t0 = a * c, t1 = b * s;
        const float na = t0 - t1;
        t0 = b * c;
        t1 = a * s;
        const float nb = t0 + t1;
        row[ia] = f32_to_half(na, bf16);
        row[ib] = f32_to_half(nb, bf16);
    }
}

void orc_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* q_weight, const uint16_t* k_weight,
                      const uint16_t* cos_sin, const int64_t* pos, int T, int Hq, int Hkv, int D,
                      float eps, int is_neox, int bf16) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        const uint16_t* cs = cos_sin + pos[t] * D;
        for (int h = 0; h < Hq; ++h)
            norm_rope_row(q + ((int64_t)t * Hq + h) * D, q_weight ? q_weight + (int64_t)h * D : NULL, cs, D,
                          eps, is_neox, bf16);
        for (int h = 0; h < Hkv; ++h)
            norm_rope_row(k + ((int64_t)t * Hkv + h) * D, k_weight ? k_weight + (int64_t)h * D : NULL, cs, D,
                          eps, is_neox, bf16);
    }
}

/* ------------------------------------------------------------------------ */
/* paged decode over f16 / bf16 / q8_0 / q4_0 pages                         */
/* ------------------------------------------------------------------------ */

/* Gather one sequence's K (or V) entries for kv-head h through the block
 * table: row i = token i.  Returns the number of tokens gathered (tokens
 * whose block-table entry is < 0 are dropped). */
static int gather_entries(const uint8_t* cache, int fmt, int hnd, const int32_t* bt,
                          int seq_len, int h, int Hkv, int D, int64_t bs,
                          uint8_t* dst) {
    const int64_t E = orc_kv_entry_bytes(fmt, D);
    int cnt = 0;
    for (int pos = 0; pos < seq_len; ++pos) {
        const int32_t blk = bt[pos / bs];
        if (blk < 0) continue;
        const int64_t off = kv_entry_offset((int64_t)blk * bs + pos % bs, h, bs, Hkv, E, hnd);
        memcpy(dst + (int64_t)cnt * E, cache + off, (size_t)E);
        cnt++;
    }
    return cnt;
}

void orc_paged_decode_exact(double* out, const float* q, const uint8_t* kc,
                            const uint8_t* vc, int fmt, int hnd, const int32_t* bt,
                            const int32_t* seq_lens, int B, int Hq, int Hkv, int D,
                            double scale, int64_t bs, int64_t max_blocks, int nthreads) {
    const int kv_group = Hq / Hkv;
    const int64_t E = orc_kv_entry_bytes(fmt, D);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq, kvh = h / kv_group;
        const int n = seq_lens[b] > 0 ? seq_lens[b] : 0;
        uint8_t* kb = (uint8_t*)malloc((size_t)E * (size_t)(n + 1));
        uint8_t* vb = (uint8_t*)malloc((size_t)E * (size_t)(n + 1));
        double* K = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        double* V = (double*)malloc(sizeof(double) * (size_t)(n + 1) * (size_t)D);
        const int cnt = gather_entries(kc, fmt, hnd, bt + (int64_t)b * max_blocks, n, kvh, Hkv, D, bs, kb);
        gather_entries(vc, fmt, hnd, bt + (int64_t)b * max_blocks, n, kvh, Hkv, D, bs, vb);
        float tmp[256];
        double qd[256];
        for (int i = 0; i < cnt; ++i) {
            orc_kv_dequant_entry(kb + (int64_t)i * E, fmt, D, tmp);
            for (int d = 0; d < D; ++d) K[(int64_t)i * D + d] = tmp[d];
            orc_kv_dequant_entry(vb + (int64_t)i * E, fmt, D, tmp);
            for (int d = 0; d < D; ++d) V[(int64_t)i * D + d] = tmp[d];
        }
        for (int d = 0; d < D; ++d) qd[d] = q[(int64_t)bh * D + d];
        softmax_av_exact(qd, K, V, cnt, D, scale, out + (int64_t)bh * D);
        free(kb); free(vb); free(K); free(V);
    }
}

/* ggml-cpu vec_dot of K row (fmt) with Q converted to K's vec_dot type:
 * f16 K: ggml_vec_dot_f16 (vec.cpp) -> double-accumulated fp32 products;
 * q8_0/q4_0 K: Q quantised to q8_0 (quantize_row_q8_0 -> _ref in vm_c's
 * SSE-only ggml build), per-block integer dot times d_k*d_q
 * (ggml-cpu/quants.c ggml_vec_dot_q8_0_q8_0_generic / q4_0_q8_0_generic). */
static float kq_dot(const uint8_t* k, int fmt, const uint16_t* q16, const uint8_t* q8, int D) {
    if (fmt == ORC_KV_F16 || fmt == ORC_KV_BF16) {
        double sum = 0.0;
        for (int d = 0; d < D; ++d) {
            const uint16_t kh = (uint16_t)(k[2 * d] | (k[2 * d + 1] << 8));
            const float kf = half_to_f32(kh, fmt == ORC_KV_BF16);
            const float qf = half_to_f32(q16[d], fmt == ORC_KV_BF16);
            sum += (double)(kf * qf);
        }
        return (float)sum;
    }
    float sumf = 0.0f;
    const int E = fmt == ORC_KV_Q8_0 ? Q8_0_BYTES : Q4_0_BYTES;
    for (int ib = 0; ib < D / QK; ++ib) {
        const uint8_t* kb = k + ib * E;
        const uint8_t* qb = q8 + ib * Q8_0_BYTES;
        int sumi = 0;
        if (fmt == ORC_KV_Q8_0) {
            for (int j = 0; j < QK; ++j) sumi += (int)(int8_t)kb[2 + j] * (int)(int8_t)qb[2 + j];
        } else {
            for (int j = 0; j < QK / 2; ++j) {
                const int v0 = (kb[2 + j] & 0x0f) - 8;
                const int v1 = (kb[2 + j] >> 4) - 8;
                sumi += v0 * (int)(int8_t)qb[2 + j] + v1 * (int)(int8_t)qb[2 + j + QK / 2];
            }
        }
        const float dk = orc_f16_to_f32((uint16_t)(kb[0] | (kb[1] << 8)));
        const float dq = orc_f16_to_f32((uint16_t)(qb[0] | (qb[1] << 8)));
        sumf += (float)sumi * (dk * dq);
    }
    return sumf;
}

/* ggml/src/ggml-cpu/ops.cpp:8214-8450 (one_chunk) over [ic0, ic1) for one query
 * row; writes M, S and the fp32 VKQ accumulator. */
static void ggml_one_chunk(const float* q, const uint8_t* K, const uint8_t* V, int fmt,
                           int D, int64_t E, int ic0, int ic1, float scale, float* M_out,
                           float* S_out, float* vkq32) {
    uint16_t q16[256], vkq16[256];
    uint8_t q8[8 * Q8_0_BYTES];
    float v32[256];
    const int f16v = (fmt == ORC_KV_F16);
    if (fmt == ORC_KV_F16 || fmt == ORC_KV_BF16) {
        for (int d = 0; d < D; ++d) q16[d] = f32_to_half(q[d], fmt == ORC_KV_BF16);
    } else {
        orc_quantize_row_q8_0(q, q8, D);
    }
    if (f16v) memset(vkq16, 0, sizeof(uint16_t) * (size_t)D);
    else memset(vkq32, 0, sizeof(float) * (size_t)D);
    float S = 0.0f, M = -INFINITY;
    for (int ic = ic0; ic < ic1; ++ic) {
        float s = kq_dot(K + (int64_t)ic * E, fmt, q16, q8, D);
        s = s * scale;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        const uint8_t* vd = V + (int64_t)ic * E;
        if (f16v) {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                /* ggml_vec_scale_f16: y = fp16(fp32(y)*v) */
                for (int d = 0; d < D; ++d) vkq16[d] = orc_f32_to_f16(orc_f16_to_f32(vkq16[d]) * ms);
            } else {
                vs = expf(s - M);
            }
            /* ggml_vec_mad_f16: y = fp16(fp32(y) + fp32(x)*v), no FMA */
            for (int d = 0; d < D; ++d) {
                const float xv = orc_f16_to_f32((uint16_t)(vd[2 * d] | (vd[2 * d + 1] << 8)));
                volatile float prod = xv * vs;
                vkq16[d] = orc_f32_to_f16(orc_f16_to_f32(vkq16[d]) + prod);
            }
        } else {
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                for (int d = 0; d < D; ++d) vkq32[d] *= ms;
            } else {
                vs = expf(s - M);
            }
            orc_kv_dequant_entry(vd, fmt, D, v32);
            for (int d = 0; d < D; ++d) {
                volatile float prod = v32[d] * vs;
                vkq32[d] = vkq32[d] + prod;
            }
        }
        S = S * ms + vs;
    }
    if (f16v)
        for (int d = 0; d < D; ++d) vkq32[d] = orc_f16_to_f32(vkq16[d]);
    *M_out = M;
    *S_out = S;
}

void orc_decode_ggml(float* out, const float* q, const uint8_t* kc, const uint8_t* vc,
                     int fmt, int hnd, const int32_t* bt, const int32_t* seq_lens, int B,
                     int Hq, int Hkv, int D, float scale, int64_t bs, int64_t max_blocks,
                     int nth, int nthreads) {
    const int kv_group = Hq / Hkv;
    const int64_t E = orc_kv_entry_bytes(fmt, D);
    if (nth < 1) nth = 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int bh = 0; bh < B * Hq; ++bh) {
        const int b = bh / Hq, h = bh % Hq, kvh = h / kv_group;
        const int n = seq_lens[b] > 0 ? seq_lens[b] : 0;
        uint8_t* kb = (uint8_t*)malloc((size_t)E * (size_t)(n + 1));
        uint8_t* vb = (uint8_t*)malloc((size_t)E * (size_t)(n + 1));
        const int cnt = gather_entries(kc, fmt, hnd, bt + (int64_t)b * max_blocks, n, kvh, Hkv, D, bs, kb);
        gather_entries(vc, fmt, hnd, bt + (int64_t)b * max_blocks, n, kvh, Hkv, D, bs, vb);
        float* o = out + (int64_t)bh * D;
        const float* qh = q + (int64_t)bh * D;
        float vkq[256];
        /* ops.cpp:8848-8893: split-KV only for f16/f32 K==V type and >= 512 KV */
        const int split = (fmt == ORC_KV_F16) && cnt >= 512;
        if (!split) {
            float M, S;
            ggml_one_chunk(qh, kb, vb, fmt, D, E, 0, cnt, scale, &M, &S, vkq);
            const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
            for (int d = 0; d < D; ++d) o[d] = vkq[d] * S_inv;
        } else {
            /* ops.cpp:8742-8810 reduce_partials */
            const int chunk = (cnt + nth - 1) / nth;
            float Mf = -INFINITY, Sf = 0.0f, acc[256];
            for (int d = 0; d < D; ++d) acc[d] = 0.0f;
            for (int c = 0; c < nth; ++c) {
                const int i0 = c * chunk;
                if (i0 >= cnt) continue;
                const int i1 = i0 + chunk < cnt ? i0 + chunk : cnt;
                float M, S;
                ggml_one_chunk(qh, kb, vb, fmt, D, E, i0, i1, scale, &M, &S, vkq);
                if (S == 0.0f) continue;
                const float Mn = fmaxf(Mf, M);
                const float so = expf(Mf - Mn), sn = expf(M - Mn);
                for (int d = 0; d < D; ++d) {
                    volatile float a = acc[d] * so;
                    volatile float bb = vkq[d] * sn;
                    acc[d] = a + bb;
                }
                Sf = Sf * so + S * sn;
                Mf = Mn;
            }
            const float S_inv = Sf != 0.0f ? 1.0f / Sf : 1.0f;
            for (int d = 0; d < D; ++d) o[d] = acc[d] * S_inv;
        }
        free(kb);
        free(vb);
    }
}

/* ------------------------------------------------------------------------ */
/* causal prefill: exact fp64 rows                                          */
/* ------------------------------------------------------------------------ */

void orc_prefill_exact_rows(double* out, const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, int is_bf16, const int32_t* cu, int B,
                            int Hq, int Hkv, int D, double scale, const int64_t* tokens,
                            const int32_t* heads, int64_t nrows, int nthreads) {
    const int kv_group = Hq / Hkv;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic)
#endif
    for (int64_t r = 0; r < nrows; ++r) {
        const int64_t t = tokens[r];
        const int h = heads[r], kvh = h / kv_group;
        int b = 0;
        while (b < B - 1 && t >= cu[b + 1]) b++;
        const int64_t t0 = cu[b];
        const int n = (int)(t - t0 + 1);
        double* K = (double*)malloc(sizeof(double) * (size_t)n * (size_t)D);
        double* V = (double*)malloc(sizeof(double) * (size_t)n * (size_t)D);
        double qd[256];
        for (int i = 0; i < n; ++i)
            for (int d = 0; d < D; ++d) {
                const int64_t idx = ((t0 + i) * Hkv + kvh) * D + d;
                K[(int64_t)i * D + d] = half_to_f32(k[idx], is_bf16);
                V[(int64_t)i * D + d] = half_to_f32(v[idx], is_bf16);
            }
        for (int d = 0; d < D; ++d) qd[d] = half_to_f32(q[(t * Hq + h) * D + d], is_bf16);
        softmax_av_exact(qd, K, V, n, D, scale, out + r * D);
        free(K);
        free(V);
    }
}

/* ------------------------------------------------------------------------ */
/* deterministic inputs                                                     */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t orc_rand_u64(uint64_t seed, uint64_t stream, uint64_t index) {
    return splitmix64(splitmix64(splitmix64(seed) ^ stream) ^ index);
}

double orc_randn(uint64_t seed, uint64_t stream, uint64_t index) {
    const double u1 = ((double)(orc_rand_u64(seed, stream, 2 * index) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(orc_rand_u64(seed, stream, 2 * index + 1) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_randn_f16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16((float)orc_randn(seed, stream, (uint64_t)i));
}

void orc_randn_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16((float)orc_randn(seed, stream, (uint64_t)i));
}
