/*
 * ref_harness.c -- drives the vendored ggml CPU backend (built from the
 * reference sources into oracle/_ref/ by oracle/Makefile) through ggml's
 * public API, so tests can compare the oracle with the reference itself.
 *
 * TEST INFRASTRUCTURE ONLY; it is never part of the product.
 *
 * Entry points:
 *   ref_from_float(type, x, y, k)      the CPU set_rows row encoder
 *                                      (ggml-cpu/ops.cpp:4950-5020 calls the
 *                                      type's from_float trait).
 *   ref_quantize_q8_0_ref / q4_0_ref   ggml-quants.c:234-257 / :71-104.
 *   ref_flash_attn(...)                ggml_flash_attn_ext on the CPU backend
 *                                      (ggml-cpu/ops.cpp:8214-8957), F32 prec.
 *   ref_flash_attn_timed(...)          the same, computed reps times and timed.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "ggml.h"
#include "ggml-cpu.h"

#define QTYPE(fmt) ((fmt) == 0 ? GGML_TYPE_F16 : (fmt) == 1 ? GGML_TYPE_BF16 : (fmt) == 2 ? GGML_TYPE_Q8_0 : GGML_TYPE_Q4_0)

void quantize_row_q8_0_ref(const float* x, void* y, int64_t k);
void quantize_row_q4_0_ref(const float* x, void* y, int64_t k);

void ref_quantize_q8_0_ref(const float* x, void* y, int64_t k) { quantize_row_q8_0_ref(x, y, k); }
void ref_quantize_q4_0_ref(const float* x, void* y, int64_t k) { quantize_row_q4_0_ref(x, y, k); }

int ref_from_float(int fmt, const float* x, void* y, int64_t k) {
    const struct ggml_type_traits_cpu* t = ggml_get_type_traits_cpu(QTYPE(fmt));
    if (!t || !t->from_float) return -1;
    t->from_float(x, y, k);
    return 0;
}

/* out[n_q][Hq][D] (ggml's permuted output) = flash_attn_ext(q, k, v, mask).
 *   q    : fp32 [Hq][n_q][D]
 *   k, v : rows of type fmt, [Hkv][n_kv][row]
 *   mask : NULL, or fp16 bits [n_q][n_kv] (0 or -inf) when causal != 0 it is
 *          built here as mask[i][j] = j <= i + (n_kv - n_q) ? 0 : -inf. */
int ref_flash_attn(float* out, const float* q, const void* k, const void* v, int fmt,
                   int n_q, int n_kv, int Hq, int Hkv, int D, float scale, int causal,
                   int n_threads) {
    const enum ggml_type kt = QTYPE(fmt);
    const size_t row = ggml_row_size(kt, D);
    size_t need = (size_t)Hq * n_q * D * 4 + 2 * (size_t)Hkv * n_kv * row +
                  (size_t)n_q * n_kv * 2 + (size_t)Hq * n_q * D * 4 + 64 * 1024 * 1024;
    struct ggml_init_params ip = {need, NULL, false};
    struct ggml_context* ctx = ggml_init(ip);
    if (!ctx) return -1;
    struct ggml_tensor* tq = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, D, n_q, Hq, 1);
    struct ggml_tensor* tk = ggml_new_tensor_4d(ctx, kt, D, n_kv, Hkv, 1);
    struct ggml_tensor* tv = ggml_new_tensor_4d(ctx, kt, D, n_kv, Hkv, 1);
    memcpy(tq->data, q, ggml_nbytes(tq));
    memcpy(tk->data, k, ggml_nbytes(tk));
    memcpy(tv->data, v, ggml_nbytes(tv));
    struct ggml_tensor* tm = NULL;
    if (causal) {
        tm = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, n_kv, n_q, 1, 1);
        ggml_fp16_t* m = (ggml_fp16_t*)tm->data;
        const ggml_fp16_t zero = ggml_fp32_to_fp16(0.0f);
        const ggml_fp16_t ninf = ggml_fp32_to_fp16(-INFINITY);
        for (int i = 0; i < n_q; ++i)
            for (int j = 0; j < n_kv; ++j) m[(size_t)i * n_kv + j] = (j <= i + (n_kv - n_q)) ? zero : ninf;
    }
    struct ggml_tensor* fa = ggml_flash_attn_ext(ctx, tq, tk, tv, tm, scale, 0.0f, 0.0f);
    ggml_flash_attn_ext_set_prec(fa, GGML_PREC_F32);
    struct ggml_cgraph* gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, fa);
    const enum ggml_status st = ggml_graph_compute_with_ctx(ctx, gf, n_threads);
    if (st == GGML_STATUS_SUCCESS) memcpy(out, fa->data, ggml_nbytes(fa));
    ggml_free(ctx);
    return st == GGML_STATUS_SUCCESS ? 0 : -2;
}

/* ref_flash_attn_timed: the same graph as ref_flash_attn, built once and
 * computed `reps` times; *secs = mean wall time of one ggml_graph_compute
 * (inputs already in ggml tensors, so graph building and copies are not
 * counted).  Used as the CPU baseline: the reference's own flash-attention
 * path on the host cores. */
int ref_flash_attn_timed(float* out, const float* q, const void* k, const void* v, int fmt,
                         int n_q, int n_kv, int Hq, int Hkv, int D, float scale, int causal,
                         int n_threads, int reps, double* secs) {
    const enum ggml_type kt = QTYPE(fmt);
    const size_t row = ggml_row_size(kt, D);
    size_t need = (size_t)Hq * n_q * D * 4 + 2 * (size_t)Hkv * n_kv * row +
                  (size_t)n_q * n_kv * 2 + (size_t)Hq * n_q * D * 4 + 64 * 1024 * 1024;
    struct ggml_init_params ip = {need, NULL, false};
    struct ggml_context* ctx = ggml_init(ip);
    if (!ctx) return -1;
    struct ggml_tensor* tq = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, D, n_q, Hq, 1);
    struct ggml_tensor* tk = ggml_new_tensor_4d(ctx, kt, D, n_kv, Hkv, 1);
    struct ggml_tensor* tv = ggml_new_tensor_4d(ctx, kt, D, n_kv, Hkv, 1);
    memcpy(tq->data, q, ggml_nbytes(tq));
    memcpy(tk->data, k, ggml_nbytes(tk));
    memcpy(tv->data, v, ggml_nbytes(tv));
    struct ggml_tensor* tm = NULL;
    if (causal) {
        tm = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, n_kv, n_q, 1, 1);
        ggml_fp16_t* m = (ggml_fp16_t*)tm->data;
        const ggml_fp16_t zero = ggml_fp32_to_fp16(0.0f);
        const ggml_fp16_t ninf = ggml_fp32_to_fp16(-INFINITY);
        for (int i = 0; i < n_q; ++i)
            for (int j = 0; j < n_kv; ++j) m[(size_t)i * n_kv + j] = (j <= i + (n_kv - n_q)) ? zero : ninf;
    }
    struct ggml_tensor* fa = ggml_flash_attn_ext(ctx, tq, tk, tv, tm, scale, 0.0f, 0.0f);
    ggml_flash_attn_ext_set_prec(fa, GGML_PREC_F32);
    struct ggml_cgraph* gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, fa);
    struct ggml_cplan plan = ggml_graph_plan(gf, n_threads, NULL);
    uint8_t* work = plan.work_size ? (uint8_t*)malloc(plan.work_size) : NULL;
    plan.work_data = work;
    enum ggml_status st = GGML_STATUS_SUCCESS;
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int r = 0; r < reps && st == GGML_STATUS_SUCCESS; ++r) st = ggml_graph_compute(gf, &plan);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (secs) *secs = ((t1.tv_sec - t0.tv_sec) + 1e-9 * (t1.tv_nsec - t0.tv_nsec)) / (reps > 0 ? reps : 1);
    if (st == GGML_STATUS_SUCCESS && out) memcpy(out, fa->data, ggml_nbytes(fa));
    free(work);
    ggml_free(ctx);
    return st == GGML_STATUS_SUCCESS ? 0 : -2;
}
