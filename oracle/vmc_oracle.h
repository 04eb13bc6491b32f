/*
 * vmc_oracle.h -- CPU restatement of vm_c's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in vm_c_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Citations are relative to the vm_c source tree; ggml paths are relative to
 * third_party/vm_c_official/ggml/.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   - fp16/bf16 conversion: exhaustive round trip + torch's converters.
 *   - q8_0 / q4_0 quantizers: bit-exact against the vendored ggml
 *     quantize_row_*_ref built from source (oracle/_ref), and the committed
 *     golden vectors in tests/golden/.
 *   - Hadamard: closed form (-1)^popcount(i&j)/sqrt(d) and H*H = I.
 *   - Lloyd-Max centroids: classic Max (1960) Gaussian quantizer tables
 *     scaled by 1/sqrt(d); committed fp32 bit patterns.
 *   - TQ store: slot sizes 134/102/118 B for d=128 (tp_runtime.cpp:257-261),
 *     unpack(pack) round trip, all-equal V -> codes 0, zero K -> norm 0,
 *     codes equal the nearest-centroid index of the exactly rotated vector.
 *   - TQ decode / paged decode: equals exact fp64 attention over the
 *     dequantized pages; split-count invariance; permuted block tables.
 *   - ggml CPU flash-attention restatement: against the vendored ggml CPU
 *     flash_attn_ext (oracle/_ref) and fp64 exact attention.
 *   - OCP fp8 conversion: every fp16 and bf16 value, random fp32 and every
 *     midpoint between neighbouring codes (and the floats either side of
 *     it) against a nearest-value search over the 256 codes with ties to
 *     the even code; the specification's max / min values.
 */
#ifndef VMC_ORACLE_H
#define VMC_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (round-to-nearest-even) ---- */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float    orc_bf16_to_f32(uint16_t h);
void     orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n);
void     orc_f16_to_f32_n(const uint16_t* x, float* y, int64_t n);

/* ---- GGUF q8_0 / q4_0 blocks (ggml-common.h:184-188, :241-245) ---- */
void orc_quantize_row_q8_0(const float* x, void* y, int64_t k);
void orc_dequantize_row_q8_0(const void* x, float* y, int64_t k);
void orc_quantize_row_q4_0(const float* x, void* y, int64_t k);
void orc_dequantize_row_q4_0(const void* x, float* y, int64_t k);

/* ---- OCP 8-bit floating point (OCP "8-bit Floating Point Specification
 *      (OFP8)" v1.0, 2023: E4M3 bias 7, max 448, NaN S.1111.111, no inf;
 *      E5M2 bias 15, max 57344, IEEE inf / NaN) from fp32: round to nearest
 *      even, |x| >= max (inf included) saturated to +-max, NaN -> 0x7f.
 *      This is the conversion of vm_c's fp8 KV paths
 *      (cache_kernels.cu:43-46 and :184 cast to __nv_fp8_e4m3 / _e5m2,
 *      whose float constructors saturate to finite); NaN's byte is not
 *      fixed by those call sites (parity unpinned for NaN inputs). ---- */
uint8_t orc_f32_to_ofp8(float x, int e5m2);
void    orc_f32_to_ofp8_n(const float* x, uint8_t* y, int64_t n, int e5m2);
float   orc_ofp8_to_f32(uint8_t b, int e5m2);
/* reshape_and_cache with kv_cache_dtype "fp8_e4m3" or "fp8_e5m2"
 * (cache_kernels.cu:101-131, :14-54): both write E4M3 bytes of x / scale
 * (the reference casts to __nv_fp8_e4m3 for either string); one byte per
 * value; page addressing as orc_kv_append with E = head_dim and the block
 * stride `stride` bytes (0 = bs*Hkv*head_dim). */
void orc_reshape_and_cache_fp8(const uint16_t* key, const uint16_t* value, int src_bf16,
                               uint8_t* key_cache, uint8_t* value_cache,
                               const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                               int head_dim, int64_t block_size, int64_t stride, float k_scale,
                               float v_scale, int hnd);
/* convert_fp8 (cache_kernels.cu:175-212): dst[i] = fp8(src[i] * scale),
 * E4M3 for "fp8_e4m3", else E5M2. */
void orc_convert_fp8(uint8_t* dst, const uint16_t* src, int src_bf16, float scale, int64_t n, int e5m2);

/* ---- paged KV formats for the non-TurboQuant path ---- */
enum { ORC_KV_F16 = 0, ORC_KV_BF16 = 1, ORC_KV_Q8_0 = 2, ORC_KV_Q4_0 = 3 };
/* bytes of one (token, kv-head) entry of head_dim values */
int64_t orc_kv_entry_bytes(int fmt, int head_dim);
/* Append K/V rows [T][Hkv][D] (fp16 or bf16 bits) into K and V page pools.
 * NHD: blk*stride + off*Hkv*E + h*E ; HND: blk*stride + h*bs*E + off*E,
 * stride = bs*Hkv*E.  slot < 0 skips the token. */
void orc_kv_append(const uint16_t* key, const uint16_t* value, int src_bf16,
                   uint8_t* key_cache, uint8_t* value_cache,
                   const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                   int head_dim, int64_t block_size, int fmt, int hnd);
void orc_kv_dequant_entry(const uint8_t* entry, int fmt, int head_dim, float* out);

/* ---- TurboQuant (src/cuda/turboquant_kernels.cu, kernels_turboquant.h) ---- */
typedef struct {
    int head_dim;
    int key_quant_bits;
    int value_quant_bits;
    int norm_correction;
    int mse_bytes;
    int key_packed_size;
    int val_data_bytes;
    int value_packed_size;
    int slot_size;
    int slot_size_aligned;
    int n_centroids;
    int key_fp8;     /* turboquant_k8v4: K stored as 128 fp8 bytes, no norm */
    int fp8_e4b15;   /* fp8 flavour of those keys: e4m3 (0) or e4b15 (1)  */
} orc_tq_layout;

/* the reference's own fp8 converters (turboquant_kernels.cu:47-143): bias 7
 * (e4m3) or 15 (e4b15), no NaN/inf codes, exponent 0 with a non-zero
 * mantissa decodes as (1 + m/8) 2^-bias like every other code. */
uint8_t orc_f32_to_fp8(float v, int e4b15);
float   orc_fp8_to_f32(uint8_t b, int e4b15);

int  orc_tq_layout_from_method(int head_dim, const char* method, orc_tq_layout* out);
void orc_tq_hadamard(float* out, int d);
void orc_tq_lloyd_max(float* centroids_out, int d, int bits);
void orc_tq_midpoints(const float* centroids, int n_centroids, float* midpoints);
/* y = H x in the declared order: in-place Walsh-Hadamard butterflies with
 * half-width h = 1, 2, 4, ..., d/2, then y *= 1/sqrtf(d).  signs (may be NULL)
 * multiplies x elementwise first. */
void orc_tq_rotate(const float* x, const float* signs, float* y, int d);
void orc_tq_store(const uint16_t* key, const uint16_t* value, uint8_t* kv_cache,
                  const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                  int head_dim, int64_t block_size, const orc_tq_layout* L,
                  const float* midpoints, int half_is_bf16);
/* Dequantize one slot: k_out = rotated-domain K (centroid * norm-correction *
 * norm), v_out = code*scale + zero. */
void orc_tq_dequant_slot(const uint8_t* slot, const orc_tq_layout* L,
                         const float* centroids, int half_is_bf16,
                         float* k_out, float* v_out);
/* Two-stage split-KV decode with the intended single-execution semantics of
 * tq_decode_stage1_kernel / stage2 (one body per (b,h,split)). */
void orc_tq_decode(uint16_t* out, const uint16_t* query, const uint8_t* kv_cache,
                   const int32_t* block_tables, const int32_t* seq_lens,
                   int batch, int num_heads, int num_kv_heads, int head_dim,
                   float scale, int64_t block_size, int64_t max_blocks_per_req,
                   const orc_tq_layout* L, const float* centroids,
                   int num_kv_splits, int half_is_bf16, int nthreads);
/* Exact fp64 attention over the dequantized TQ pages (rotation exact). */
void orc_tq_decode_exact(double* out, const uint16_t* query, const uint8_t* kv_cache,
                         const int32_t* block_tables, const int32_t* seq_lens,
                         int batch, int num_heads, int num_kv_heads, int head_dim,
                         double scale, int64_t block_size, int64_t max_blocks_per_req,
                         const orc_tq_layout* L, const float* centroids,
                         int half_is_bf16, int nthreads);

/* ---- TurboQuant per-32-group variant (configuration text, no reference
 * code; format defined in vmc_oracle.c) ---- */
void orc_g32_signs(uint64_t seed, float* s, int d);
int  orc_g32_part_bytes(int bits);
void orc_g32_quantize_part(const float* y, int bits, uint8_t* dst);
void orc_g32_dequant_part(const uint8_t* src, int bits, float* y);
void orc_g32_store(const uint16_t* key, const uint16_t* value, uint8_t* kv_cache,
                   const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                   int head_dim, int64_t block_size, int bits, uint64_t seed,
                   int half_is_bf16);
void orc_g32_decode_exact(double* out, const uint16_t* query, const uint8_t* kv_cache,
                          const int32_t* block_tables, const int32_t* seq_lens,
                          int batch, int num_heads, int num_kv_heads, int head_dim,
                          double scale, int64_t block_size, int64_t max_blocks_per_req,
                          int bits, uint64_t seed, int q_is_bf16, int nthreads);

/* ---- fused Q/K RMSNorm + RoPE (src/cuda/fused_attn_kernels.cu:39-313),
 * in place; weights and cos/sin cache of the element type; either weight may
 * be NULL (no norm).  The append that follows is orc_kv_append /
 * orc_tq_store / orc_g32_store on the updated k and the original v. ---- */
void orc_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* q_weight,
                      const uint16_t* k_weight, const uint16_t* cos_sin,
                      const int64_t* pos, int num_tokens, int num_heads,
                      int num_kv_heads, int head_dim, float eps, int is_neox,
                      int half_is_bf16);

/* ---- paged decode over f16/bf16/q8_0/q4_0 pages ---- */
/* exact fp64 softmax attention over the dequantized pages; q is fp32 */
void orc_paged_decode_exact(double* out, const float* q,
                            const uint8_t* key_cache, const uint8_t* value_cache,
                            int fmt, int hnd, const int32_t* block_tables,
                            const int32_t* seq_lens, int batch, int num_heads,
                            int num_kv_heads, int head_dim, double scale,
                            int64_t block_size, int64_t max_blocks_per_req,
                            int nthreads);
/* ggml CPU flash_attn_ext restatement (decode, one query row per sequence)
 * over K/V gathered from pages: Q converted to K's vec_dot type (f16, or q8_0
 * for a quantized K), fp16 V accumulator for an f16 V, KV split into `nth`
 * chunks with a partial reduce when K/V are f16 and S >= 512. fp32 out. */
void orc_decode_ggml(float* out, const float* q,
                     const uint8_t* key_cache, const uint8_t* value_cache,
                     int fmt, int hnd, const int32_t* block_tables,
                     const int32_t* seq_lens, int batch, int num_heads,
                     int num_kv_heads, int head_dim, float scale,
                     int64_t block_size, int64_t max_blocks_per_req, int nth,
                     int nthreads);

/* ---- causal prefill ---- */
/* Exact fp64 causal attention for selected rows.  q [T][Hq][D], k/v
 * [T][Hkv][D] (bf16 bits if is_bf16 else fp16 bits); cu_seqlens[B+1] gives
 * each sequence's token range; row r = (tokens[r], heads[r]). */
void orc_prefill_exact_rows(double* out, const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, int is_bf16,
                            const int32_t* cu_seqlens, int batch,
                            int num_heads, int num_kv_heads, int head_dim,
                            double scale, const int64_t* tokens,
                            const int32_t* heads, int64_t nrows, int nthreads);

/* ---- deterministic inputs ---- */
/* counter-based N(0,1): splitmix64(seed, stream, index) -> Box-Muller (double) */
double orc_randn(uint64_t seed, uint64_t stream, uint64_t index);
void   orc_randn_f16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream);
void   orc_randn_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream);
uint64_t orc_rand_u64(uint64_t seed, uint64_t stream, uint64_t index);

#ifdef __cplusplus
}
#endif
#endif
