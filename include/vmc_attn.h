/*
 * vmc_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * The drop-in boundary for vm_c's attention kernels: plain pointers, sizes
 * and enums, no C++ or framework types.  Every entry point is stream-ordered
 * and asynchronous (no host synchronisation, no device allocation); errors are
 * returned as negative errno-style codes.  The C++ layer in
 * vm_c_amd/host/ (namespace vm_c) keeps vm_c's own signatures and calls these.
 *
 * All pointers are device pointers unless a comment says otherwise.
 */
#ifndef VMC_ATTN_H
#define VMC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vmc_stream_t; /* == hipStream_t */

/* ---- status codes ---- */
#define VMC_OK 0
#define VMC_EINVAL (-22) /* bad shape / dtype / format / pointer            */
#define VMC_ENOMEM (-12) /* caller workspace smaller than the query says    */
#define VMC_EIO (-5)     /* HIP launch or runtime error                       */

/* ---- element types of Q / K / V / O ---- */
typedef enum { VMC_DTYPE_F16 = 0, VMC_DTYPE_BF16 = 1 } vmc_dtype;

/* ---- paged KV formats (kv_cache_dtype strings "fp16", "bf16", "q8_0",
 *      "q4_0"; the TurboQuant packed slot has its own entry points) ---- */
typedef enum {
    VMC_KV_F16 = 0,
    VMC_KV_BF16 = 1,
    VMC_KV_Q8_0 = 2, /* GGUF block_q8_0: fp16 d + 32 x int8, 34 B / 32 values */
    VMC_KV_Q4_0 = 3  /* GGUF block_q4_0: fp16 d + 16 B nibbles, 18 B / 32     */
} vmc_kv_format;

/* "nhd": page [block][token][head][entry]; "hnd": [block][head][token][entry] */
typedef enum { VMC_LAYOUT_NHD = 0, VMC_LAYOUT_HND = 1 } vmc_kv_layout;

/* bytes of one (token, kv-head) entry of head_dim values, < 0 if invalid */
int64_t vmc_kv_entry_bytes(int kv_format, int head_dim);

/*
 * Append K/V rows into the paged cache, quantizing on the way.
 * Replaces vm_c::reshape_and_cache (include/vm_c/cuda/kernels_cache.h:17-27,
 * src/cuda/cache_kernels.cu:88-157); kv_cache_dtype becomes kv_format and
 * q8_0/q4_0 follow ggml's set_rows encoders (ggml-quants.c:234-257, :71-104).
 *   key, value    [num_tokens][num_kv_heads][head_dim] of src_dtype
 *   key_cache, value_cache   page pools, cache_stride bytes per block
 *                 (0 = block_size*num_kv_heads*entry_bytes)
 *   slot_mapping  int64 [num_tokens]; slot = block*block_size + offset, < 0 skips
 */
int vmc_reshape_and_cache(const void* key, const void* value, void* key_cache,
                          void* value_cache, const int64_t* slot_mapping, int num_tokens,
                          int num_kv_heads, int head_dim, int64_t block_size,
                          int64_t cache_stride, int kv_format, int src_dtype, int layout,
                          vmc_stream_t stream);

/*
 * fp8 pages: reshape_and_cache with kv_cache_dtype "fp8_e4m3" or "fp8_e5m2"
 * (src/cuda/cache_kernels.cu:101-131, :14-54).  Both strings store OCP FP8
 * E4M3 bytes (the reference casts to __nv_fp8_e4m3 for either): one byte per
 * value, x / k_scale for K and x / v_scale for V, rounded to nearest even and
 * saturated to +-448 (NaN -> 0x7f).  Page addressing and slot_mapping as in
 * vmc_reshape_and_cache with one-byte entries (head_dim bytes per (token,
 * head)); cache_stride 0 = block_size * num_kv_heads * head_dim.
 *   k_scale, v_scale   HOST pointers to one float each, read at the call
 *                      (cache_kernels.cu:102-104); NULL = 1.0
 * head_dim % 16 == 0; cache_stride % 16 == 0; key/value/pools 16-byte aligned.
 */
int vmc_reshape_and_cache_fp8(const void* key, const void* value, void* key_cache,
                              void* value_cache, const int64_t* slot_mapping, int num_tokens,
                              int num_kv_heads, int head_dim, int64_t block_size,
                              int64_t cache_stride, const float* k_scale, const float* v_scale,
                              int src_dtype, int layout, vmc_stream_t stream);

/*
 * Cache conversion to fp8: replaces vm_c::convert_fp8 (src/cuda/
 * cache_kernels.cu:175-212): dst[i] = fp8(src[i] * (float)scale) for
 * num_elements values of src_dtype, E5M2 when e5m2 != 0 ("fp8_e5m2"), else
 * E4M3 ("fp8_e4m3"); OCP FP8, rounded to nearest even, saturated to the
 * largest finite value (E4M3 448, E5M2 57344), NaN -> 0x7f.
 */
int vmc_convert_fp8(void* dst_cache, const void* src_cache, double scale, int64_t num_elements,
                    int e5m2, int src_dtype, vmc_stream_t stream);

/*
 * Paged decode attention, one query token per sequence, over f16/bf16/q8_0/
 * q4_0 pages read through the block table, split-KV with an fp32 LSE merge.
 * Replaces vm_c::paged_attention_v1 / _v2 (include/vm_c/cuda/
 * kernels_attention.h:30-78); semantics are those of ggml's flash_attn_ext
 * (ggml-cpu/ops.cpp:8214-8957) on the gathered K/V, GQA head = q_head /
 * (num_heads / num_kv_heads).
 *   out, query    [batch][num_heads][head_dim] of q_dtype
 *   block_tables  int32 [batch][max_num_blocks_per_req]; entries < 0 are holes
 *   seq_lens      int32 [batch]; <= 0 writes a zero row
 *   workspace     >= vmc_paged_decode_workspace_size(...) bytes (device memory;
 *                 may be NULL when that size is 0)
 *   max_num_kv_splits  1: one pass per sequence, no workspace (paged_attention_v1);
 *                 > 1: the batch's pages are split evenly over the GPU with at
 *                 most batch * max_num_kv_splits pieces; <= 0: no cap
 * Limits: head_dim 64, 128 or 256; block_size 16 at head_dim 128.  At
 * head_dim 128 with num_kv_heads <= 8 and num_heads / num_kv_heads <= 16 the
 * tuned kernel runs: two launches on `stream` (split pass, merge of cut
 * sequences).  Other head dims and head counts run a one-wave-per-row kernel
 * (one launch, no workspace).  No host synchronisation.  The workspace size
 * depends on the current device's CU count.
 */
size_t vmc_paged_decode_workspace_size(int batch_size, int num_heads, int num_kv_heads,
                                       int head_dim, int max_num_blocks_per_req, int block_size,
                                       int max_num_kv_splits);
int vmc_paged_attention_decode(void* out, const void* query, const void* key_cache,
                               const void* value_cache, const int32_t* block_tables,
                               const int32_t* seq_lens, int batch_size, int num_heads,
                               int num_kv_heads, int head_dim, int block_size,
                               int max_num_blocks_per_req, float scale, int q_dtype,
                               int kv_format, int layout, int max_num_kv_splits,
                               void* workspace, size_t workspace_bytes, vmc_stream_t stream);

/* ---- TurboQuant packed KV (src/cuda/turboquant_kernels.cu) ---- */

/* Mirrors vm_c::TQConfig (include/vm_c/cuda/kernels_turboquant.h:10-75). */
typedef struct vmc_tq_config {
    int head_dim;
    int key_quant_bits;
    int value_quant_bits;
    int norm_correction;
    int key_fp8;
    int fp8_e4b15;
    int mse_bytes;
    int key_packed_size;
    int val_data_bytes;
    int value_packed_size;
    int slot_size;
    int slot_size_aligned;
    int n_centroids;
    int max_num_kv_splits;
    /* The two fields below have no counterpart in vm_c::TQConfig: they select
     * the per-32-group variant the benchmark configurations describe
     * ("seeded random-sign Walsh-Hadamard, 4-bit / 3-bit codes with a 16-bit
     * scale (+zero) per 32-value group"), for which the reference has no
     * code.  group_size 0 is the reference layout above. */
    int group_size;              /* 0, or 32 */
    unsigned long long sign_seed; /* rotation signs (0: all +1) */
} vmc_tq_config;

/* TQConfig::from_method: "turboquant_4bit_nc" (default), "turboquant_3bit_nc",
 * "turboquant_k3v4_nc", "turboquant_k8v4" (fp8 keys: 128 bytes of the
 * reference's own e4m3 codes -- fp8_e4b15 = 1 selects its e4b15 codes -- then
 * 4-bit V codes, fp16 scale and zero; 196-byte slots; no rotation, no norm).
 * Returns VMC_EINVAL for an unknown method.
 * The per-32-group variant (no reference counterpart): "turboquant_4bit_g32"
 * and "turboquant_3bit_g32".  For both K and V, y = H (s * x) / sqrt(128)
 * (s = +-1 signs from sign_seed), then per 32 values of y:
 *   4-bit: {fp16 d, fp16 m, 16 bytes, byte j = code j | code j+16 << 4},
 *          y ~ code * d + m, d = (max - min) / 15;
 *   3-bit: {fp16 d, 12 bytes of codes, 8 codes per 3 bytes little endian,
 *          code i at bits 3i}, y ~ (code - 4) * d, d = v / -4 with v the
 *          first value of largest magnitude.
 * A slot is the K part then the V part: 2 x 80 = 160 bytes (4-bit) or
 * 2 x 56 = 112 bytes (3-bit); the fields above describe one part (mse_bytes
 * = code bytes, key_packed_size = value_packed_size = part bytes,
 * n_centroids = 0, norm_correction = 0).  sign_seed starts at 0; the caller
 * sets it, identically for the store and the decode. */
int vmc_tq_config_from_method(int head_dim, const char* method, vmc_tq_config* out);

/* Host-side constant tables (Lloyd-Max centroids for N(0, 1/d), midpoints),
 * identical to src/cuda/turboquant_kernels.cu:578-623 / :662-664.  Host
 * pointers; n_centroids floats and n_centroids-1 floats. */
int vmc_tq_host_tables(int head_dim, int bits, float* centroids, float* midpoints);

/*
 * Prefill attention over the paged cache (a cached prefix plus this step's
 * tokens, already appended): token t is token_positions[t] of sequence
 * token_to_seq[t] and attends that sequence's positions 0 .. token_positions[t]
 * through its block_tables row.  Replaces vm_c::paged_attention_prefill
 * (src/cuda/attention_kernels.cu:416-436, the path of
 * PagedAttentionBackend::forward_prefill); semantics as
 * vmc_paged_attention_decode with one row per token (formats, layouts,
 * workspace: vmc_paged_decode_workspace_size(num_tokens, ...), none when
 * max_num_kv_splits == 1).  query / out [num_tokens][num_heads][head_dim].
 */
int vmc_paged_attention_prefill(void* out, const void* query, const void* key_cache,
                                const void* value_cache, int num_tokens, int num_heads,
                                int num_kv_heads, int head_dim, float scale, int block_size,
                                int max_num_blocks_per_req, const int32_t* block_tables,
                                const int32_t* token_to_seq, const int32_t* token_positions,
                                int q_dtype, int kv_format, int layout, int max_num_kv_splits,
                                void* workspace, size_t workspace_bytes, vmc_stream_t stream);

/*
 * Tiled MFMA prefill over the paged cache (chunked prefill: this step's
 * tokens, already appended, attend a cached prefix plus themselves).
 * Replaces vm_c::flash_attention_prefill_v2 (include/vm_c/cuda/
 * kernels_flash_attn.h:46-66, src/cuda/flash_attn_v2_kernels.cu:194-250;
 * called from PagedAttentionBackend::forward_prefill,
 * src/model/attention_backend.cpp:44-64).  Token t is position
 * token_positions[t] of sequence token_to_seq[t] and attends that sequence's
 * positions 0 .. token_positions[t] through its block_tables row
 * [num_reqs][max_num_blocks_per_req]; pages with a negative entry are
 * skipped; a token whose sequence is outside [0, num_reqs) or whose position
 * is negative gets zeros.  seq_lens is not read (the positions bound the
 * keys) and may be NULL.  A workgroup takes 32-row blocks of up to 4 query
 * heads of one KV head and streams 64-key tiles of the sequence's pages
 * through LDS once for all of them; rows of several sequences in one block
 * are processed one sequence at a time.  kv_format: VMC_KV_F16, VMC_KV_BF16
 * (load-to-LDS rows), VMC_KV_Q8_0, VMC_KV_Q4_0 (dequantized to fp16 as
 * vmc_paged_attention_decode does); q_dtype VMC_DTYPE_F16 / VMC_DTYPE_BF16,
 * rounded to the page type when they differ (q8_0 / q4_0: fp16).  Limits:
 * head_dim 128 with block_size 16 and pools 16-byte aligned for the tiled
 * kernel; head_dim 64 and 256 run a one-wave-per-row kernel.  No workspace.
 */
int vmc_flash_attention_prefill_v2(void* out, const void* query, const void* key_cache,
                                   const void* value_cache, int num_tokens, int num_heads,
                                   int num_kv_heads, int head_dim, float scale, int block_size,
                                   int max_num_blocks_per_req, const int32_t* block_tables,
                                   const int32_t* seq_lens, const int32_t* token_to_seq,
                                   const int32_t* token_positions, int num_reqs, int q_dtype,
                                   int kv_format, int layout, vmc_stream_t stream);

/*
 * Quantize-on-append of K/V into packed TurboQuant slots.
 * Replaces vm_c::turboquant_store (kernels_turboquant.h:107-119;
 * turboquant_kernels.cu:792-860).  key/value [num_tokens][num_kv_heads]
 * [head_dim] of half_dtype; norm, scale and zero are stored as half_dtype.
 * One fused kernel, no workspace.
 */
int vmc_turboquant_store(const void* key, const void* value, void* kv_cache,
                         const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                         int head_dim, int64_t block_size, const vmc_tq_config* cfg,
                         int half_dtype, vmc_stream_t stream);

/*
 * Fused Q/K RMSNorm + RoPE + quantize-on-append, one launch.
 * Replaces vm_c::fused_qk_norm_rope_store and vm_c::fused_qk_norm_rope
 * (include/vm_c/cuda/kernels_fused_attn.h:51-93; fused_attn_kernels.cu:39-313).
 *   q_buf [num_tokens][num_heads][head_dim], k_buf, v_buf [num_tokens]
 *   [num_kv_heads][head_dim], all of dtype; q and k are updated in place.
 *   q_norm_weight [num_heads*head_dim], k_norm_weight [num_kv_heads*head_dim]
 *   of dtype, or NULL (no norm for that side):
 *     y = (x * (1/sqrtf(sum(x^2)/head_dim + eps))) * w, rounded to dtype.
 *   cos_sin_cache [max_pos][head_dim] of dtype, cos in [0, head_dim/2), sin in
 *   [head_dim/2, head_dim); position_ids int64 [num_tokens].  Neox pairs
 *   (d, d + head_dim/2), GPT-J pairs (2d, 2d+1); a' = a cos - b sin,
 *   b' = b cos + a sin, rounded to dtype.
 *   key_cache == NULL: norm + RoPE only (fused_qk_norm_rope).  Otherwise the
 *   rotated K row and the V row are appended at slot_mapping (int64, < 0
 *   skips): tq_config == NULL -> paged pools key_cache / value_cache with
 *   kv_format, layout and cache_stride as in vmc_reshape_and_cache;
 *   tq_config != NULL -> packed TurboQuant slots in key_cache (value_cache
 *   unused), as vmc_turboquant_store writes them.
 * Limits: head_dim == 128.  The reference's 128-thread reduction across
 * warps and its GPT-J read of the neox pairs are not reproduced.
 */
int vmc_fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                                 const void* q_norm_weight, const void* k_norm_weight,
                                 const void* cos_sin_cache, const int64_t* position_ids,
                                 void* key_cache, void* value_cache,
                                 const int64_t* slot_mapping, int num_tokens, int num_heads,
                                 int num_kv_heads, int head_dim, float rms_norm_eps,
                                 int is_neox, int64_t block_size, int64_t cache_stride,
                                 int kv_format, int layout, const vmc_tq_config* tq_config,
                                 int dtype, vmc_stream_t stream);

/*
 * Split-KV paged decode over packed TurboQuant slots.
 * Replaces vm_c::turboquant_decode_attention (kernels_turboquant.h:121-138;
 * turboquant_kernels.cu:939-1007): q rotated by the Hadamard transform, K
 * reconstructed from centroids (norm-corrected, times the stored norm), V =
 * code*scale + zero, fp32 online softmax, LSE merge.  The caller provides the
 * workspace (the reference grew it inside the call); max_num_kv_splits and
 * limits as for vmc_paged_attention_decode.  half_dtype (VMC_DTYPE_F16 or
 * VMC_DTYPE_BF16) is the dtype of query, output and the stored norms, scales
 * and zeros (the reference dispatches on its compute dtype,
 * turboquant_kernels.cu:966; the per-32-group layout takes fp16).
 * norm_correction 0 scales keys by the stored norm alone (the reference's
 * 4/4 decode without it, turboquant_kernels.cu:889-912).  At head_dim 128,
 * shapes past 8 KV heads or 16 query heads per KV head, and fp8 keys with
 * bf16 halves, run on a one-wave-per-row kernel.
 */
size_t vmc_turboquant_decode_workspace_size(int batch_size, int num_heads, int num_kv_heads,
                                            int head_dim, int64_t max_num_blocks_per_req,
                                            int64_t block_size, int max_num_kv_splits);
int vmc_turboquant_decode_attention(void* output, const void* query, const void* kv_cache,
                                    const int32_t* block_tables, const int32_t* seq_lens,
                                    int batch_size, int num_heads, int num_kv_heads,
                                    int head_dim, float scale, int64_t block_size,
                                    int64_t max_num_blocks_per_req, const vmc_tq_config* cfg,
                                    int half_dtype, int max_num_kv_splits, void* workspace,
                                    size_t workspace_bytes, vmc_stream_t stream);

/*
 * vmc_turboquant_decode_attention without a workspace argument: the split
 * partials go to a device array inside the library (one per GPU, held until
 * the process ends, vmc_noalloc_scratch_bytes() = 64 MiB), so the call
 * allocates nothing -- no hipMalloc, hipFree or allocating library routine --
 * and records no memset.  No counterpart in the reference: for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid allocation).  Same arguments, semantics and kernels as
 * vmc_turboquant_decode_attention; returns VMC_ENOMEM when
 * vmc_turboquant_decode_workspace_size(...) exceeds the array.  Calls that
 * overlap on one GPU share the array and race: serialise them (one stream,
 * or events).
 */
size_t vmc_noalloc_scratch_bytes(void);
int vmc_turboquant_decode_attention_noalloc(void* output, const void* query, const void* kv_cache,
                                            const int32_t* block_tables, const int32_t* seq_lens,
                                            int batch_size, int num_heads, int num_kv_heads,
                                            int head_dim, float scale, int64_t block_size,
                                            int64_t max_num_blocks_per_req, const vmc_tq_config* cfg,
                                            int half_dtype, int max_num_kv_splits,
                                            vmc_stream_t stream);

/*
 * Prefill attention over packed TurboQuant pages with a cached prefix: token
 * t is token_positions[t] of sequence token_to_seq[t] and attends positions
 * 0 .. token_positions[t] through its block_tables row (this step's tokens
 * already stored).  No counterpart in the reference, whose TurboQuant prefill
 * attends only the step's local K/V (attention_backend.cpp:153-196).
 * Steps of 16 tokens or more over reference-layout slots (codebook or fp8
 * keys; head_dim 128, block_size 16, kv_cache 4-byte aligned) run the tiled
 * MFMA prefill: each 64-key tile of a sequence is read once per block of
 * query rows, no workspace.  Other steps run the arithmetic of
 * vmc_turboquant_decode_attention with one row per token (workspace:
 * vmc_turboquant_decode_workspace_size(num_tokens, ...), none when
 * max_num_kv_splits == 1).
 */
int vmc_turboquant_prefill_attention(void* output, const void* query, const void* kv_cache,
                                     const int32_t* block_tables, const int32_t* token_to_seq,
                                     const int32_t* token_positions, int num_tokens, int num_heads,
                                     int num_kv_heads, int head_dim, float scale, int64_t block_size,
                                     int64_t max_num_blocks_per_req, const vmc_tq_config* cfg,
                                     int half_dtype, int max_num_kv_splits, void* workspace,
                                     size_t workspace_bytes, vmc_stream_t stream);

/*
 * One (sequence, position) row per token of an Engine step, for
 * vmc_turboquant_prefill_attention.  The Engine uploads block_tables and
 * seq_lens per request (src/core/engine.cpp:731-757) and token_to_seq /
 * token_positions only for prefill requests' tokens (:686-691, :760-766; a
 * decode request's token keeps 0 / 0).  The ggml TurboQuant node
 * (src/official/turboquant_kv_bridge.cpp:99-107) decodes num_tokens rows over
 * the per-request arrays, which is exact only for decode-only steps; this
 * gives every token of a prefill or mixed step its row: a prefill token keeps
 * (token_to_seq, token_positions), a decode token of request r (counted from
 * the request boundaries in token order) gets (r, seq_lens[r] - 1).  Rows of
 * a request outside [0, num_reqs) get (0, -1): no keys, a zero output row.
 *   row_seq, row_pos   int32 [num_tokens] (written)
 *   token_to_seq, token_positions int32 [num_tokens]; seq_lens int32 [num_reqs]
 * No counterpart in the reference (it has no such mapping).  One workgroup;
 * stream-ordered.
 */
int vmc_batch_token_rows(int32_t* row_seq, int32_t* row_pos, const int32_t* token_to_seq,
                         const int32_t* token_positions, const int32_t* seq_lens, int num_tokens,
                         int num_reqs, vmc_stream_t stream);

/*
 * Causal flash-attention prefill over contiguous ("local") K/V, bf16 or fp16,
 * MFMA for QK^T and PV, fp32 softmax.  Each sequence's tokens are contiguous
 * with positions 0..n-1, so token t attends tokens [t - pos(t), t].
 * Replaces vm_c::flash_attention_prefill_local (include/vm_c/cuda/
 * kernels_flash_attn.h:81-93).
 *   output, query [num_tokens][num_heads][head_dim]; key, value
 *   [num_tokens][num_kv_heads][head_dim]; token_positions int32 [num_tokens].
 * Optional fused quantize-on-append: when key_cache != NULL the same launch
 * writes every K/V row into the paged cache (kv_format/layout as in
 * vmc_reshape_and_cache, slot_mapping int64 [num_tokens]).
 * Limits: head_dim 64, 128 or 256 (64 and 256: a one-wave-per-row kernel,
 * then the append by vmc_reshape_and_cache), num_heads % num_kv_heads == 0.
 */
int vmc_flash_attention_prefill(void* output, const void* query, const void* key,
                                const void* value, int num_tokens, int num_heads,
                                int num_kv_heads, int head_dim, float scale,
                                const int32_t* token_positions, int dtype, void* key_cache,
                                void* value_cache, const int64_t* slot_mapping,
                                int64_t block_size, int kv_format, int layout,
                                vmc_stream_t stream);

/*
 * vmc_flash_attention_prefill with a caller workspace (no counterpart in the
 * reference, whose prefill takes none): the same arguments and results, plus
 * workspace / workspace_bytes, at least
 * vmc_flash_attention_prefill_workspace_size(num_tokens, num_kv_heads,
 * head_dim) bytes, 16-byte aligned (VMC_ENOMEM when smaller, VMC_EINVAL when
 * NULL at head_dim 128).  A first launch writes the fp16 V^T tiles of the
 * step's V (16 KB per 64 keys and KV head) into the workspace once, so the
 * attention kernel fetches them instead of transposing V in every
 * workgroup that reads it.  Outputs equal vmc_flash_attention_prefill's bit
 * for bit, except that bf16 V which that function would run in its exact
 * mode for some workgroups may run exact in more of them here (a tile's
 * flag covers all of its rows).  head_dim 64 / 256 ignore the workspace.
 * Concurrent calls on one workspace race.
 */
size_t vmc_flash_attention_prefill_workspace_size(int num_tokens, int num_kv_heads, int head_dim);
int vmc_flash_attention_prefill_ws(void* output, const void* query, const void* key,
                                   const void* value, int num_tokens, int num_heads,
                                   int num_kv_heads, int head_dim, float scale,
                                   const int32_t* token_positions, int dtype, void* key_cache,
                                   void* value_cache, const int64_t* slot_mapping,
                                   int64_t block_size, int kv_format, int layout, void* workspace,
                                   size_t workspace_bytes, vmc_stream_t stream);

/*
 * Measurement only (no counterpart in the reference): one streaming read of
 * bytes (a multiple of 16) at src (16-byte aligned).  mode 0: 16-byte
 * non-temporal vector loads into registers (sink: 1 KB of device memory the
 * kernel may write); mode 1: 16-byte non-temporal load-to-LDS transfers;
 * mode 2: 16-byte load-to-LDS transfers, the request type of the TurboQuant
 * decode (modes 1, 2: sink unused).  bench.py times them for the measured
 * HBM read ceilings and runs mode 2 under rocprofv3 to scale FETCH_SIZE for
 * the decode.
 */
int vmc_hbm_read_probe(const void* src, size_t bytes, int mode, void* sink, vmc_stream_t stream);

/* Device self-check of the lane-level assumptions the kernels rely on (MFMA
 * operand/result layouts of the shapes used, cross-row reductions, the
 * wave-private LDS exchange).  No counterpart in the reference: a guard for
 * toolchain / hardware changes.  Synchronous.  Returns 0 when all pass, a
 * bitmask of failed checks (> 0), or a negative status. */
int vmc_selftest(void);

/* Library self-description: "vmc_attn <version> gfx950". */
const char* vmc_version(void);

#ifdef __cplusplus
}
#endif
#endif /* VMC_ATTN_H */
