// vm_c/kernels_attention.hpp -- paged KV append, paged decode and causal
// prefill entry points on HIP.
//
// Same names, argument order and meaning as vm_c
// include/vm_c/cuda/kernels_cache.h:8-48, kernels_attention.h:12-78 and
// kernels_flash_attn.h:46-82 (hipStream_t for cudaStream_t).
// kv_cache_dtype strings: "auto" (the activation type), "fp16", "bf16",
// "q8_0", "q4_0" (GGUF blocks, quantized on append); layout "nhd" | "hnd".
// k_scale / v_scale (fp8 scaling) and alibi_slopes must be null: those
// features are not on this path and a non-null value throws.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "vm_c/common.hpp"

namespace vm_c {

struct AttentionParams {
    int batch_size = 0;
    int num_tokens = 0;
    int num_heads = 0;
    int num_kv_heads = 0;
    int head_dim = 0;
    int block_size = 0;
    int max_seq_len = 0;
    int max_num_blocks_per_req = 0;
    float scale = 1.0f;
    ScalarType dtype = ScalarType::FLOAT16;
    int tp_rank = 0;
    int blocksparse_local_blocks = 0;
    int blocksparse_vert_stride = 0;
    int blocksparse_block_size = 0;
    int blocksparse_head_sliding_step = 0;
};

// Copies whole blocks between pools: block_mapping holds num_blocks
// (src_block, dst_block) pairs on the host (cache_kernels.cu:58-86).
void swap_blocks(void* src, void* dst, int64_t block_size_in_bytes, const int64_t* block_mapping,
                 int64_t num_blocks, int src_device, int dst_device, hipStream_t stream = nullptr);

void reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                       const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                       int head_dim, int64_t block_size, int64_t cache_stride,
                       const std::string& kv_cache_dtype, const void* k_scale,
                       const void* v_scale, ScalarType dtype, hipStream_t stream = nullptr,
                       const std::string& layout = "nhd");

// kernels_cache.h:29-39: the reference's flash-layout entry is the same append
// (cache_kernels.cu:146-157 forwards to reshape_and_cache); so is this one.
void reshape_and_cache_flash(const void* key, const void* value, void* key_cache, void* value_cache,
                             const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                             int head_dim, int64_t block_size, int64_t cache_stride,
                             const std::string& kv_cache_dtype, const void* k_scale,
                             const void* v_scale, ScalarType dtype, hipStream_t stream = nullptr,
                             const std::string& layout = "nhd");

// kernels_cache.h:41-46 (cache_kernels.cu:175-212): dst = fp8(src * scale),
// OCP E4M3 for "fp8_e4m3", E5M2 otherwise (vmc_convert_fp8).  reshape_and_cache
// above writes E4M3 pages for "fp8_e4m3" and "fp8_e5m2" (x / k_scale, x /
// v_scale; the scales are host float pointers, null = 1).
void convert_fp8(void* dst_cache, const void* src_cache, double scale, int64_t num_elements,
                 const std::string& kv_cache_dtype, ScalarType dtype, hipStream_t stream = nullptr);

// Prefill over the paged cache (cached prefix + this step's appended tokens):
// token t attends positions 0 .. token_positions[t] of sequence
// token_to_seq[t] (attention_kernels.cu:416-436).  seq_lens and num_reqs are
// accepted for signature compatibility; no workspace (one pass per token).
void paged_attention_prefill(void* out, const void* query, const void* key_cache,
                             const void* value_cache, int num_tokens, int num_heads,
                             int num_kv_heads, int head_dim, float scale, int64_t block_size,
                             int64_t max_num_blocks_per_req, const int32_t* block_tables,
                             const int32_t* seq_lens, const int32_t* token_to_seq,
                             const int32_t* token_positions, int num_reqs,
                             const std::string& kv_cache_dtype, ScalarType dtype,
                             hipStream_t stream = nullptr, const std::string& layout = "nhd");

// Tiled MFMA prefill over the paged cache (chunked prefill), the same
// semantics as paged_attention_prefill with every K/V tile of a sequence
// read once per block of query rows instead of once per token
// (kernels_flash_attn.h:46-66).  kv_cache_dtype "auto", "fp16", "bf16",
// "q8_0", "q4_0"; head_dim 128, block_size 16.  No workspace.
void flash_attention_prefill_v2(void* output, const void* query, const void* key_cache,
                                const void* value_cache, int num_tokens, int num_heads,
                                int num_kv_heads, int head_dim, float scale, int64_t block_size,
                                int64_t max_num_blocks_per_req, const int32_t* block_tables,
                                const int32_t* seq_lens, const int32_t* token_to_seq,
                                const int32_t* token_positions, int num_reqs,
                                const std::string& kv_cache_dtype, ScalarType dtype,
                                hipStream_t stream = nullptr, const std::string& layout = "nhd");

// One pass per sequence (no split, no workspace): one workgroup per request.
void paged_attention_v1(void* out, const void* query, const void* key_cache,
                        const void* value_cache, const AttentionParams& params,
                        const int32_t* block_tables, const int32_t* seq_lens,
                        const float* alibi_slopes, const std::string& kv_cache_dtype,
                        const void* k_scale, const void* v_scale, hipStream_t stream = nullptr,
                        const std::string& layout = "nhd");

// Split-KV decode: the batch's pages are spread evenly over the GPU.
// exp_sums / max_logits are unused (the partial max and sum live next to each
// partial output); tmp_out is the split workspace and must hold
// paged_attention_v2_workspace_size(params) bytes.
size_t paged_attention_v2_workspace_size(const AttentionParams& params);
void paged_attention_v2(void* out, void* exp_sums, void* max_logits, void* tmp_out,
                        const void* query, const void* key_cache, const void* value_cache,
                        const AttentionParams& params, const int32_t* block_tables,
                        const int32_t* seq_lens, const float* alibi_slopes,
                        const std::string& kv_cache_dtype, const void* k_scale,
                        const void* v_scale, hipStream_t stream = nullptr,
                        const std::string& layout = "nhd");

// Causal prefill over contiguous K/V ("local"): each sequence's tokens are
// contiguous and start at position 0, token t attends [t - pos(t), t].
// token_to_seq is accepted for signature compatibility (positions suffice).
void flash_attention_prefill_local(void* output, const void* query, const void* key,
                                   const void* value, int num_tokens, int num_heads,
                                   int num_kv_heads, int head_dim, float scale,
                                   const int32_t* token_to_seq, const int32_t* token_positions,
                                   ScalarType dtype, hipStream_t stream = nullptr);

// The same launch also appends every K/V row into the paged cache
// (quantize-on-append); no counterpart in the reference, which appends with
// a separate reshape_and_cache launch.
void flash_attention_prefill_local_with_cache(
    void* output, const void* query, const void* key, const void* value, int num_tokens,
    int num_heads, int num_kv_heads, int head_dim, float scale, const int32_t* token_positions,
    ScalarType dtype, void* key_cache, void* value_cache, const int64_t* slot_mapping,
    int64_t block_size, const std::string& kv_cache_dtype, const std::string& layout,
    hipStream_t stream = nullptr);

}  // namespace vm_c
