// vm_c/kernels_fused_attn.hpp -- fused Q/K RMSNorm + RoPE (+ quantize-on-
// append of K/V) on HIP.
//
// Same names, argument order and meaning as vm_c
// include/vm_c/cuda/kernels_fused_attn.h:51-93 (hipStream_t for cudaStream_t),
// with three trailing additions: dtype (the reference reads the global
// compute dtype), layout (the reference always writes the HND placement
// h*head_dim*block_size + offset*head_dim, which is the default here) and,
// for the TurboQuant overload, the slot configuration.
// kv_cache_dtype: "auto" | "fp16" | "bf16" | "q8_0" | "q4_0" (GGUF blocks,
// quantized on append).  cache_stride: bytes per block, 0 = packed.
// Limits: head_dim == 128.
#pragma once

#include <cstdint>
#include <string>

#include "vm_c/common.hpp"
#include "vm_c/kernels_turboquant.hpp"

namespace vm_c {

// key_cache == nullptr or slot_mapping == nullptr: norm + RoPE only.
void fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                              const void* q_norm_weight, const void* k_norm_weight,
                              const void* cos_sin_cache, const int64_t* position_ids,
                              void* key_cache, void* value_cache, const int64_t* slot_mapping,
                              int num_tokens, int num_heads, int num_kv_heads, int head_dim,
                              float rms_norm_eps, bool is_neox, int64_t block_size,
                              int64_t cache_stride, const std::string& kv_cache_dtype,
                              hipStream_t stream = nullptr,
                              ScalarType dtype = ScalarType::FLOAT16,
                              const std::string& layout = "hnd");

// Append into packed TurboQuant slots (kv_cache as for turboquant_store);
// no counterpart in the reference, whose fused kernel only copies fp16 rows.
void fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                              const void* q_norm_weight, const void* k_norm_weight,
                              const void* cos_sin_cache, const int64_t* position_ids,
                              void* kv_cache, const int64_t* slot_mapping, int num_tokens,
                              int num_heads, int num_kv_heads, int head_dim, float rms_norm_eps,
                              bool is_neox, int64_t block_size, const TQConfig& config,
                              hipStream_t stream = nullptr,
                              ScalarType dtype = ScalarType::FLOAT16);

void fused_qk_norm_rope(void* q_buf, void* k_buf, const void* q_norm_weight,
                        const void* k_norm_weight, const void* cos_sin_cache,
                        const int64_t* position_ids, int num_tokens, int num_heads,
                        int num_kv_heads, int head_dim, float rms_norm_eps, bool is_neox,
                        hipStream_t stream = nullptr, ScalarType dtype = ScalarType::FLOAT16);

}  // namespace vm_c
