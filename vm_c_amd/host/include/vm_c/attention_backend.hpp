// vm_c/attention_backend.hpp -- the attention operator interface src/model
// uses (vm_c include/vm_c/model/attention_backend.hpp:15-140), on HIP.
//
// PagedAttentionBackend: standard pages (fp16 / bf16, and GGUF q8_0 / q4_0
// quantized on append) in "nhd" or "hnd" layout.  TurboQuantBackend: packed
// rotated low-bit slots (value_cache is null).  forward_decode uses
// meta.num_reqs query rows (one token per request).  forward_prefill runs the
// causal prefill over this step's contiguous K/V when nothing is cached yet;
// with a cached prefix (meta.num_computed_tokens > 0) every step token attends
// its sequence's positions 0 .. its own through the block table (the step's
// K/V are stored first).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "vm_c/attention_metadata.hpp"
#include "vm_c/kernels_attention.hpp"
#include "vm_c/kernels_turboquant.hpp"

namespace vm_c {

class AttentionBackend {
public:
    virtual ~AttentionBackend() = default;

    virtual void store_kv(const void* key, const void* value, void* key_cache, void* value_cache,
                          const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                          int head_dim, int64_t block_size, int64_t cache_stride,
                          hipStream_t stream) = 0;

    virtual void forward_prefill(void* output, const void* query, const void* key,
                                 const void* value, const void* key_cache,
                                 const void* value_cache, const AttentionMetadata& meta,
                                 int num_heads, int num_kv_heads, int head_dim, float scale,
                                 int64_t block_size, ScalarType dtype, hipStream_t stream) = 0;

    virtual void forward_decode(void* output, const void* query, const void* key_cache,
                                const void* value_cache, const AttentionMetadata& meta,
                                int num_heads, int num_kv_heads, int head_dim, float scale,
                                int64_t block_size, ScalarType dtype, hipStream_t stream) = 0;

    virtual size_t workspace_size() const = 0;

    virtual void ensure_workspace(int max_num_batched_tokens, int max_num_seqs,
                                  int num_attention_heads, int num_kv_heads, int head_dim,
                                  int gpu_device) = 0;
};

class PagedAttentionBackend : public AttentionBackend {
public:
    // kv_cache_dtype: "auto" (the activation type), "fp16", "bf16", "q8_0", "q4_0"
    explicit PagedAttentionBackend(const std::string& kv_cache_layout = "nhd",
                                   const std::string& kv_cache_dtype = "auto",
                                   ScalarType activation_dtype = ScalarType::BFLOAT16);
    ~PagedAttentionBackend() override;

    void store_kv(const void* key, const void* value, void* key_cache, void* value_cache,
                  const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                  int64_t block_size, int64_t cache_stride, hipStream_t stream) override;

    void forward_prefill(void* output, const void* query, const void* key, const void* value,
                         const void* key_cache, const void* value_cache,
                         const AttentionMetadata& meta, int num_heads, int num_kv_heads,
                         int head_dim, float scale, int64_t block_size, ScalarType dtype,
                         hipStream_t stream) override;

    void forward_decode(void* output, const void* query, const void* key_cache,
                        const void* value_cache, const AttentionMetadata& meta, int num_heads,
                        int num_kv_heads, int head_dim, float scale, int64_t block_size,
                        ScalarType dtype, hipStream_t stream) override;

    // split-KV decode workspace, also the local prefill's V^T tiles (0 until
    // ensure_workspace)
    size_t workspace_size() const override { return ws_bytes_; }
    void ensure_workspace(int max_num_batched_tokens, int max_num_seqs, int num_attention_heads,
                          int num_kv_heads, int head_dim, int gpu_device) override;

private:
    std::string kv_cache_layout_;
    std::string kv_cache_dtype_;
    ScalarType activation_dtype_;
    void* ws_ = nullptr;
    size_t ws_bytes_ = 0;
    int max_num_seqs_ = 0, num_heads_ = 0;
};

class TurboQuantBackend : public AttentionBackend {
public:
    // activation_dtype (no counterpart in vm_c, which reads the process-wide
    // compute dtype): the dtype of key/value in store_kv, and so of the
    // stored norms, scales and zeros
    TurboQuantBackend(int head_dim, const std::string& quant_method, int num_attention_heads,
                      int num_kv_heads, int gpu_device,
                      ScalarType activation_dtype = ScalarType::FLOAT16);
    ~TurboQuantBackend() override;

    void store_kv(const void* key, const void* value, void* key_cache, void* value_cache,
                  const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                  int64_t block_size, int64_t cache_stride, hipStream_t stream) override;

    void forward_prefill(void* output, const void* query, const void* key, const void* value,
                         const void* key_cache, const void* value_cache,
                         const AttentionMetadata& meta, int num_heads, int num_kv_heads,
                         int head_dim, float scale, int64_t block_size, ScalarType dtype,
                         hipStream_t stream) override;

    void forward_decode(void* output, const void* query, const void* key_cache,
                        const void* value_cache, const AttentionMetadata& meta, int num_heads,
                        int num_kv_heads, int head_dim, float scale, int64_t block_size,
                        ScalarType dtype, hipStream_t stream) override;

    size_t workspace_size() const override;
    void ensure_workspace(int max_num_batched_tokens, int max_num_seqs, int num_attention_heads,
                          int num_kv_heads, int head_dim, int gpu_device) override;

    const TQConfig& config() const { return config_; }

private:
    TQBuffers buffers_;
    TQConfig config_;
    TQWorkspace workspace_;
    void* prefill_ws_ = nullptr;  // the local prefill's V^T tiles (ensure_workspace)
    size_t prefill_ws_bytes_ = 0;
    int gpu_device_;
    ScalarType activation_dtype_;
    int max_num_batched_tokens_ = 0;
    int max_num_seqs_ = 0;
    int num_attention_heads_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
};

}  // namespace vm_c
