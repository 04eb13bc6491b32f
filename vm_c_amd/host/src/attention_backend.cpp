// attention_backend.cpp -- the operator interface src/model uses
// (vm_c src/model/attention_backend.cpp:15-238) over the gfx950 kernels.
#include "vm_c/attention_backend.hpp"

namespace vm_c {

namespace {
void require_no_cached_prefix(const AttentionMetadata& meta, const char* who) {
    if (meta.num_computed_tokens > 0 || meta.num_decode_tokens > 0)
        throw std::runtime_error(std::string(who) +
                                 ": prefill over a cached prefix or mixed with decode tokens is "
                                 "not on this path (split the batch: decode rows go to forward_decode)");
}
}  // namespace

// ------------------------------------------------------------ paged

PagedAttentionBackend::PagedAttentionBackend(const std::string& kv_cache_layout,
                                             const std::string& kv_cache_dtype,
                                             ScalarType activation_dtype)
    : kv_cache_layout_(kv_cache_layout.empty() ? "nhd" : kv_cache_layout),
      kv_cache_dtype_(kv_cache_dtype.empty() ? "auto" : kv_cache_dtype),
      activation_dtype_(activation_dtype) {
    (void)vmc_layout_of(kv_cache_layout_);
    (void)vmc_kv_format_of(kv_cache_dtype_, activation_dtype_);
}

PagedAttentionBackend::~PagedAttentionBackend() {
    if (ws_) (void)hipFree(ws_);
}

// attention_backend.cpp:15-32 (the reference stores the activation type)
void PagedAttentionBackend::store_kv(const void* key, const void* value, void* key_cache,
                                     void* value_cache, const int64_t* slot_mapping, int num_tokens,
                                     int num_kv_heads, int head_dim, int64_t block_size,
                                     int64_t cache_stride, hipStream_t stream) {
    reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_kv_heads,
                      head_dim, block_size, cache_stride, kv_cache_dtype_, nullptr, nullptr,
                      activation_dtype_, stream, kv_cache_layout_);
}

// attention_backend.cpp:34-65: causal prefill of this step's tokens.  The
// local K/V of the step are the whole context when nothing is cached yet.
void PagedAttentionBackend::forward_prefill(void* output, const void* query, const void* key,
                                            const void* value, const void* key_cache,
                                            const void* value_cache, const AttentionMetadata& meta,
                                            int num_heads, int num_kv_heads, int head_dim,
                                            float scale, int64_t block_size, ScalarType dtype,
                                            hipStream_t stream) {
    if (meta.num_computed_tokens > 0 && meta.num_decode_tokens == 0) {
        // a cached prefix: attend through the pages (store_kv has appended
        // this step's tokens) with the tiled kernel the reference's
        // flash_attention_prefill_v2 call stands for
        flash_attention_prefill_v2(output, query, key_cache, value_cache, meta.num_tokens, num_heads,
                                   num_kv_heads, head_dim, scale, block_size, meta.max_num_blocks_per_req,
                                   meta.block_tables, meta.seq_lens, meta.token_to_seq,
                                   meta.token_positions, meta.num_reqs, kv_cache_dtype_, dtype, stream,
                                   kv_cache_layout_);
        return;
    }
    require_no_cached_prefix(meta, "PagedAttentionBackend::forward_prefill");
    if (!key || !value) throw std::runtime_error("PagedAttentionBackend::forward_prefill: needs the step's K/V");
    if (ws_ && vmc_flash_attention_prefill_workspace_size(meta.num_tokens, num_kv_heads, head_dim) <= ws_bytes_) {
        // the step's V^T tiles built once in the workspace
        VMC_CALL(vmc_flash_attention_prefill_ws(output, query, key, value, meta.num_tokens, num_heads, num_kv_heads,
                                                head_dim, scale, meta.token_positions, vmc_dtype_of(dtype), nullptr,
                                                nullptr, nullptr, 16, VMC_KV_F16, VMC_LAYOUT_NHD, ws_, ws_bytes_,
                                                reinterpret_cast<vmc_stream_t>(stream)));
        return;
    }
    flash_attention_prefill_local(output, query, key, value, meta.num_tokens, num_heads, num_kv_heads,
                                  head_dim, scale, meta.token_to_seq, meta.token_positions, dtype, stream);
}

// attention_backend.cpp:67-99: one query row per request
void PagedAttentionBackend::forward_decode(void* output, const void* query, const void* key_cache,
                                           const void* value_cache, const AttentionMetadata& meta,
                                           int num_heads, int num_kv_heads, int head_dim, float scale,
                                           int64_t block_size, ScalarType dtype, hipStream_t stream) {
    AttentionParams p;
    p.batch_size = meta.num_reqs;
    p.num_tokens = meta.num_tokens;
    p.num_heads = num_heads;
    p.num_kv_heads = num_kv_heads;
    p.head_dim = head_dim;
    p.block_size = (int)block_size;
    p.max_num_blocks_per_req = meta.max_num_blocks_per_req;
    p.max_seq_len = meta.max_num_blocks_per_req * (int)block_size;
    p.scale = scale;
    p.dtype = dtype;
    const size_t need = paged_attention_v2_workspace_size(p);
    if (ws_ && need <= ws_bytes_) {
        paged_attention_v2(output, nullptr, nullptr, ws_, query, key_cache, value_cache, p,
                           meta.block_tables, meta.seq_lens, nullptr, kv_cache_dtype_, nullptr,
                           nullptr, stream, kv_cache_layout_);
    } else {
        paged_attention_v1(output, query, key_cache, value_cache, p, meta.block_tables, meta.seq_lens,
                           nullptr, kv_cache_dtype_, nullptr, nullptr, stream, kv_cache_layout_);
    }
}

// pre-sizes the split workspace for max_num_seqs requests of up to 32768
// tokens (a batch that needs more runs one pass per request, without it),
// and the local prefill's V^T tiles for max_num_batched_tokens tokens (the
// same buffer: prefill and decode calls are ordered on the stream)
void PagedAttentionBackend::ensure_workspace(int max_num_batched_tokens, int max_num_seqs,
                                             int num_attention_heads, int num_kv_heads,
                                             int head_dim, int gpu_device) {
    const size_t need = std::max(vmc_paged_decode_workspace_size(max_num_seqs, num_attention_heads, num_kv_heads,
                                                                 head_dim, 32768 / 16, 16, 0),
                                 vmc_flash_attention_prefill_workspace_size(max_num_batched_tokens, num_kv_heads,
                                                                            head_dim));
    if (need <= ws_bytes_) return;
    HIP_CHECK(hipSetDevice(gpu_device));
    if (ws_) HIP_CHECK(hipFree(ws_));
    ws_ = nullptr;
    ws_bytes_ = 0;
    HIP_CHECK(hipMalloc(&ws_, need));
    ws_bytes_ = need;
    max_num_seqs_ = max_num_seqs;
    num_heads_ = num_attention_heads;
}

// ------------------------------------------------------------ TurboQuant

// attention_backend.cpp:101-113
TurboQuantBackend::TurboQuantBackend(int head_dim, const std::string& quant_method,
                                     int num_attention_heads, int num_kv_heads, int gpu_device,
                                     ScalarType activation_dtype)
    : gpu_device_(gpu_device), activation_dtype_(activation_dtype),
      num_attention_heads_(num_attention_heads), num_kv_heads_(num_kv_heads), head_dim_(head_dim) {
    if (activation_dtype != ScalarType::FLOAT16 && activation_dtype != ScalarType::BFLOAT16)
        throw std::runtime_error("TurboQuantBackend: activations must be fp16 or bf16");
    HIP_CHECK(hipSetDevice(gpu_device_));
    config_ = TQConfig::from_method(head_dim, quant_method.c_str(), gpu_device_);
    // fp8 keys (turboquant_k8v4) use no codebook and no rotation
    if (!config_.key_fp8) buffers_.init(head_dim, config_.key_quant_bits, gpu_device);
}

TurboQuantBackend::~TurboQuantBackend() {
    buffers_.free_buf();
    workspace_.free_buf();
    if (prefill_ws_) (void)hipFree(prefill_ws_);
}

// attention_backend.cpp:120-136: the decode workspace for max_num_seqs
// requests of any length (the split count, and so the workspace, stops
// growing with the context once every CU has a page range), so no decode
// call of up to max_num_seqs requests allocates
void TurboQuantBackend::ensure_workspace(int max_num_batched_tokens, int max_num_seqs,
                                         int num_attention_heads, int num_kv_heads, int head_dim,
                                         int gpu_device) {
    max_num_batched_tokens_ = max_num_batched_tokens;
    max_num_seqs_ = max_num_seqs;
    num_attention_heads_ = num_attention_heads;
    num_kv_heads_ = num_kv_heads;
    head_dim_ = head_dim;
    workspace_.ensure_decode(max_num_seqs, num_attention_heads, num_kv_heads, head_dim,
                             int64_t{1} << 26, 16, config_.max_num_kv_splits, gpu_device);
    // the local prefill's V^T tiles for max_num_batched_tokens tokens
    const size_t pneed = vmc_flash_attention_prefill_workspace_size(max_num_batched_tokens, num_kv_heads, head_dim);
    if (pneed > prefill_ws_bytes_) {
        HIP_CHECK(hipSetDevice(gpu_device));
        if (prefill_ws_) HIP_CHECK(hipFree(prefill_ws_));
        prefill_ws_ = nullptr;
        prefill_ws_bytes_ = 0;
        HIP_CHECK(hipMalloc(&prefill_ws_, pneed));
        prefill_ws_bytes_ = pneed;
    }
}

void TurboQuantBackend::store_kv(const void* key, const void* value, void* key_cache,
                                 void* value_cache, const int64_t* slot_mapping, int num_tokens,
                                 int num_kv_heads, int head_dim, int64_t block_size,
                                 int64_t cache_stride, hipStream_t stream) {
    (void)value_cache;
    (void)cache_stride;
    turboquant_store(key, value, key_cache, slot_mapping, num_tokens, num_kv_heads, head_dim,
                     block_size, config_, buffers_, workspace_, stream, activation_dtype_);
}

// attention_backend.cpp:153-197: prefill runs on the step's local K/V
void TurboQuantBackend::forward_prefill(void* output, const void* query, const void* key,
                                        const void* value, const void* key_cache,
                                        const void* value_cache, const AttentionMetadata& meta,
                                        int num_heads, int num_kv_heads, int head_dim, float scale,
                                        int64_t block_size, ScalarType dtype, hipStream_t stream) {
    (void)value_cache;
    if (meta.num_computed_tokens > 0 && meta.num_decode_tokens == 0) {
        // a cached prefix: one row per token through the packed pages
        // (store_kv has appended this step's tokens); the reference attends
        // only the local K/V here
        const vmc_tq_config c = config_.to_c();
        VMC_CALL(vmc_turboquant_prefill_attention(
            output, query, key_cache, meta.block_tables, meta.token_to_seq, meta.token_positions,
            meta.num_tokens, num_heads, num_kv_heads, head_dim, scale, block_size,
            meta.max_num_blocks_per_req, &c, vmc_dtype_of(dtype), 1, nullptr, 0, stream));
        return;
    }
    require_no_cached_prefix(meta, "TurboQuantBackend::forward_prefill");
    if (prefill_ws_ &&
        vmc_flash_attention_prefill_workspace_size(meta.num_tokens, num_kv_heads, head_dim) <= prefill_ws_bytes_) {
        VMC_CALL(vmc_flash_attention_prefill_ws(output, query, key, value, meta.num_tokens, num_heads, num_kv_heads,
                                                head_dim, scale, meta.token_positions, vmc_dtype_of(dtype), nullptr,
                                                nullptr, nullptr, 16, VMC_KV_F16, VMC_LAYOUT_NHD, prefill_ws_,
                                                prefill_ws_bytes_, reinterpret_cast<vmc_stream_t>(stream)));
        return;
    }
    flash_attention_prefill_local(output, query, key, value, meta.num_tokens, num_heads, num_kv_heads,
                                  head_dim, scale, meta.token_to_seq, meta.token_positions, dtype, stream);
}

// attention_backend.cpp:199-215
void TurboQuantBackend::forward_decode(void* output, const void* query, const void* key_cache,
                                       const void* value_cache, const AttentionMetadata& meta,
                                       int num_heads, int num_kv_heads, int head_dim, float scale,
                                       int64_t block_size, ScalarType dtype, hipStream_t stream) {
    (void)value_cache;
    if (dtype != activation_dtype_)
        throw std::runtime_error("TurboQuantBackend::forward_decode: query dtype differs from the "
                                 "activation dtype the pages were stored in");
    turboquant_decode_attention(output, query, key_cache, meta.block_tables, meta.seq_lens,
                                meta.num_reqs, num_heads, num_kv_heads, head_dim, scale, block_size,
                                meta.max_num_blocks_per_req, config_, buffers_, workspace_,
                                config_.max_num_kv_splits, stream, dtype);
}

size_t TurboQuantBackend::workspace_size() const { return workspace_.decode_bytes + prefill_ws_bytes_; }

}  // namespace vm_c
