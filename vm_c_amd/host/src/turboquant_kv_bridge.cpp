// turboquant_kv_bridge.cpp -- the TurboQuant attention node over the HIP
// kernels (vm_c src/official/turboquant_kv_bridge.cpp:28-114, :118-254).
#include "vm_c/turboquant_kv_bridge.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace vm_c::official {
namespace {

// q is the head-split view [head_dim, n_head, n_tokens] when its third stride
// is set and its second extent exceeds one (turboquant_kv_bridge.cpp:28-43)
bool q_is_head_split_3d(const int64_t ne[4], const size_t nb[4]) { return nb[2] != 0 && ne[1] > 1; }

void q_layout(const int64_t ne[4], const size_t nb[4], int* n_embd, int* num_tokens) {
    if (q_is_head_split_3d(ne, nb)) {
        *n_embd = static_cast<int>(ne[0] * ne[1]);
        *num_tokens = static_cast<int>(ne[2]);
    } else {
        *n_embd = static_cast<int>(ne[0]);
        *num_tokens = static_cast<int>(ne[1]);
    }
}

}  // namespace

TurboQuantKvBridge::~TurboQuantKvBridge() {
    tq_buffers_.free_buf();
    tq_workspace_.free_buf();
    if (d_rows_) (void)hipFree(d_rows_);
}

int32_t* TurboQuantKvBridge::token_rows(int num_tokens) {
    if (num_tokens > rows_cap_) {
        HIP_CHECK(hipSetDevice(gpu_device_));
        if (d_rows_) HIP_CHECK(hipFree(d_rows_));
        d_rows_ = nullptr;
        rows_cap_ = 0;
        HIP_CHECK(hipMalloc(&d_rows_, sizeof(int32_t) * 2 * (size_t)num_tokens));
        rows_cap_ = num_tokens;
    }
    return d_rows_;
}

void TurboQuantKvBridge::initialize(const CacheConfig& cache, int num_attention_heads, int num_key_value_heads,
                                    int head_dim, KVCacheManager* kv_cache_mgr, int gpu_device, int num_layers,
                                    int tp_size, ScalarType compute_dtype) {
    if (!kv_cache_mgr || !kv_cache_mgr->is_turboquant()) {
        throw std::runtime_error("TurboQuantKvBridge::initialize: KVCacheManager is not TurboQuant");
    }
    if (tp_size <= 0) {
        throw std::runtime_error("TurboQuantKvBridge::initialize: tp_size must be positive");
    }
    if (compute_dtype != ScalarType::FLOAT16 && compute_dtype != ScalarType::BFLOAT16) {
        throw std::runtime_error("TurboQuantKvBridge::initialize: compute dtype must be fp16 or bf16");
    }
    kv_cache_mgr_ = kv_cache_mgr;
    gpu_device_ = gpu_device;
    num_layers_ = num_layers;
    // column TP: each rank holds num_heads / tp_size query heads and at least
    // one KV head (turboquant_kv_bridge.cpp:151-153)
    num_attention_heads_ = num_attention_heads / tp_size;
    num_kv_heads_ = std::max(1, num_key_value_heads / tp_size);
    head_dim_ = head_dim;
    compute_dtype_ = compute_dtype;
    if (num_attention_heads_ <= 0) {
        throw std::runtime_error("TurboQuantKvBridge::initialize: num_attention_heads per rank is zero");
    }
    tq_config_ = TQConfig::from_method(head_dim_, cache.kv_cache_quant_method.c_str(), gpu_device_);
    // the reference sizes its decode workspace here (turboquant_kv_bridge.cpp:
    // 162-163); this one allocates nothing until reserve_decode or the first
    // node, so set-up stays free of device calls
    kv_ptrs_.assign(static_cast<size_t>(std::max(num_layers, 0)), nullptr);
    for (int l = 0; l < num_layers; ++l)
        if (kv_cache_mgr_->is_layer_turboquant(l)) kv_ptrs_[static_cast<size_t>(l)] = kv_cache_mgr_->key_cache_ptr(l);
}

void TurboQuantKvBridge::set_batch_metadata(const int64_t* d_slot_mapping, const int32_t* d_block_tables,
                                            const int32_t* d_seq_lens, int num_tokens, int num_reqs,
                                            int max_num_blocks_per_req, int64_t block_size, bool is_prefill,
                                            int num_prefill_tokens, int num_decode_tokens,
                                            const int32_t* d_token_to_seq, const int32_t* d_token_positions,
                                            hipStream_t stream) {
    d_slot_mapping_ = d_slot_mapping;
    d_block_tables_ = d_block_tables;
    d_seq_lens_ = d_seq_lens;
    num_tokens_ = num_tokens;
    num_reqs_ = num_reqs;
    max_num_blocks_per_req_ = max_num_blocks_per_req;
    block_size_ = block_size;
    is_prefill_ = is_prefill;
    num_prefill_tokens_ = num_prefill_tokens;
    num_decode_tokens_ = num_decode_tokens;
    d_token_to_seq_ = d_token_to_seq;
    d_token_positions_ = d_token_positions;
    stream_ = stream;
}

void TurboQuantKvBridge::mark_decode_mode(int num_tokens) {
    is_prefill_ = false;
    num_prefill_tokens_ = 0;
    num_decode_tokens_ = num_tokens;
    num_tokens_ = num_tokens;
}

void TurboQuantKvBridge::reserve_decode(int max_num_tokens, int64_t max_num_blocks_per_req) {
    if (!kv_cache_mgr_) throw std::runtime_error("TurboQuantKvBridge::reserve_decode: not initialized");
    tq_workspace_.ensure_decode(max_num_tokens, num_attention_heads_, num_kv_heads_, head_dim_,
                                max_num_blocks_per_req, kv_cache_mgr_->block_size(),
                                tq_config_.max_num_kv_splits, gpu_device_);
    if (max_num_tokens > 0) token_rows(max_num_tokens);
}

void* TurboQuantKvBridge::kv_cache_ptr(int layer) const {
    if (layer < 0 || static_cast<size_t>(layer) >= kv_ptrs_.size()) return nullptr;
    return kv_ptrs_[static_cast<size_t>(layer)];
}

int TurboQuantKvBridge::tq_layer_enabled_count() const {
    if (!kv_cache_mgr_) return 0;
    int n = 0;
    for (int l = 0; l < kv_cache_mgr_->num_layers(); ++l)
        if (kv_cache_mgr_->is_layer_turboquant(l)) ++n;
    return n;
}

void turboquant_attn_op(const void* op_params, const void* q, const int64_t q_ne[4], const size_t q_nb[4],
                        const void* k, const void* v, void* dst) {
    int32_t layer = 0;
    float kq_scale = 0.0f;
    void* bridge_ptr = nullptr;
    const auto* pb = static_cast<const unsigned char*>(op_params);
    std::memcpy(&layer, pb + kTqAttnOpLayer, sizeof(layer));
    std::memcpy(&kq_scale, pb + kTqAttnOpScale, sizeof(kq_scale));
    std::memcpy(&bridge_ptr, pb + kTqAttnOpBridge, sizeof(bridge_ptr));
    auto* bridge = static_cast<TurboQuantKvBridge*>(bridge_ptr);
    if (!bridge) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: null bridge");
    }
    int n_embd = 0, num_tokens = 0;
    q_layout(q_ne, q_nb, &n_embd, &num_tokens);
    const int num_heads = bridge->num_attention_heads();
    const int num_kv_heads = bridge->num_kv_heads();
    const int head_dim = bridge->head_dim();
    if (n_embd != num_heads * head_dim) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: q embedding dim mismatch: ne0=" + std::to_string(n_embd) +
                                 " expected=" + std::to_string(num_heads * head_dim));
    }
    void* kv_cache = bridge->kv_cache_ptr(layer);
    if (!kv_cache) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: null kv cache for layer " + std::to_string(layer));
    }
    const int64_t* slot_mapping = bridge->slot_mapping();
    if (!slot_mapping) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: slot_mapping not set");
    }
    // the batch metadata is checked before any launch
    const int num_reqs = bridge->num_reqs();
    const bool decode_only = !bridge->is_prefill();
    if (decode_only && num_tokens != num_reqs) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: decode step of " + std::to_string(num_tokens) +
                                 " tokens over " + std::to_string(num_reqs) +
                                 " requests (token_to_seq / token_positions are set only with prefill tokens)");
    }
    if (!decode_only && num_tokens > 0 &&
        (!bridge->token_to_seq() || !bridge->token_positions() || !bridge->seq_lens() || num_reqs <= 0)) {
        throw std::runtime_error("ggml_vm_c_turboquant_attn: prefill step without token_to_seq / token_positions");
    }
    hipStream_t stream = bridge->stream();
    const ScalarType dtype = bridge->compute_dtype();
    turboquant_store(k, v, kv_cache, slot_mapping, num_tokens, num_kv_heads, head_dim, bridge->block_size(),
                     bridge->tq_config(), bridge->tq_buffers(), bridge->tq_workspace(), stream, dtype);
    const int splits = bridge->tq_config().max_num_kv_splits;
    if (decode_only) {
        // token t is request t's one query row
        turboquant_decode_attention(dst, q, kv_cache, bridge->block_tables(), bridge->seq_lens(), num_reqs,
                                    num_heads, num_kv_heads, head_dim, kq_scale, bridge->block_size(),
                                    bridge->max_num_blocks_per_req(), bridge->tq_config(), bridge->tq_buffers(),
                                    bridge->tq_workspace(), splits, stream, dtype);
        return;
    }
    // prefill or mixed step: one (sequence, position) row per token
    if (num_tokens == 0) return;
    int32_t* rows = bridge->token_rows(num_tokens);
    int32_t* row_pos = rows + bridge->token_rows_capacity();
    VMC_CALL(vmc_batch_token_rows(rows, row_pos, bridge->token_to_seq(), bridge->token_positions(),
                                  bridge->seq_lens(), num_tokens, num_reqs, stream));
    TQWorkspace& ws = bridge->tq_workspace();
    ws.ensure_decode(num_tokens, num_heads, num_kv_heads, head_dim, bridge->max_num_blocks_per_req(),
                     bridge->block_size(), splits, bridge->gpu_device());
    const vmc_tq_config c = bridge->tq_config().to_c();
    VMC_CALL(vmc_turboquant_prefill_attention(dst, q, kv_cache, bridge->block_tables(), rows, row_pos, num_tokens,
                                              num_heads, num_kv_heads, head_dim, kq_scale, bridge->block_size(),
                                              bridge->max_num_blocks_per_req(), &c, vmc_dtype_of(dtype), splits,
                                              ws.decode_workspace, ws.decode_bytes, stream));
}

}  // namespace vm_c::official

extern "C" bool vm_c_tq_bridge_layer_uses_turboquant(void* bridge, int32_t layer) {
    if (!bridge) return false;
    return static_cast<vm_c::official::TurboQuantKvBridge*>(bridge)->is_layer_turboquant(layer);
}
