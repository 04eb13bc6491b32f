// vm_c/turboquant_kv_bridge.hpp -- the TurboQuant attention node of a ggml
// graph (vm_c include/vm_c/official/turboquant_kv_bridge.hpp:18-113,
// src/official/turboquant_kv_bridge.cpp:45-114, :134-254) over the HIP
// kernels.
//
// The reference registers ggml_cuda_vm_c_turboquant_attn_impl(ggml_tensor*)
// as the CUDA body of GGML_OP_VM_C_TURBOQUANT_ATTN.  The node carries
// op_params = {int32 layer, float kq_scale, TurboQuantKvBridge*} and sources
// q, k, v; the body appends k / v into the layer's TurboQuant slots through
// the bridge's slot mapping, then runs the paged decode over the bridge's
// block tables and sequence lengths with one query row per token.
// turboquant_attn_op is that body over the node's raw fields (data pointers,
// q's ne / nb), so this library needs no ggml headers; the four-line callback
// a ggml build registers is shown in INTEGRATION.md.  The ggml tensor wrappers
// of the layer pools (kv_cache_tensor) belong to the graph side and are not
// made here: kv_cache_ptr gives the same memory.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "vm_c/common.hpp"
#include "vm_c/kernels_turboquant.hpp"
#include "vm_c/kv_cache_manager.hpp"

namespace vm_c::official {

// Byte offsets of the node's op_params (turboquant_kv_bridge.cpp:46-50).
constexpr size_t kTqAttnOpLayer = 0;                                    // int32_t
constexpr size_t kTqAttnOpScale = sizeof(int32_t);                      // float
constexpr size_t kTqAttnOpBridge = sizeof(int32_t) + sizeof(float);     // TurboQuantKvBridge*
constexpr size_t kTqAttnOpBytes = kTqAttnOpBridge + sizeof(void*);

class TurboQuantKvBridge {
public:
    TurboQuantKvBridge() = default;
    ~TurboQuantKvBridge();

    TurboQuantKvBridge(const TurboQuantKvBridge&) = delete;
    TurboQuantKvBridge& operator=(const TurboQuantKvBridge&) = delete;

    // The model fields the reference reads from VmCConfig (num_attention_heads,
    // num_key_value_heads, head_dim; cache.kv_cache_quant_method), split by
    // tp_size as its column TP does.  compute_dtype is the activation type of
    // q / k / v / out and of the stored norms and scales (the reference's
    // gpu().compute_dtype(): bf16 where the GPU has it).  Throws
    // std::runtime_error as the reference does.
    void initialize(const CacheConfig& cache, int num_attention_heads, int num_key_value_heads, int head_dim,
                    KVCacheManager* kv_cache_mgr, int gpu_device, int num_layers, int tp_size = 1,
                    ScalarType compute_dtype = ScalarType::BFLOAT16);

    void set_batch_metadata(const int64_t* d_slot_mapping, const int32_t* d_block_tables, const int32_t* d_seq_lens,
                            int num_tokens, int num_reqs, int max_num_blocks_per_req, int64_t block_size,
                            bool is_prefill, int num_prefill_tokens, int num_decode_tokens,
                            const int32_t* d_token_to_seq, const int32_t* d_token_positions, hipStream_t stream);

    void mark_decode_mode(int num_tokens);

    // Decode workspace for nodes of up to max_num_tokens query rows over
    // max_num_blocks_per_req pages: nodes within it allocate nothing (a
    // larger node grows it before its launch).
    void reserve_decode(int max_num_tokens, int64_t max_num_blocks_per_req);

    bool is_layer_turboquant(int layer) const {
        return kv_cache_mgr_ && kv_cache_mgr_->is_layer_turboquant(layer);
    }

    const TQConfig& tq_config() const { return tq_config_; }
    // kept for the reference's signature; the HIP kernels read no device tables
    TQBuffers& tq_buffers() { return tq_buffers_; }
    TQWorkspace& tq_workspace() { return tq_workspace_; }
    int gpu_device() const { return gpu_device_; }
    int num_attention_heads() const { return num_attention_heads_; }
    int num_kv_heads() const { return num_kv_heads_; }
    int head_dim() const { return head_dim_; }
    ScalarType compute_dtype() const { return compute_dtype_; }

    int tq_layer_enabled_count() const;

    const int64_t* slot_mapping() const { return d_slot_mapping_; }
    const int32_t* block_tables() const { return d_block_tables_; }
    const int32_t* seq_lens() const { return d_seq_lens_; }
    int num_tokens() const { return num_tokens_; }
    int num_reqs() const { return num_reqs_; }
    int max_num_blocks_per_req() const { return max_num_blocks_per_req_; }
    int64_t block_size() const { return block_size_; }
    bool is_prefill() const { return is_prefill_; }
    int num_prefill_tokens() const { return num_prefill_tokens_; }
    int num_decode_tokens() const { return num_decode_tokens_; }
    const int32_t* token_to_seq() const { return d_token_to_seq_; }
    const int32_t* token_positions() const { return d_token_positions_; }
    hipStream_t stream() const { return stream_; }

    // the layer's slot pool, or null for a layer without TurboQuant slots
    void* kv_cache_ptr(int layer) const;

    // Device rows [2][capacity] (sequence, then position) for num_tokens
    // query tokens of a step with prefill tokens; grown when a step needs
    // more than reserve_decode set aside.
    int32_t* token_rows(int num_tokens);
    int token_rows_capacity() const { return rows_cap_; }

private:
    KVCacheManager* kv_cache_mgr_ = nullptr;
    int gpu_device_ = 0;
    int num_layers_ = 0;
    int num_attention_heads_ = 0;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    ScalarType compute_dtype_ = ScalarType::BFLOAT16;

    TQConfig tq_config_;
    TQBuffers tq_buffers_;
    TQWorkspace tq_workspace_;

    std::vector<void*> kv_ptrs_;
    int32_t* d_rows_ = nullptr;
    int rows_cap_ = 0;

    const int64_t* d_slot_mapping_ = nullptr;
    const int32_t* d_block_tables_ = nullptr;
    const int32_t* d_seq_lens_ = nullptr;
    int num_tokens_ = 0;
    int num_reqs_ = 0;
    int max_num_blocks_per_req_ = 0;
    int64_t block_size_ = 0;
    bool is_prefill_ = false;
    int num_prefill_tokens_ = 0;
    int num_decode_tokens_ = 0;
    const int32_t* d_token_to_seq_ = nullptr;
    const int32_t* d_token_positions_ = nullptr;
    hipStream_t stream_ = nullptr;
};

// The node body (ggml_cuda_vm_c_turboquant_attn_impl,
// turboquant_kv_bridge.cpp:45-114): op_params as laid out above; q, k, v and
// dst the data of src[0], src[1], src[2] and the node; q_ne / q_nb q's ne[4] /
// nb[4].  q is [head_dim, n_head, n_tokens] (nb[2] != 0 and ne[1] > 1) or
// [n_embd, n_tokens]; k / v hold n_tokens x num_kv_heads x head_dim values,
// dst n_tokens x n_embd.  Throws std::runtime_error (null bridge, q width
// other than num_attention_heads x head_dim, a layer without slots, no slot
// mapping) before any launch, as the reference does.
//
// The attention reads the batch metadata as vm_c's Engine uploads it
// (engine.cpp:653-793): block tables and sequence lengths per request.  A
// decode-only step (is_prefill false) has one token per request and runs the
// paged decode over num_reqs rows.  A step with prefill tokens gets one
// (sequence, position) row per token (vmc_batch_token_rows: the prefill
// tokens' token_to_seq / token_positions, each decode token's request and
// seq_lens - 1) and runs the paged prefill attention over those rows.  (The
// reference decodes num_tokens rows over the per-request arrays in every
// step, reading past both whenever a step holds prefill tokens.)  Also
// throws for a decode-only step whose token count differs from its request
// count, and for a prefill step without token_to_seq / token_positions.
void turboquant_attn_op(const void* op_params, const void* q, const int64_t q_ne[4], const size_t q_nb[4],
                        const void* k, const void* v, void* dst);

}  // namespace vm_c::official

// turboquant_kv_bridge.cpp:226-231: whether the graph builder should emit the
// TurboQuant node for this layer (false for a null bridge)
extern "C" bool vm_c_tq_bridge_layer_uses_turboquant(void* bridge, int32_t layer);
