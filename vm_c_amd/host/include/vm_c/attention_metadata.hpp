// vm_c/attention_metadata.hpp -- per-step batch metadata handed to the
// attention operators (vm_c include/vm_c/model/attention_metadata.hpp:8-28,
// same fields and meaning), plus the host-side builder that fills it the way
// vm_c's Engine does (src/core/engine.cpp:653-793).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "vm_c/common.hpp"

namespace vm_c {

struct AttentionMetadata {
    int32_t* block_tables = nullptr;   // device [num_reqs][max_num_blocks_per_req], -1 pad
    int32_t* seq_lens = nullptr;       // device [num_reqs], tokens including this step's
    int64_t* slot_mapping = nullptr;   // device [num_tokens], block_id*block_size+pos%block_size, -1 pad
    int32_t* token_to_seq = nullptr;   // device [num_tokens] (prefill tokens)
    const int32_t* host_token_to_seq = nullptr;
    int32_t* token_positions = nullptr;  // device [num_tokens] (prefill tokens)
    const int32_t* cu_seqlens = nullptr;  // host [num_reqs + 1]
    int num_reqs = 0;
    int num_tokens = 0;
    int max_num_blocks_per_req = 0;
    int block_size = 0;
    int num_prev_tokens = 0;
    int num_computed_tokens = 0;
    int num_prefills = 0;
    int num_prefill_tokens = 0;
    int num_decodes = 0;
    int num_decode_tokens = 0;
    bool is_prefill = false;
    float decode_threshold = 0.0f;
};

class KVCacheManager;

// One scheduled request of a step: vm_c's Request fields the metadata needs.
struct ScheduledRequest {
    std::string request_id;
    int num_computed_tokens = 0;  // tokens already in the cache
    int num_scheduled_tokens = 1;  // tokens computed this step (1 for decode)
    bool is_prefill = false;
    std::vector<uint64_t> prefix_block_hashes;
    int num_cached_tokens = 0;
    std::vector<int64_t> computed_block_ids;
};

// Host images of the metadata arrays, built exactly as the Engine builds
// them: slots are allocated through the block manager for
// num_computed + num_scheduled (+ lookahead) tokens; prefill tokens map to
// positions num_computed .. +num_scheduled-1, a decode token to position
// num_computed; seq_lens = num_computed + num_scheduled; block tables are
// row-major, padded with -1 to the widest request.
struct HostBatchMetadata {
    std::vector<int64_t> slot_mapping;
    std::vector<int32_t> seq_lens;
    std::vector<int32_t> token_to_seq;
    std::vector<int32_t> token_positions;
    std::vector<int32_t> cu_seqlens;
    std::vector<int32_t> block_tables;
    int num_reqs = 0;
    int num_tokens = 0;
    int max_num_blocks_per_req = 0;
    int num_prefills = 0;
    int num_prefill_tokens = 0;
    int num_decodes = 0;
    int num_decode_tokens = 0;
    int num_computed_tokens = 0;  // cached-prefix tokens of the prefill requests
    bool ok = true;  // false if the block manager could not allocate
};

HostBatchMetadata build_batch_metadata(KVCacheManager& mgr,
                                       const std::vector<ScheduledRequest>& reqs,
                                       int kv_lookahead_tokens = 0);

// Device buffers for one step's metadata, sized once for the largest batch.
class DeviceBatchMetadata {
public:
    DeviceBatchMetadata(int max_num_reqs, int max_num_tokens, int max_num_blocks_per_req);
    ~DeviceBatchMetadata();
    DeviceBatchMetadata(const DeviceBatchMetadata&) = delete;
    DeviceBatchMetadata& operator=(const DeviceBatchMetadata&) = delete;

    // stream-ordered host->device copies; the host vectors must stay alive
    // until the stream has executed them (vm_c keeps them in the Engine)
    AttentionMetadata upload(const HostBatchMetadata& h, int block_size, hipStream_t stream);

private:
    int max_reqs_, max_tokens_, max_blocks_;
    int32_t* block_tables_ = nullptr;
    int32_t* seq_lens_ = nullptr;
    int64_t* slot_mapping_ = nullptr;
    int32_t* token_to_seq_ = nullptr;
    int32_t* token_positions_ = nullptr;
};

}  // namespace vm_c
