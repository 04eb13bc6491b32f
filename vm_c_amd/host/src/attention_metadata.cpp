// attention_metadata.cpp -- host-side metadata builder (the Engine's step
// preparation, src/core/engine.cpp:653-793) and its device buffers.
#include "vm_c/attention_metadata.hpp"

#include <algorithm>

#include "vm_c/kv_cache_manager.hpp"

namespace vm_c {

HostBatchMetadata build_batch_metadata(KVCacheManager& mgr, const std::vector<ScheduledRequest>& reqs,
                                       int kv_lookahead_tokens) {
    HostBatchMetadata h;
    const int64_t bs = mgr.block_size();
    h.num_reqs = (int)reqs.size();
    int total = 0;
    for (const auto& r : reqs) total += r.is_prefill ? r.num_scheduled_tokens : 1;
    h.num_tokens = total;
    h.slot_mapping.assign(total, -1);
    h.seq_lens.assign(h.num_reqs, 0);
    h.token_to_seq.assign(total, 0);
    h.token_positions.assign(total, 0);
    h.cu_seqlens.assign(h.num_reqs + 1, 0);
    std::vector<std::vector<int64_t>> ids(h.num_reqs);
    int off = 0;
    for (int ri = 0; ri < h.num_reqs; ++ri) {
        const auto& r = reqs[ri];
        const int nsched = r.is_prefill ? r.num_scheduled_tokens : 1;
        auto slots = mgr.allocate_slots(r.request_id, r.num_computed_tokens + nsched + kv_lookahead_tokens,
                                        r.prefix_block_hashes, r.num_cached_tokens, r.computed_block_ids);
        if (slots.empty() && r.num_computed_tokens + nsched + kv_lookahead_tokens > 0) h.ok = false;
        for (const auto& s : slots) ids[ri].push_back(s.block_id);
        h.max_num_blocks_per_req = std::max(h.max_num_blocks_per_req, (int)slots.size());
        for (int i = 0; i < nsched; ++i) {
            const int pos = r.num_computed_tokens + i;
            const int64_t blk = pos / bs, in_blk = pos % bs;
            if (r.is_prefill) {
                h.token_to_seq[off + i] = ri;
                h.token_positions[off + i] = pos;
            }
            if (blk < (int64_t)slots.size()) h.slot_mapping[off + i] = slots[blk].block_id * bs + in_blk;
        }
        if (r.is_prefill) {
            ++h.num_prefills;
            h.num_prefill_tokens += nsched;
            h.num_computed_tokens += r.num_computed_tokens;
        } else {
            ++h.num_decodes;
            h.num_decode_tokens += 1;
        }
        h.seq_lens[ri] = r.num_computed_tokens + nsched;
        h.cu_seqlens[ri + 1] = h.cu_seqlens[ri] + nsched;
        off += nsched;
    }
    const int mb = h.max_num_blocks_per_req;
    h.block_tables.assign((size_t)h.num_reqs * mb, -1);
    for (int ri = 0; ri < h.num_reqs; ++ri)
        for (size_t bi = 0; bi < ids[ri].size(); ++bi) h.block_tables[(size_t)ri * mb + bi] = (int32_t)ids[ri][bi];
    return h;
}

DeviceBatchMetadata::DeviceBatchMetadata(int max_num_reqs, int max_num_tokens, int max_num_blocks_per_req)
    : max_reqs_(max_num_reqs), max_tokens_(max_num_tokens), max_blocks_(max_num_blocks_per_req) {
    HIP_CHECK(hipMalloc(&block_tables_, sizeof(int32_t) * std::max(1, max_reqs_ * max_blocks_)));
    HIP_CHECK(hipMalloc(&seq_lens_, sizeof(int32_t) * std::max(1, max_reqs_)));
    HIP_CHECK(hipMalloc(&slot_mapping_, sizeof(int64_t) * std::max(1, max_tokens_)));
    HIP_CHECK(hipMalloc(&token_to_seq_, sizeof(int32_t) * std::max(1, max_tokens_)));
    HIP_CHECK(hipMalloc(&token_positions_, sizeof(int32_t) * std::max(1, max_tokens_)));
}

DeviceBatchMetadata::~DeviceBatchMetadata() {
    for (void* p : {(void*)block_tables_, (void*)seq_lens_, (void*)slot_mapping_, (void*)token_to_seq_,
                    (void*)token_positions_})
        if (p) (void)hipFree(p);
}

AttentionMetadata DeviceBatchMetadata::upload(const HostBatchMetadata& h, int block_size, hipStream_t s) {
    if (h.num_reqs > max_reqs_ || h.num_tokens > max_tokens_ || h.max_num_blocks_per_req > max_blocks_)
        throw std::runtime_error("DeviceBatchMetadata: batch exceeds the sizes the buffers were made for");
    auto cp = [&](void* dst, const void* src, size_t n) {
        if (n) HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s));
    };
    cp(block_tables_, h.block_tables.data(), h.block_tables.size() * sizeof(int32_t));
    cp(seq_lens_, h.seq_lens.data(), h.seq_lens.size() * sizeof(int32_t));
    cp(slot_mapping_, h.slot_mapping.data(), h.slot_mapping.size() * sizeof(int64_t));
    if (h.num_prefills > 0) {
        cp(token_to_seq_, h.token_to_seq.data(), h.token_to_seq.size() * sizeof(int32_t));
        cp(token_positions_, h.token_positions.data(), h.token_positions.size() * sizeof(int32_t));
    }
    AttentionMetadata m;
    m.block_tables = h.max_num_blocks_per_req > 0 ? block_tables_ : nullptr;
    m.seq_lens = seq_lens_;
    m.slot_mapping = slot_mapping_;
    m.token_to_seq = token_to_seq_;
    m.token_positions = token_positions_;
    m.cu_seqlens = h.cu_seqlens.data();
    m.host_token_to_seq = h.token_to_seq.data();
    m.num_reqs = h.num_reqs;
    m.num_tokens = h.num_tokens;
    m.max_num_blocks_per_req = h.max_num_blocks_per_req;
    m.block_size = block_size;
    m.is_prefill = h.num_prefills > 0;
    m.num_prefills = h.num_prefills;
    m.num_prefill_tokens = h.num_prefill_tokens;
    m.num_decodes = h.num_decodes;
    m.num_decode_tokens = h.num_decode_tokens;
    m.num_computed_tokens = h.num_computed_tokens;
    return m;
}

}  // namespace vm_c
