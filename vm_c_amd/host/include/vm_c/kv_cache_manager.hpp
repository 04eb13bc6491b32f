// vm_c/kv_cache_manager.hpp -- paged KV block manager on HIP.
//
// Public API and behaviour of vm_c's KVCacheManager
// (include/vm_c/memory/kv_cache_manager.hpp:17-322, src/memory/
// kv_cache_manager.cpp): FIFO free queue with O(1) removal, block 0 taken as
// the null block, ref-counted sharing, prefix-cache hash map per group,
// all-or-nothing allocation, freed blocks returned in reverse order, TQ and
// standard layer groups.  Page pools are one allocation per layer and group
// (hipMalloc); a TurboQuant layer has one packed pool (value pointer null).
//
// Device memory goes through a KVMemory object (default: HIP), so the
// allocation and bookkeeping logic runs, and is tested, without a GPU.
#pragma once

#include <cstdint>
#include <list>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "vm_c/common.hpp"

namespace vm_c {

struct BlockHashKey {
    uint64_t hash;
    int group_id;
    bool operator==(const BlockHashKey& o) const { return hash == o.hash && group_id == o.group_id; }
};

struct BlockHashKeyHash {
    size_t operator()(const BlockHashKey& k) const;
};

struct KVCacheBlock {
    int64_t block_id = -1;
    int ref_cnt = 0;
    BlockHashKey block_hash{0, -1};
    bool has_hash = false;
    bool is_null = false;

    KVCacheBlock* prev_free = nullptr;
    KVCacheBlock* next_free = nullptr;

    void set_hash(uint64_t hash, int group_id) {
        block_hash = {hash, group_id};
        has_hash = true;
    }
    void reset_hash() {
        block_hash = {0, -1};
        has_hash = false;
    }
};

// Doubly linked FIFO of free blocks threaded through the blocks themselves.
class FreeKVCacheBlockQueue {
public:
    explicit FreeKVCacheBlockQueue(std::vector<KVCacheBlock>& blocks);

    KVCacheBlock* popleft();
    // n blocks from the front, or none if fewer than n are free
    std::vector<KVCacheBlock*> popleft_n(int64_t n);
    void remove(KVCacheBlock* block);
    void append(KVCacheBlock* block);
    void append_n(const std::vector<KVCacheBlock*>& blocks);

    int64_t num_free_blocks() const { return num_free_; }
    // block ids front to back (diagnostics and tests)
    std::vector<int64_t> ids() const;

private:
    KVCacheBlock head_;
    KVCacheBlock tail_;
    int64_t num_free_ = 0;
};

class BlockHashToBlockMap {
public:
    KVCacheBlock* get(uint64_t hash, int group_id);
    void insert(uint64_t hash, int group_id, KVCacheBlock* block);
    KVCacheBlock* pop(uint64_t hash, int group_id, int64_t block_id);
    void clear() { cache_.clear(); }
    size_t size() const { return cache_.size(); }

private:
    // blocks sharing one hash, by block id (one entry in the common case)
    std::unordered_map<BlockHashKey, std::unordered_map<int64_t, KVCacheBlock*>, BlockHashKeyHash> cache_;
};

struct KVCacheSlot {
    int64_t block_id;
    int slot_offset;
};

struct KVCacheGroupSpec {
    int group_id;
    std::vector<int> layer_indices;
    size_t bytes_per_block;
    bool is_tq;
};

struct TurboQuantLayout {
    int head_dim = 0;
    int key_quant_bits = 4;
    int value_quant_bits = 4;
    bool norm_correction = true;
    bool key_fp8 = false;
    bool fp8_e4b15 = false;

    int mse_bytes = 0;
    int key_packed_size = 0;
    int val_data_bytes = 0;
    int value_packed_size = 0;
    int slot_size = 0;
    int slot_size_aligned = 0;
    int n_centroids = 0;
    int group_size = 0;  // not in vm_c: 32 for the "*_g32" variants (vmc_attn.h)

    // kv_cache_manager.hpp:121-162; an unknown method leaves the 4-bit
    // defaults, as there.  fp8_e4b15 is false (gfx950 has e4m3).
    static TurboQuantLayout create(int head_dim, const std::string& method, int gpu_device = 0);
    // first and last n layers (none for hybrid layer lists), :164-184
    static std::vector<int> get_boundary_skip_layers(int num_layers, int n = 2,
                                                     const std::vector<std::string>& layer_types = {});
};

// The CacheConfig / ModelConfig fields the block manager reads
// (include/vm_c/core/config.hpp:147-167, :136-144).
struct CacheConfig {
    int64_t block_size = 16;
    std::string kv_cache_dtype = "auto";  // auto | fp16 | bf16 | fp8_e4m3 | fp8_e5m2 | q8_0 | q4_0
    std::string kv_cache_quant_method;    // turboquant_* (takes precedence)
    std::string kv_cache_layout = "nhd";  // nhd | hnd
    int64_t num_gpu_blocks = 0;
    int64_t num_cpu_blocks = 0;
    bool enable_prefix_caching = true;
};

struct ModelConfig {
    // per-layer "has a KV cache" (empty: every layer has one)
    std::vector<bool> kv_cache_layers;
    bool layer_needs_kv_cache(int layer) const {
        return kv_cache_layers.empty() ||
               (layer >= 0 && layer < (int)kv_cache_layers.size() && kv_cache_layers[layer]);
    }
};

// Device / pinned-host memory used for the page pools.
class KVMemory {
public:
    virtual ~KVMemory() = default;
    virtual void* alloc_device(size_t bytes) = 0;
    virtual void free_device(void* p) = 0;
    virtual void* alloc_host(size_t bytes) = 0;
    virtual void free_host(void* p) = 0;
    // synchronous copy between any two of the above
    virtual void copy(void* dst, const void* src, size_t bytes) = 0;
    // stream-ordered device copy
    virtual void copy_async(void* dst, const void* src, size_t bytes, hipStream_t stream) = 0;
};
std::shared_ptr<KVMemory> hip_kv_memory(int gpu_device);

class KVCacheManager {
public:
    KVCacheManager(const CacheConfig& config, const ModelConfig& model_config, int num_layers,
                   int num_kv_heads, int head_dim, int gpu_device = 0, bool is_mla = false,
                   std::shared_ptr<KVMemory> memory = nullptr);
    ~KVCacheManager();

    KVCacheManager(const KVCacheManager&) = delete;
    KVCacheManager& operator=(const KVCacheManager&) = delete;

    void set_tq_boundary_layers(const std::vector<int>& skip_layers);

    void reserve_gpu_blocks(int64_t total_blocks);
    void allocate_gpu_blocks_for_group(int group_id, int64_t num_blocks);
    void allocate_cpu_blocks_for_group(int group_id, int64_t num_blocks);

    std::vector<KVCacheSlot> allocate_slots(const std::string& request_id, int num_tokens,
                                            const std::vector<uint64_t>& prefix_block_hashes = {},
                                            int num_new_computed_tokens = 0,
                                            const std::vector<int64_t>& new_computed_block_ids = {});
    void free_slots(const std::string& request_id);
    void trim_request_to_tokens(const std::string& request_id, int num_tokens);

    size_t kv_bytes_per_token(int layer) const;
    void read_kv_token(int layer, int64_t global_slot, void* dst, hipStream_t stream) const;
    void write_kv_token(int layer, int64_t global_slot, const void* src, hipStream_t stream) const;

    void swap_request_slots(const std::string& request_id);
    void swap_back_request_slots(const std::string& request_id);

    void cache_full_blocks(const std::string& request_id, const std::vector<uint64_t>& block_hashes,
                           int num_cached_blocks, int num_full_blocks);
    int find_longest_prefix_hit(const std::vector<uint64_t>& block_hashes, int max_num_blocks,
                                std::vector<int64_t>& out_block_ids) const;

    int64_t num_free_gpu_blocks() const;
    int64_t num_free_cpu_blocks() const { return num_free_cpu_blocks_; }
    int64_t num_gpu_blocks() const;
    const std::vector<KVCacheBlock>& gpu_blocks() const { return gpu_blocks_; }
    const std::unordered_map<std::string, std::vector<KVCacheSlot>>& request_slots() const {
        return request_slots_;
    }
    std::vector<int64_t> free_block_ids() const;

    void* key_cache_ptr(int layer);
    void* value_cache_ptr(int layer);
    void* cpu_key_cache_ptr(int layer);
    void* cpu_value_cache_ptr(int layer);

    int64_t block_size() const { return block_size_; }
    int num_layers() const { return num_layers_; }
    int num_kv_heads() const { return num_kv_heads_; }
    int head_dim() const { return head_dim_; }

    bool is_turboquant() const { return tq_layout_.slot_size > 0; }
    bool is_mla() const { return is_mla_; }
    bool is_layer_turboquant(int layer) const {
        return is_turboquant() && layer >= 0 && layer < num_layers_ && tq_layer_enabled_[layer];
    }
    const TurboQuantLayout& tq_layout() const { return tq_layout_; }
    // kv_cache_dtype / quant method in effect ("fp16", "bf16", "q8_0", ...)
    const std::string& kv_cache_dtype() const { return kv_cache_dtype_; }

    bool is_hnd_layout() const { return kv_cache_layout_ == "hnd"; }
    const std::string& kv_cache_layout() const { return kv_cache_layout_; }

    int num_kv_cache_groups() const { return (int)groups_.size(); }
    const KVCacheGroupSpec& group(int group_id) const { return groups_[group_id]; }
    int group_id_for_layer(int layer) const;
    int64_t group_num_gpu_blocks(int group_id) const;
    int64_t group_num_free_gpu_blocks(int group_id) const;

    bool compress_kv_block(int64_t) { return true; }
    bool decompress_kv_block(int64_t) { return true; }

    void offload_to_cpu(int64_t block_id);
    void load_from_cpu(int64_t block_id);

    size_t gpu_kv_cache_bytes() const;
    size_t cpu_kv_cache_bytes() const;
    float usage() const;
    bool reset_prefix_cache();

private:
    void build_groups();
    size_t compute_bytes_per_block(bool tq) const;
    size_t std_entry_bytes() const;  // one (token, head) entry of a standard pool
    void copy_block(int64_t gpu_block, int64_t cpu_block, bool to_cpu);

    int64_t block_size_;
    int num_layers_;
    int num_kv_heads_;
    int head_dim_;
    int gpu_device_;
    ModelConfig model_config_;
    std::string kv_cache_dtype_;
    std::string kv_cache_layout_ = "nhd";
    DataType kv_dtype_;
    TurboQuantLayout tq_layout_;
    std::vector<bool> tq_layer_enabled_;
    bool is_mla_ = false;
    bool enable_caching_;
    std::shared_ptr<KVMemory> mem_;

    std::vector<KVCacheGroupSpec> groups_;
    std::unordered_map<int, int> layer_to_group_;
    std::vector<int64_t> group_num_gpu_blocks_;
    std::vector<int64_t> group_num_free_gpu_blocks_;
    int64_t num_cpu_blocks_ = 0;
    int64_t num_free_cpu_blocks_ = 0;

    std::vector<void*> gpu_key_caches_, gpu_value_caches_;
    std::vector<void*> cpu_key_caches_, cpu_value_caches_;

    std::vector<KVCacheBlock> gpu_blocks_;
    std::vector<KVCacheBlock> cpu_blocks_;
    KVCacheBlock* null_block_ = nullptr;

    std::unique_ptr<FreeKVCacheBlockQueue> free_queue_;
    BlockHashToBlockMap hash_cache_;

    std::unordered_map<std::string, std::vector<KVCacheSlot>> request_slots_;
    std::unordered_map<int64_t, int64_t> gpu_to_cpu_mapping_;
    std::unordered_map<int64_t, int64_t> cpu_to_gpu_mapping_;
};

}  // namespace vm_c
