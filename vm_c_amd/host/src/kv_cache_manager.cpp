// kv_cache_manager.cpp -- vm_c's paged KV block manager on HIP.
// Behaviour follows src/memory/kv_cache_manager.cpp (cited per function);
// the page pools are allocated through KVMemory.
#include "vm_c/kv_cache_manager.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace vm_c {

size_t BlockHashKeyHash::operator()(const BlockHashKey& k) const {
    size_t h = std::hash<uint64_t>()(k.hash);
    h ^= std::hash<int>()(k.group_id) + 0x9e3779b9 + (h << 6) + (h >> 2);
    return h;
}

// ------------------------------------------------------------ free queue
// kv_cache_manager.cpp:11-105: intrusive doubly linked list between two
// sentinels; popleft_n is all-or-nothing.

FreeKVCacheBlockQueue::FreeKVCacheBlockQueue(std::vector<KVCacheBlock>& blocks) {
    head_.next_free = &tail_;
    tail_.prev_free = &head_;
    for (auto& b : blocks) {
        b.prev_free = b.next_free = nullptr;
        append(&b);
    }
}

KVCacheBlock* FreeKVCacheBlockQueue::popleft() {
    KVCacheBlock* first = head_.next_free;
    if (first == &tail_) return nullptr;
    head_.next_free = first->next_free;
    first->next_free->prev_free = &head_;
    first->prev_free = first->next_free = nullptr;
    --num_free_;
    return first;
}

std::vector<KVCacheBlock*> FreeKVCacheBlockQueue::popleft_n(int64_t n) {
    std::vector<KVCacheBlock*> out;
    if (n <= 0 || num_free_ < n) return out;
    out.reserve((size_t)n);
    for (int64_t i = 0; i < n; ++i) out.push_back(popleft());
    return out;
}

void FreeKVCacheBlockQueue::remove(KVCacheBlock* b) {
    if (!b || !b->prev_free || !b->next_free) return;
    b->prev_free->next_free = b->next_free;
    b->next_free->prev_free = b->prev_free;
    b->prev_free = b->next_free = nullptr;
    --num_free_;
}

void FreeKVCacheBlockQueue::append(KVCacheBlock* b) {
    if (!b) return;
    KVCacheBlock* last = tail_.prev_free;
    last->next_free = b;
    b->prev_free = last;
    b->next_free = &tail_;
    tail_.prev_free = b;
    ++num_free_;
}

void FreeKVCacheBlockQueue::append_n(const std::vector<KVCacheBlock*>& blocks) {
    for (KVCacheBlock* b : blocks) append(b);
}

std::vector<int64_t> FreeKVCacheBlockQueue::ids() const {
    std::vector<int64_t> out;
    for (const KVCacheBlock* b = head_.next_free; b != &tail_; b = b->next_free) out.push_back(b->block_id);
    return out;
}

// ------------------------------------------------------------ hash map
// kv_cache_manager.cpp:107-172: several blocks may carry one hash; get()
// returns any of them, pop() removes one by id.

KVCacheBlock* BlockHashToBlockMap::get(uint64_t hash, int group_id) {
    auto it = cache_.find({hash, group_id});
    if (it == cache_.end() || it->second.empty()) return nullptr;
    return it->second.begin()->second;
}

void BlockHashToBlockMap::insert(uint64_t hash, int group_id, KVCacheBlock* block) {
    cache_[{hash, group_id}][block->block_id] = block;
}

KVCacheBlock* BlockHashToBlockMap::pop(uint64_t hash, int group_id, int64_t block_id) {
    auto it = cache_.find({hash, group_id});
    if (it == cache_.end()) return nullptr;
    auto bit = it->second.find(block_id);
    if (bit == it->second.end()) return nullptr;
    KVCacheBlock* b = bit->second;
    it->second.erase(bit);
    if (it->second.empty()) cache_.erase(it);
    return b;
}

// ------------------------------------------------------------ TQ layout

TurboQuantLayout TurboQuantLayout::create(int head_dim, const std::string& method, int gpu_device) {
    (void)gpu_device;
    TurboQuantLayout l;
    l.head_dim = head_dim;
    if (method == "turboquant_k8v4") {
        l.key_quant_bits = 8;
        l.value_quant_bits = 4;
        l.norm_correction = false;
        l.key_fp8 = true;
    } else if (method == "turboquant_k3v4_nc") {
        l.key_quant_bits = 3;
        l.value_quant_bits = 4;
    } else if (method == "turboquant_3bit_nc") {
        l.key_quant_bits = 3;
        l.value_quant_bits = 3;
    } else if (method == "turboquant_4bit_g32" || method == "turboquant_3bit_g32") {
        // per-32-group variant (not in vm_c): K part + V part of four blocks
        const int b = method == "turboquant_4bit_g32" ? 4 : 3;
        const int part = b == 4 ? 80 : 56;
        l.key_quant_bits = l.value_quant_bits = b;
        l.norm_correction = false;
        l.group_size = 32;
        l.n_centroids = 0;
        l.mse_bytes = l.val_data_bytes = 16 * b;
        l.key_packed_size = l.value_packed_size = part;
        l.slot_size = l.slot_size_aligned = 2 * part;
        return l;
    }
    l.n_centroids = 1 << l.key_quant_bits;
    l.mse_bytes = l.key_fp8 ? head_dim : (head_dim * l.key_quant_bits + 7) / 8;
    l.key_packed_size = l.key_fp8 ? head_dim : l.mse_bytes + 2;
    l.val_data_bytes = (head_dim * l.value_quant_bits + 7) / 8;
    l.value_packed_size = l.val_data_bytes + 4;
    l.slot_size = l.key_packed_size + l.value_packed_size;
    l.slot_size_aligned = l.slot_size + (l.slot_size % 2);
    return l;
}

std::vector<int> TurboQuantLayout::get_boundary_skip_layers(int num_layers, int n,
                                                            const std::vector<std::string>& types) {
    if (n <= 0 || num_layers <= 0) return {};
    for (const auto& t : types)
        if (t != "full_attention" && t != "attention") return {};
    n = std::min(n, num_layers / 2);
    std::vector<int> r;
    for (int i = 0; i < n; ++i) r.push_back(i);
    for (int i = num_layers - n; i < num_layers; ++i) r.push_back(i);
    std::sort(r.begin(), r.end());
    r.erase(std::unique(r.begin(), r.end()), r.end());
    return r;
}

// ------------------------------------------------------------ HIP memory

namespace {
class HipKVMemory : public KVMemory {
public:
    explicit HipKVMemory(int dev) : dev_(dev) {}
    void* alloc_device(size_t n) override {
        HIP_CHECK(hipSetDevice(dev_));
        void* p = nullptr;
        HIP_CHECK(hipMalloc(&p, n));
        return p;
    }
    void free_device(void* p) override {
        if (p) (void)hipFree(p);
    }
    void* alloc_host(size_t n) override {
        void* p = nullptr;
        HIP_CHECK(hipHostMalloc(&p, n, hipHostMallocDefault));
        return p;
    }
    void free_host(void* p) override {
        if (p) (void)hipHostFree(p);
    }
    void copy(void* dst, const void* src, size_t n) override {
        HIP_CHECK(hipMemcpy(dst, src, n, hipMemcpyDefault));
    }
    void copy_async(void* dst, const void* src, size_t n, hipStream_t s) override {
        HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDefault, s));
    }

private:
    int dev_;
};
}  // namespace

std::shared_ptr<KVMemory> hip_kv_memory(int gpu_device) {
    return std::make_shared<HipKVMemory>(gpu_device);
}

// ------------------------------------------------------------ manager

namespace {
DataType kv_dtype_for(const std::string& s) {
    // kv_cache_manager.cpp:180-194; gfx950 supports bf16
    if (s.find("turboquant") != std::string::npos) return DataType::BFLOAT16;
    if (s == "fp8_e4m3") return DataType::FLOAT8_E4M3;
    if (s == "fp8_e5m2") return DataType::FLOAT8_E5M2;
    if (s == "fp16") return DataType::FLOAT16;
    return DataType::BFLOAT16;  // bf16, auto, q8_0/q4_0 (their activations)
}
}  // namespace

KVCacheManager::KVCacheManager(const CacheConfig& config, const ModelConfig& model_config,
                               int num_layers, int num_kv_heads, int head_dim, int gpu_device,
                               bool is_mla, std::shared_ptr<KVMemory> memory)
    : block_size_(config.block_size),
      num_layers_(num_layers),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim),
      gpu_device_(gpu_device),
      model_config_(model_config),
      kv_cache_dtype_(config.kv_cache_quant_method.empty() ? config.kv_cache_dtype
                                                           : config.kv_cache_quant_method),
      kv_cache_layout_(config.kv_cache_layout.empty() ? "nhd" : config.kv_cache_layout),
      kv_dtype_(kv_dtype_for(kv_cache_dtype_)),
      is_mla_(is_mla),
      enable_caching_(config.enable_prefix_caching),
      mem_(memory ? std::move(memory) : hip_kv_memory(gpu_device)) {
    if (block_size_ <= 0 || num_kv_heads_ <= 0 || head_dim_ <= 0)
        throw std::runtime_error("KVCacheManager: block_size, num_kv_heads and head_dim must be > 0");
    if (kv_cache_dtype_.find("turboquant") != std::string::npos) {
        tq_layout_ = TurboQuantLayout::create(head_dim, kv_cache_dtype_, gpu_device);
        tq_layer_enabled_.assign(num_layers, true);
    }
    if ((kv_cache_dtype_ == "q8_0" || kv_cache_dtype_ == "q4_0") && head_dim_ % 32 != 0)
        throw std::runtime_error("KVCacheManager: q8_0/q4_0 need head_dim % 32 == 0");
    build_groups();
}

KVCacheManager::~KVCacheManager() {
    for (void* p : gpu_key_caches_) mem_->free_device(p);
    for (void* p : gpu_value_caches_) mem_->free_device(p);
    for (void* p : cpu_key_caches_) mem_->free_host(p);
    for (void* p : cpu_value_caches_) mem_->free_host(p);
}

// kv_cache_manager.cpp:225-271: TQ layers form group 0, boundary layers on
// the standard format group 1; without TQ one group of every cached layer.
void KVCacheManager::build_groups() {
    groups_.clear();
    std::vector<int> tq, std_layers;
    for (int i = 0; i < num_layers_; ++i) {
        if (!model_config_.layer_needs_kv_cache(i)) continue;
        if (is_turboquant() && tq_layer_enabled_[i]) tq.push_back(i);
        else std_layers.push_back(i);
    }
    if (!tq.empty()) groups_.push_back({0, tq, compute_bytes_per_block(true), true});
    if (!std_layers.empty())
        groups_.push_back({(int)groups_.size(), std_layers, compute_bytes_per_block(false), false});
    layer_to_group_.clear();
    for (const auto& g : groups_)
        for (int l : g.layer_indices) layer_to_group_[l] = g.group_id;
    group_num_gpu_blocks_.resize(groups_.size(), 0);
    group_num_free_gpu_blocks_.resize(groups_.size(), 0);
}

size_t KVCacheManager::std_entry_bytes() const {
    if (kv_cache_dtype_ == "q8_0") return (size_t)head_dim_ / 32 * 34;
    if (kv_cache_dtype_ == "q4_0") return (size_t)head_dim_ / 32 * 18;
    return (size_t)head_dim_ * dtype_size(kv_dtype_);
}

// :273-281 (TQ: one packed slot per token and head; MLA: one latent row)
size_t KVCacheManager::compute_bytes_per_block(bool tq) const {
    if (tq) return (size_t)block_size_ * num_kv_heads_ * tq_layout_.slot_size_aligned;
    if (is_mla_) return (size_t)block_size_ * head_dim_ * dtype_size(kv_dtype_);
    return (size_t)block_size_ * num_kv_heads_ * std_entry_bytes();
}

int KVCacheManager::group_id_for_layer(int layer) const {
    auto it = layer_to_group_.find(layer);
    return it != layer_to_group_.end() ? it->second : 0;
}

int64_t KVCacheManager::group_num_gpu_blocks(int g) const {
    return g >= 0 && g < (int)group_num_gpu_blocks_.size() ? group_num_gpu_blocks_[g] : 0;
}

int64_t KVCacheManager::group_num_free_gpu_blocks(int g) const {
    return g >= 0 && g < (int)group_num_free_gpu_blocks_.size() ? group_num_free_gpu_blocks_[g] : 0;
}

void KVCacheManager::set_tq_boundary_layers(const std::vector<int>& skip_layers) {
    if (!is_turboquant()) return;
    for (int l : skip_layers)
        if (l >= 0 && l < num_layers_) tq_layer_enabled_[l] = false;
    build_groups();
}

void KVCacheManager::reserve_gpu_blocks(int64_t total_blocks) { gpu_blocks_.reserve(total_blocks); }

// :314-372: one pool per layer of the group; new blocks join the free queue
// in id order; the first block ever popped becomes the null block.
void KVCacheManager::allocate_gpu_blocks_for_group(int group_id, int64_t num_blocks) {
    if (group_id < 0 || group_id >= (int)groups_.size() || num_blocks <= 0) return;
    const auto& g = groups_[group_id];
    group_num_gpu_blocks_[group_id] = num_blocks;
    group_num_free_gpu_blocks_[group_id] = num_blocks;
    const size_t bytes = (size_t)num_blocks * g.bytes_per_block;
    for (int layer : g.layer_indices) {
        if ((int)gpu_key_caches_.size() <= layer) {
            gpu_key_caches_.resize(layer + 1, nullptr);
            gpu_value_caches_.resize(layer + 1, nullptr);
        }
        gpu_key_caches_[layer] = mem_->alloc_device(bytes);
        gpu_value_caches_[layer] = (g.is_tq || is_mla_) ? nullptr : mem_->alloc_device(bytes);
    }
    // growing the block vector moves the blocks: keep the free order, the
    // hash map and the null block across the move
    const std::vector<int64_t> free_ids = free_queue_ ? free_queue_->ids() : std::vector<int64_t>{};
    const int64_t null_id = null_block_ ? null_block_->block_id : -1;
    const int64_t prev = (int64_t)gpu_blocks_.size();
    gpu_blocks_.resize(prev + num_blocks);
    for (int64_t i = prev; i < prev + num_blocks; ++i) {
        gpu_blocks_[i] = KVCacheBlock{};
        gpu_blocks_[i].block_id = i;
    }
    std::vector<KVCacheBlock> none;
    free_queue_ = std::make_unique<FreeKVCacheBlockQueue>(none);
    for (auto& b : gpu_blocks_) b.prev_free = b.next_free = nullptr;
    for (int64_t id : free_ids) free_queue_->append(&gpu_blocks_[id]);
    for (int64_t i = prev; i < prev + num_blocks; ++i) free_queue_->append(&gpu_blocks_[i]);
    hash_cache_.clear();
    for (auto& b : gpu_blocks_)
        if (b.has_hash)
            for (int gg = 0; gg < (int)groups_.size(); ++gg) hash_cache_.insert(b.block_hash.hash, gg, &b);
    null_block_ = null_id >= 0 ? &gpu_blocks_[null_id] : nullptr;
    if (!null_block_) {
        null_block_ = free_queue_->popleft();
        null_block_->is_null = true;
        null_block_->ref_cnt = 1;
    }
}

// :375-437: pinned host pools, grown by copy
void KVCacheManager::allocate_cpu_blocks_for_group(int group_id, int64_t num_blocks) {
    if (group_id < 0 || group_id >= (int)groups_.size() || num_blocks <= 0) return;
    const auto& g = groups_[group_id];
    const int64_t prev = num_cpu_blocks_;
    num_cpu_blocks_ += num_blocks;
    num_free_cpu_blocks_ += num_blocks;
    const size_t old_bytes = (size_t)prev * g.bytes_per_block;
    const size_t new_bytes = (size_t)num_cpu_blocks_ * g.bytes_per_block;
    for (int layer : g.layer_indices) {
        if ((int)cpu_key_caches_.size() <= layer) {
            cpu_key_caches_.resize(layer + 1, nullptr);
            cpu_value_caches_.resize(layer + 1, nullptr);
        }
        const bool two = !(g.is_tq || is_mla_);
        for (int kv = 0; kv < (two ? 2 : 1); ++kv) {
            void*& slot = kv == 0 ? cpu_key_caches_[layer] : cpu_value_caches_[layer];
            void* np = mem_->alloc_host(new_bytes);
            if (slot) {
                std::memcpy(np, slot, old_bytes);
                mem_->free_host(slot);
            }
            slot = np;
        }
    }
    const int64_t old = (int64_t)cpu_blocks_.size();
    cpu_blocks_.resize(num_cpu_blocks_);
    for (int64_t i = old; i < num_cpu_blocks_; ++i) {
        cpu_blocks_[i] = KVCacheBlock{};
        cpu_blocks_[i].block_id = i;
    }
}

// :439-456
int KVCacheManager::find_longest_prefix_hit(const std::vector<uint64_t>& block_hashes,
                                            int max_num_blocks,
                                            std::vector<int64_t>& out_block_ids) const {
    if (!enable_caching_ || block_hashes.empty()) return 0;
    out_block_ids.clear();
    const int n = std::min(max_num_blocks, (int)block_hashes.size());
    auto& map = const_cast<BlockHashToBlockMap&>(hash_cache_);
    for (int i = 0; i < n; ++i) {
        KVCacheBlock* b = map.get(block_hashes[i], 0);
        if (!b) break;
        out_block_ids.push_back(b->block_id);
    }
    return (int)out_block_ids.size();
}

// :458-511: reuse computed (prefix-cache) blocks first, then take the
// missing blocks from the front of the free queue, all or nothing; a reused
// block leaves the free queue, a newly taken one drops its stale hash.
std::vector<KVCacheSlot> KVCacheManager::allocate_slots(const std::string& request_id,
                                                        int num_tokens,
                                                        const std::vector<uint64_t>& prefix_block_hashes,
                                                        int num_new_computed_tokens,
                                                        const std::vector<int64_t>& new_computed_block_ids) {
    (void)prefix_block_hashes;
    (void)num_new_computed_tokens;
    if (!free_queue_) return {};
    const int64_t needed = (num_tokens + block_size_ - 1) / block_size_;
    std::vector<KVCacheSlot> slots;
    auto it = request_slots_.find(request_id);
    if (it != request_slots_.end()) slots = it->second;
    for (int64_t bid : new_computed_block_ids) {
        if (bid < 0 || bid >= (int64_t)gpu_blocks_.size()) continue;
        KVCacheBlock& b = gpu_blocks_[bid];
        if (b.ref_cnt == 0 && !b.is_null) free_queue_->remove(&b);
        ++b.ref_cnt;
        slots.push_back({bid, 0});
    }
    const int64_t more = needed - (int64_t)slots.size();
    if (more > 0) {
        auto got = free_queue_->popleft_n(more);
        if ((int64_t)got.size() < more) return {};
        for (KVCacheBlock* b : got) {
            if (enable_caching_ && b->has_hash) {
                for (int g = 0; g < (int)groups_.size(); ++g) hash_cache_.pop(b->block_hash.hash, g, b->block_id);
                b->reset_hash();
            }
            b->ref_cnt = 1;
            slots.push_back({b->block_id, 0});
        }
    }
    request_slots_[request_id] = slots;
    return slots;
}

// :513-532: drop one reference per block; blocks reaching zero return to
// the free queue in reverse order (the request's tail is evicted first).
void KVCacheManager::free_slots(const std::string& request_id) {
    auto it = request_slots_.find(request_id);
    if (it == request_slots_.end()) return;
    std::vector<KVCacheBlock*> freed;
    for (const auto& s : it->second) {
        if (s.block_id < 0 || s.block_id >= (int64_t)gpu_blocks_.size()) continue;
        KVCacheBlock& b = gpu_blocks_[s.block_id];
        if (--b.ref_cnt <= 0 && !b.is_null) {
            b.ref_cnt = 0;
            freed.push_back(&b);
        }
    }
    std::reverse(freed.begin(), freed.end());
    free_queue_->append_n(freed);
    request_slots_.erase(it);
}

// :848-880
void KVCacheManager::trim_request_to_tokens(const std::string& request_id, int num_tokens) {
    if (num_tokens < 0) throw std::runtime_error("trim_request_to_tokens: num_tokens must be non-negative");
    auto it = request_slots_.find(request_id);
    if (it == request_slots_.end()) return;
    const int64_t keep = num_tokens > 0 ? (num_tokens + block_size_ - 1) / block_size_ : 0;
    if (keep >= (int64_t)it->second.size()) return;
    std::vector<KVCacheBlock*> freed;
    for (size_t i = (size_t)keep; i < it->second.size(); ++i) {
        const int64_t bid = it->second[i].block_id;
        if (bid < 0 || bid >= (int64_t)gpu_blocks_.size()) continue;
        KVCacheBlock& b = gpu_blocks_[bid];
        if (--b.ref_cnt <= 0 && !b.is_null) {
            b.ref_cnt = 0;
            freed.push_back(&b);
        }
    }
    std::reverse(freed.begin(), freed.end());
    free_queue_->append_n(freed);
    it->second.resize((size_t)keep);
}

// :623-649: registers the request's full blocks [num_cached, num_full) under
// their hashes in every group
void KVCacheManager::cache_full_blocks(const std::string& request_id,
                                       const std::vector<uint64_t>& block_hashes,
                                       int num_cached_blocks, int num_full_blocks) {
    if (!enable_caching_ || block_hashes.empty()) return;
    auto it = request_slots_.find(request_id);
    if (it == request_slots_.end()) return;
    const auto& slots = it->second;
    for (int i = num_cached_blocks; i < num_full_blocks && i < (int)slots.size(); ++i) {
        const int64_t bid = slots[i].block_id;
        if (bid < 0 || bid >= (int64_t)gpu_blocks_.size()) continue;
        KVCacheBlock& b = gpu_blocks_[bid];
        if (b.is_null || b.has_hash || i >= (int)block_hashes.size()) continue;
        b.set_hash(block_hashes[i], 0);
        for (int g = 0; g < (int)groups_.size(); ++g) hash_cache_.insert(block_hashes[i], g, &b);
    }
}

int64_t KVCacheManager::num_free_gpu_blocks() const { return free_queue_ ? free_queue_->num_free_blocks() : 0; }

std::vector<int64_t> KVCacheManager::free_block_ids() const {
    return free_queue_ ? free_queue_->ids() : std::vector<int64_t>{};
}

int64_t KVCacheManager::num_gpu_blocks() const {
    int64_t t = 0;
    for (int64_t n : group_num_gpu_blocks_) t += n;
    return t;
}

// :661-666: the null block does not count
float KVCacheManager::usage() const {
    const int64_t total = num_gpu_blocks();
    if (total <= 1) return 0.0f;
    return 1.0f - (float)num_free_gpu_blocks() / (float)(total - 1);
}

// :668-683: only when nothing but the null block is in use
bool KVCacheManager::reset_prefix_cache() {
    if (!enable_caching_) return false;
    if (num_gpu_blocks() - num_free_gpu_blocks() > 1) return false;
    hash_cache_.clear();
    for (auto& b : gpu_blocks_) b.reset_hash();
    return true;
}

void* KVCacheManager::key_cache_ptr(int l) {
    return l >= 0 && l < (int)gpu_key_caches_.size() ? gpu_key_caches_[l] : nullptr;
}
void* KVCacheManager::value_cache_ptr(int l) {
    return l >= 0 && l < (int)gpu_value_caches_.size() ? gpu_value_caches_[l] : nullptr;
}
void* KVCacheManager::cpu_key_cache_ptr(int l) {
    return l >= 0 && l < (int)cpu_key_caches_.size() ? cpu_key_caches_[l] : nullptr;
}
void* KVCacheManager::cpu_value_cache_ptr(int l) {
    return l >= 0 && l < (int)cpu_value_caches_.size() ? cpu_value_caches_[l] : nullptr;
}

void KVCacheManager::copy_block(int64_t gpu_block, int64_t cpu_block, bool to_cpu) {
    for (int layer = 0; layer < num_layers_; ++layer) {
        if (!model_config_.layer_needs_kv_cache(layer)) continue;
        const auto& g = groups_[group_id_for_layer(layer)];
        const size_t n = g.bytes_per_block;
        auto* gk = static_cast<uint8_t*>(gpu_key_caches_[layer]) + gpu_block * n;
        auto* ck = static_cast<uint8_t*>(cpu_key_caches_[layer]) + cpu_block * n;
        to_cpu ? mem_->copy(ck, gk, n) : mem_->copy(gk, ck, n);
        if (!g.is_tq && !is_mla_) {
            auto* gv = static_cast<uint8_t*>(gpu_value_caches_[layer]) + gpu_block * n;
            auto* cv = static_cast<uint8_t*>(cpu_value_caches_[layer]) + cpu_block * n;
            to_cpu ? mem_->copy(cv, gv, n) : mem_->copy(gv, cv, n);
        }
    }
}

// :710-748: copy to the first free host block, move the block's reference
// count and hash there
void KVCacheManager::offload_to_cpu(int64_t block_id) {
    if (block_id < 0 || block_id >= (int64_t)gpu_blocks_.size() || num_cpu_blocks_ == 0) return;
    if (gpu_to_cpu_mapping_.count(block_id)) return;
    int64_t cpu = -1;
    for (int64_t i = 0; i < num_cpu_blocks_; ++i)
        if (cpu_blocks_[i].ref_cnt == 0) {
            cpu = i;
            break;
        }
    if (cpu < 0) return;
    copy_block(block_id, cpu, true);
    cpu_blocks_[cpu].ref_cnt = gpu_blocks_[block_id].ref_cnt;
    cpu_blocks_[cpu].has_hash = gpu_blocks_[block_id].has_hash;
    cpu_blocks_[cpu].block_hash = gpu_blocks_[block_id].block_hash;
    gpu_to_cpu_mapping_[block_id] = cpu;
    cpu_to_gpu_mapping_[cpu] = block_id;
    gpu_blocks_[block_id].ref_cnt = 0;
    --num_free_cpu_blocks_;
}

// :750-784
void KVCacheManager::load_from_cpu(int64_t block_id) {
    if (block_id < 0 || block_id >= (int64_t)gpu_blocks_.size()) return;
    auto it = gpu_to_cpu_mapping_.find(block_id);
    if (it == gpu_to_cpu_mapping_.end()) return;
    const int64_t cpu = it->second;
    if (cpu < 0 || cpu >= num_cpu_blocks_ || cpu_blocks_[cpu].ref_cnt == 0) return;
    copy_block(block_id, cpu, false);
    gpu_blocks_[block_id].ref_cnt = cpu_blocks_[cpu].ref_cnt;
    gpu_blocks_[block_id].has_hash = cpu_blocks_[cpu].has_hash;
    gpu_blocks_[block_id].block_hash = cpu_blocks_[cpu].block_hash;
    gpu_to_cpu_mapping_.erase(block_id);
    cpu_to_gpu_mapping_.erase(cpu);
    cpu_blocks_[cpu].ref_cnt = 0;
    ++num_free_cpu_blocks_;
}

// :534-556: offload every block of the request, return the device blocks to
// the free queue, keep the request's slot list for swap-back
void KVCacheManager::swap_request_slots(const std::string& request_id) {
    auto it = request_slots_.find(request_id);
    if (it == request_slots_.end()) return;
    for (const auto& s : it->second)
        if (s.block_id >= 0 && s.block_id < (int64_t)gpu_blocks_.size()) offload_to_cpu(s.block_id);
    std::vector<KVCacheBlock*> freed;
    for (const auto& s : it->second) {
        if (s.block_id < 0 || s.block_id >= (int64_t)gpu_blocks_.size()) continue;
        KVCacheBlock& b = gpu_blocks_[s.block_id];
        if (b.ref_cnt <= 0 && !b.is_null && !b.prev_free) freed.push_back(&b);
    }
    free_queue_->append_n(freed);
}

// :557-621: allocate fresh device blocks (one per old block) and copy the
// host copies back in order
void KVCacheManager::swap_back_request_slots(const std::string& request_id) {
    auto it = request_slots_.find(request_id);
    if (it == request_slots_.end()) return;
    std::vector<int64_t> old_ids;
    for (const auto& s : it->second) old_ids.push_back(s.block_id);
    request_slots_.erase(it);
    const int num_tokens = (int)old_ids.size() * (int)block_size_;
    auto fresh = allocate_slots(request_id, num_tokens);
    size_t k = 0;
    for (size_t i = 0; i < old_ids.size() && k < fresh.size(); ++i) {
        auto m = gpu_to_cpu_mapping_.find(old_ids[i]);
        if (m == gpu_to_cpu_mapping_.end()) continue;
        const int64_t cpu = m->second;
        if (cpu < 0 || cpu >= num_cpu_blocks_ || cpu_blocks_[cpu].ref_cnt == 0) continue;
        const int64_t nb = fresh[k].block_id;
        copy_block(nb, cpu, false);
        gpu_blocks_[nb].ref_cnt = cpu_blocks_[cpu].ref_cnt;
        gpu_blocks_[nb].has_hash = cpu_blocks_[cpu].has_hash;
        gpu_blocks_[nb].block_hash = cpu_blocks_[cpu].block_hash;
        cpu_blocks_[cpu].ref_cnt = 0;
        gpu_to_cpu_mapping_.erase(old_ids[i]);
        cpu_to_gpu_mapping_.erase(cpu);
        ++num_free_cpu_blocks_;
        ++k;
    }
}

size_t KVCacheManager::gpu_kv_cache_bytes() const {
    size_t t = 0;
    for (size_t g = 0; g < groups_.size(); ++g) {
        const size_t one = (size_t)group_num_gpu_blocks_[g] * groups_[g].bytes_per_block *
                           groups_[g].layer_indices.size();
        t += (!groups_[g].is_tq && !is_mla_) ? 2 * one : one;
    }
    return t;
}

size_t KVCacheManager::cpu_kv_cache_bytes() const {
    size_t t = 0;
    for (size_t g = 0; g < groups_.size(); ++g) {
        const size_t one = (size_t)num_cpu_blocks_ * groups_[g].bytes_per_block * groups_[g].layer_indices.size();
        t += (!groups_[g].is_tq && !is_mla_) ? 2 * one : one;
    }
    return t;
}

// :882-895: TQ: packed slots of all heads; standard: K and V entries
size_t KVCacheManager::kv_bytes_per_token(int layer) const {
    if (layer < 0 || layer >= num_layers_)
        throw std::runtime_error("kv_bytes_per_token: invalid layer " + std::to_string(layer));
    const auto& g = groups_[group_id_for_layer(layer)];
    if (g.is_tq) return (size_t)num_kv_heads_ * tq_layout_.slot_size_aligned;
    return (size_t)num_kv_heads_ * std_entry_bytes() * 2;
}

// :897-964: a token's bytes of one layer, K then V (standard pools).  In
// "hnd" pools a token's heads are not contiguous: one copy per head.
void KVCacheManager::read_kv_token(int layer, int64_t global_slot, void* dst, hipStream_t stream) const {
    if (!dst) throw std::runtime_error("read_kv_token: dst is null");
    const auto& g = groups_[group_id_for_layer(layer)];
    const int64_t blk = global_slot / block_size_, off = global_slot % block_size_;
    auto* out = static_cast<uint8_t*>(dst);
    if (g.is_tq) {
        const size_t n = kv_bytes_per_token(layer);
        auto* c = static_cast<const uint8_t*>(gpu_key_caches_[layer]);
        mem_->copy_async(out, c + (size_t)blk * g.bytes_per_block + (size_t)off * n, n, stream);
        return;
    }
    const size_t E = std_entry_bytes(), T = (size_t)num_kv_heads_ * E;
    for (int kv = 0; kv < 2; ++kv) {
        auto* c = static_cast<const uint8_t*>(kv == 0 ? gpu_key_caches_[layer] : gpu_value_caches_[layer]);
        const uint8_t* base = c + (size_t)blk * g.bytes_per_block;
        if (!is_hnd_layout()) {
            mem_->copy_async(out + kv * T, base + (size_t)off * T, T, stream);
        } else {
            for (int h = 0; h < num_kv_heads_; ++h)
                mem_->copy_async(out + kv * T + h * E, base + ((size_t)h * block_size_ + off) * E, E, stream);
        }
    }
}

void KVCacheManager::write_kv_token(int layer, int64_t global_slot, const void* src,
                                    hipStream_t stream) const {
    if (!src) throw std::runtime_error("write_kv_token: src is null");
    const auto& g = groups_[group_id_for_layer(layer)];
    const int64_t blk = global_slot / block_size_, off = global_slot % block_size_;
    auto* in = static_cast<const uint8_t*>(src);
    if (g.is_tq) {
        const size_t n = kv_bytes_per_token(layer);
        auto* c = static_cast<uint8_t*>(gpu_key_caches_[layer]);
        mem_->copy_async(c + (size_t)blk * g.bytes_per_block + (size_t)off * n, in, n, stream);
        return;
    }
    const size_t E = std_entry_bytes(), T = (size_t)num_kv_heads_ * E;
    for (int kv = 0; kv < 2; ++kv) {
        auto* c = static_cast<uint8_t*>(kv == 0 ? gpu_key_caches_[layer] : gpu_value_caches_[layer]);
        uint8_t* base = c + (size_t)blk * g.bytes_per_block;
        if (!is_hnd_layout()) {
            mem_->copy_async(base + (size_t)off * T, in + kv * T, T, stream);
        } else {
            for (int h = 0; h < num_kv_heads_; ++h)
                mem_->copy_async(base + ((size_t)h * block_size_ + off) * E, in + kv * T + h * E, E, stream);
        }
    }
}

}  // namespace vm_c
