// CPU tests of the vm_c host layer (no GPU calls): block manager behaviour,
// layouts, metadata construction, token read/write offsets, swap paths and
// the C++ error convention.  Built and run by tests/test_host_cpp.py.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "vm_c/attention_backend.hpp"
#include "vm_c/attention_metadata.hpp"
#include "vm_c/kv_cache_manager.hpp"
#include "vm_c/turboquant_kv_bridge.hpp"

using namespace vm_c;

static int g_fail = 0;
#define CHECK(c)                                                            \
    do {                                                                    \
        if (!(c)) {                                                         \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);        \
            ++g_fail;                                                       \
        }                                                                   \
    } while (0)

// host memory standing in for device memory
class HostMemory : public KVMemory {
public:
    void* alloc_device(size_t n) override { return std::calloc(n, 1); }
    void free_device(void* p) override { std::free(p); }
    void* alloc_host(size_t n) override { return std::calloc(n, 1); }
    void free_host(void* p) override { std::free(p); }
    void copy(void* d, const void* s, size_t n) override { std::memcpy(d, s, n); }
    void copy_async(void* d, const void* s, size_t n, hipStream_t) override { std::memcpy(d, s, n); }
};

static std::shared_ptr<KVMemory> hostmem() { return std::make_shared<HostMemory>(); }

static CacheConfig cache_cfg(const std::string& dtype = "bf16", const std::string& method = "",
                             const std::string& layout = "nhd", bool prefix = true) {
    CacheConfig c;
    c.block_size = 16;
    c.kv_cache_dtype = dtype;
    c.kv_cache_quant_method = method;
    c.kv_cache_layout = layout;
    c.enable_prefix_caching = prefix;
    return c;
}

static std::vector<int64_t> ids_of(const std::vector<KVCacheSlot>& s) {
    std::vector<int64_t> r;
    for (auto& x : s) r.push_back(x.block_id);
    return r;
}

static void test_free_queue() {
    std::vector<KVCacheBlock> blocks(6);
    for (int i = 0; i < 6; ++i) blocks[i].block_id = i;
    FreeKVCacheBlockQueue q(blocks);
    CHECK(q.num_free_blocks() == 6);
    CHECK(q.popleft()->block_id == 0);
    auto two = q.popleft_n(2);
    CHECK(two.size() == 2 && two[0]->block_id == 1 && two[1]->block_id == 2);
    CHECK(q.popleft_n(4).empty());  // all or nothing
    CHECK(q.num_free_blocks() == 3);
    q.remove(&blocks[4]);
    CHECK((q.ids() == std::vector<int64_t>{3, 5}));
    q.append(&blocks[0]);
    q.append_n({&blocks[2], &blocks[1]});
    CHECK((q.ids() == std::vector<int64_t>{3, 5, 0, 2, 1}));
    q.remove(&blocks[4]);  // not queued: no effect
    CHECK(q.num_free_blocks() == 5);
}

static void test_allocation_order() {
    KVCacheManager m(cache_cfg(), ModelConfig{}, 2, 8, 128, 0, false, hostmem());
    m.allocate_gpu_blocks_for_group(0, 10);
    CHECK(m.num_gpu_blocks() == 10);
    CHECK(m.num_free_gpu_blocks() == 9);  // block 0 is the null block
    CHECK(m.gpu_blocks()[0].is_null && m.gpu_blocks()[0].ref_cnt == 1);
    CHECK((ids_of(m.allocate_slots("a", 33)) == std::vector<int64_t>{1, 2, 3}));
    CHECK((ids_of(m.allocate_slots("b", 16)) == std::vector<int64_t>{4}));
    CHECK(m.allocate_slots("c", 16 * 6).empty());  // needs 6, 5 free
    CHECK(m.num_free_gpu_blocks() == 5);
    CHECK((ids_of(m.allocate_slots("a", 49)) == std::vector<int64_t>{1, 2, 3, 5}));  // grows
    m.free_slots("a");
    CHECK((m.free_block_ids() == std::vector<int64_t>{6, 7, 8, 9, 5, 3, 2, 1}));  // reversed
    CHECK(m.request_slots().count("a") == 0);
    m.trim_request_to_tokens("b", 0);
    CHECK(m.request_slots().at("b").empty());
    CHECK(m.free_block_ids().back() == 4);
    CHECK(m.usage() == 0.0f);
    m.allocate_slots("d", 16 * 9);
    CHECK(m.usage() == 1.0f);
    bool threw = false;
    try {
        m.trim_request_to_tokens("d", -1);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw);
}

static void test_prefix_cache() {
    KVCacheManager m(cache_cfg(), ModelConfig{}, 1, 8, 128, 0, false, hostmem());
    m.allocate_gpu_blocks_for_group(0, 8);
    auto s = ids_of(m.allocate_slots("a", 48));
    CHECK((s == std::vector<int64_t>{1, 2, 3}));
    m.cache_full_blocks("a", {111, 222, 333}, 0, 2);  // blocks 1, 2 full
    std::vector<int64_t> hit;
    CHECK(m.find_longest_prefix_hit({111, 222, 333}, 3, hit) == 2);
    CHECK((hit == std::vector<int64_t>{1, 2}));
    CHECK(m.find_longest_prefix_hit({999, 222}, 2, hit) == 0);
    m.free_slots("a");
    // freed blocks keep their hash and can be reused by a new request
    CHECK(m.find_longest_prefix_hit({111, 222}, 2, hit) == 2);
    auto r = ids_of(m.allocate_slots("b", 40, {111, 222}, 32, {1, 2}));
    CHECK(r.size() == 3 && r[0] == 1 && r[1] == 2);
    CHECK(m.gpu_blocks()[1].ref_cnt == 1 && m.gpu_blocks()[2].ref_cnt == 1);
    auto fr = m.free_block_ids();
    CHECK(std::find(fr.begin(), fr.end(), 1) == fr.end());
    // sharing: a second request on the same prefix raises the count
    m.allocate_slots("c", 32, {111, 222}, 32, {1, 2});
    CHECK(m.gpu_blocks()[1].ref_cnt == 2);
    m.free_slots("c");
    CHECK(m.gpu_blocks()[1].ref_cnt == 1);
    CHECK(!m.reset_prefix_cache());  // blocks in use
    m.free_slots("b");
    // a hashed block taken for new content loses its hash
    m.allocate_slots("e", 16 * 7);
    CHECK(m.find_longest_prefix_hit({111}, 1, hit) == 0);
    m.free_slots("e");
    CHECK(m.reset_prefix_cache());
}

static void test_layouts() {
    auto l4 = TurboQuantLayout::create(128, "turboquant_4bit_nc");
    auto l3 = TurboQuantLayout::create(128, "turboquant_3bit_nc");
    auto lk = TurboQuantLayout::create(128, "turboquant_k3v4_nc");
    auto l8 = TurboQuantLayout::create(128, "turboquant_k8v4");
    CHECK(l4.slot_size_aligned == 134 && l3.slot_size_aligned == 102);
    CHECK(lk.slot_size_aligned == 118 && l8.slot_size_aligned == 196);
    // per-32-group variant (not in vm_c): K + V parts of four blocks
    auto g4 = TurboQuantLayout::create(128, "turboquant_4bit_g32");
    auto g3 = TurboQuantLayout::create(128, "turboquant_3bit_g32");
    CHECK(g4.slot_size_aligned == 160 && g3.slot_size_aligned == 112);
    CHECK(g4.group_size == 32 && g3.group_size == 32 && g3.key_quant_bits == 3);
    {
        const TQConfig c4 = TQConfig::from_method(128, "turboquant_4bit_g32");
        const vmc_tq_config cc = c4.to_c();
        CHECK(cc.group_size == 32 && cc.slot_size_aligned == 160 && cc.key_packed_size == 80);
    }
    for (const char* meth : {"turboquant_4bit_nc", "turboquant_3bit_nc", "turboquant_k3v4_nc"}) {
        TQConfig a = TQConfig::from_method(128, meth);
        vmc_tq_config b;
        CHECK(vmc_tq_config_from_method(128, meth, &b) == VMC_OK);
        vmc_tq_config c = a.to_c();
        c.max_num_kv_splits = b.max_num_kv_splits;
        CHECK(std::memcmp(&b, &c, sizeof(b)) == 0);
    }
    CHECK((TurboQuantLayout::get_boundary_skip_layers(10, 2) == std::vector<int>{0, 1, 8, 9}));
    CHECK(TurboQuantLayout::get_boundary_skip_layers(10, 2, {"attention", "linear_attention"}).empty());
    CHECK((TurboQuantLayout::get_boundary_skip_layers(3, 2) == std::vector<int>{0, 2}));

    KVCacheManager tq(cache_cfg("auto", "turboquant_3bit_nc"), ModelConfig{}, 6, 8, 128, 0, false, hostmem());
    CHECK(tq.is_turboquant() && tq.num_kv_cache_groups() == 1);
    CHECK(tq.group(0).bytes_per_block == (size_t)16 * 8 * 102);
    CHECK(tq.kv_bytes_per_token(3) == (size_t)8 * 102);
    tq.set_tq_boundary_layers(TurboQuantLayout::get_boundary_skip_layers(6, 1));
    CHECK(tq.num_kv_cache_groups() == 2);
    CHECK(tq.group_id_for_layer(0) == 1 && tq.group_id_for_layer(2) == 0);
    CHECK(tq.group(1).bytes_per_block == (size_t)16 * 8 * 128 * 2);  // bf16 standard pages
    CHECK(!tq.is_layer_turboquant(5) && tq.is_layer_turboquant(4));
    tq.allocate_gpu_blocks_for_group(0, 5);
    tq.allocate_gpu_blocks_for_group(1, 5);
    CHECK(tq.key_cache_ptr(2) && !tq.value_cache_ptr(2));  // packed TQ pool
    CHECK(tq.key_cache_ptr(0) && tq.value_cache_ptr(0));
    CHECK(tq.gpu_kv_cache_bytes() == (size_t)5 * 16 * 8 * 102 * 4 + (size_t)5 * 32768 * 2 * 2);
    // the second group's blocks extend the same id space; the queue survived the move
    CHECK(tq.num_free_gpu_blocks() == 9);
    auto s = ids_of(tq.allocate_slots("x", 16 * 9));
    CHECK(s.size() == 9 && s.front() == 1 && s.back() == 9);

    KVCacheManager q8(cache_cfg("q8_0"), ModelConfig{}, 1, 8, 128, 0, false, hostmem());
    CHECK(q8.group(0).bytes_per_block == (size_t)16 * 8 * 136);
    CHECK(q8.kv_bytes_per_token(0) == (size_t)8 * 136 * 2);
    ModelConfig skip;
    skip.kv_cache_layers = {true, false, true};
    KVCacheManager sk(cache_cfg("fp16"), skip, 3, 8, 128, 0, false, hostmem());
    CHECK((sk.group(0).layer_indices == std::vector<int>{0, 2}));
    CHECK(sk.group(0).bytes_per_block == (size_t)16 * 8 * 128 * 2);
}

static void test_token_io(const std::string& layout) {
    const int H = 4, D = 64;
    KVCacheManager m(cache_cfg("fp16", "", layout), ModelConfig{}, 1, H, D, 0, false, hostmem());
    m.allocate_gpu_blocks_for_group(0, 4);
    const size_t E = D * 2, T = H * E, page = 16 * T;
    std::vector<uint8_t> tok(2 * T);
    for (size_t i = 0; i < tok.size(); ++i) tok[i] = (uint8_t)(i * 7 + 1);
    const int64_t slot = 2 * 16 + 5;
    m.write_kv_token(0, slot, tok.data(), nullptr);
    auto* K = static_cast<uint8_t*>(m.key_cache_ptr(0));
    auto* V = static_cast<uint8_t*>(m.value_cache_ptr(0));
    for (int h = 0; h < H; ++h) {
        const size_t off = layout == "hnd" ? 2 * page + ((size_t)h * 16 + 5) * E : 2 * page + 5 * T + h * E;
        CHECK(std::memcmp(K + off, tok.data() + h * E, E) == 0);
        CHECK(std::memcmp(V + off, tok.data() + T + h * E, E) == 0);
    }
    std::vector<uint8_t> back(2 * T, 0);
    m.read_kv_token(0, slot, back.data(), nullptr);
    CHECK(back == tok);

    KVCacheManager tq(cache_cfg("auto", "turboquant_4bit_nc"), ModelConfig{}, 1, H, 128, 0, false, hostmem());
    tq.allocate_gpu_blocks_for_group(0, 3);
    std::vector<uint8_t> t2(H * 134);
    for (size_t i = 0; i < t2.size(); ++i) t2[i] = (uint8_t)(i ^ 0x5a);
    tq.write_kv_token(0, 16 + 3, t2.data(), nullptr);
    auto* P = static_cast<uint8_t*>(tq.key_cache_ptr(0));
    CHECK(std::memcmp(P + (size_t)16 * H * 134 + 3 * H * 134, t2.data(), t2.size()) == 0);
}

static void test_swap() {
    KVCacheManager m(cache_cfg("fp16"), ModelConfig{}, 2, 2, 64, 0, false, hostmem());
    m.allocate_gpu_blocks_for_group(0, 6);
    m.allocate_cpu_blocks_for_group(0, 4);
    auto s = ids_of(m.allocate_slots("r", 32));  // blocks 1, 2
    const size_t bb = m.group(0).bytes_per_block;
    for (int l = 0; l < 2; ++l)
        for (int64_t b : s) {
            std::memset(static_cast<uint8_t*>(m.key_cache_ptr(l)) + b * bb, (int)(10 * l + b), bb);
            std::memset(static_cast<uint8_t*>(m.value_cache_ptr(l)) + b * bb, (int)(50 + 10 * l + b), bb);
        }
    // quantized pages need no separate compression step (reference stubs)
    CHECK(m.compress_kv_block(s[0]) && m.decompress_kv_block(s[0]));
    m.swap_request_slots("r");
    CHECK(m.num_free_cpu_blocks() == 2);
    CHECK(m.num_free_gpu_blocks() == 5);
    for (int l = 0; l < 2; ++l)
        for (int64_t b : s) std::memset(static_cast<uint8_t*>(m.key_cache_ptr(l)) + b * bb, 0xEE, bb);
    // other requests take the device blocks meanwhile
    m.allocate_slots("other", 32);
    m.swap_back_request_slots("r");
    auto now = ids_of(m.request_slots().at("r"));
    CHECK(now.size() == 2);
    CHECK(m.num_free_cpu_blocks() == 4);
    for (int l = 0; l < 2; ++l)
        for (size_t i = 0; i < now.size(); ++i) {
            auto* k = static_cast<uint8_t*>(m.key_cache_ptr(l)) + now[i] * bb;
            auto* v = static_cast<uint8_t*>(m.value_cache_ptr(l)) + now[i] * bb;
            CHECK(k[0] == (uint8_t)(10 * l + s[i]) && k[bb - 1] == (uint8_t)(10 * l + s[i]));
            CHECK(v[0] == (uint8_t)(50 + 10 * l + s[i]));
        }
}

static void test_metadata() {
    KVCacheManager m(cache_cfg(), ModelConfig{}, 1, 8, 128, 0, false, hostmem());
    m.allocate_gpu_blocks_for_group(0, 32);
    // a request with 20 cached tokens decoding one more, and a fresh prefill of 18
    m.allocate_slots("dec", 20);  // blocks 1, 2
    std::vector<ScheduledRequest> reqs(2);
    reqs[0].request_id = "dec";
    reqs[0].num_computed_tokens = 20;
    reqs[0].is_prefill = false;
    reqs[1].request_id = "pre";
    reqs[1].num_scheduled_tokens = 18;
    reqs[1].is_prefill = true;
    auto h = build_batch_metadata(m, reqs);
    CHECK(h.ok && h.num_reqs == 2 && h.num_tokens == 19);
    CHECK(h.max_num_blocks_per_req == 2);
    CHECK((h.seq_lens == std::vector<int32_t>{21, 18}));
    CHECK((h.block_tables == std::vector<int32_t>{1, 2, 3, 4}));
    CHECK(h.slot_mapping[0] == 2 * 16 + 4);  // position 20 -> block 2, offset 4
    for (int i = 0; i < 18; ++i) {
        const int64_t blk = i < 16 ? 3 : 4;
        CHECK(h.slot_mapping[1 + i] == blk * 16 + i % 16);
        CHECK(h.token_positions[1 + i] == i && h.token_to_seq[1 + i] == 1);
    }
    CHECK((h.cu_seqlens == std::vector<int32_t>{0, 1, 19}));
    CHECK(h.num_prefills == 1 && h.num_decodes == 1 && h.num_prefill_tokens == 18);
    // a request that cannot get blocks marks the batch
    std::vector<ScheduledRequest> big(1);
    big[0].request_id = "huge";
    big[0].num_scheduled_tokens = 16 * 40;
    big[0].is_prefill = true;
    CHECK(!build_batch_metadata(m, big).ok);
}

static void test_errors() {
    bool threw = false;
    try {
        reshape_and_cache(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 8, 128, 16, 0, "fp4_e2m1",
                          nullptr, nullptr, ScalarType::FLOAT16);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("kv_cache_dtype") != std::string::npos;
    }
    CHECK(threw);
    threw = false;
    try {
        VMC_CALL(vmc_tq_config_from_method(128, "turboquant_k8v4", nullptr));
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("invalid argument") != std::string::npos;
    }
    CHECK(threw);
    threw = false;
    try {
        PagedAttentionBackend b("xyz");
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw);
    threw = false;
    try {
        convert_fp8(nullptr, nullptr, 1.0, 16, "fp8_e4m3", ScalarType::FLOAT16);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("convert_fp8") != std::string::npos;
    }
    CHECK(threw);
    convert_fp8(nullptr, nullptr, 1.0, 0, "fp8_e4m3", ScalarType::FLOAT16);  // nothing to convert
    threw = false;
    try {
        reshape_and_cache_flash(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 8, 128, 16, 0, "int4",
                                nullptr, nullptr, ScalarType::FLOAT16);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("kv_cache_dtype") != std::string::npos;
    }
    CHECK(threw);
    // fp8 pages: no tokens is no work; a head_dim the fp8 append does not
    // take is an argument error
    reshape_and_cache(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 8, 128, 16, 0, "fp8_e5m2", nullptr, nullptr,
                      ScalarType::FLOAT16);
    threw = false;
    try {
        reshape_and_cache(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 8, 100, 16, 0, "fp8_e4m3", nullptr,
                          nullptr, ScalarType::FLOAT16);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("vmc_reshape_and_cache_fp8") != std::string::npos;
    }
    CHECK(threw);
    TQWorkspace tw;
    tw.ensure_store(64, 128, 0);  // no scratch: allocates nothing
    CHECK(tw.decode_workspace == nullptr);
    CHECK(vmc_layout_of("hnd") == VMC_LAYOUT_HND);
    CHECK(vmc_kv_format_of("auto", ScalarType::BFLOAT16) == VMC_KV_BF16);
    CHECK(vmc_kv_format_of("q4_0", ScalarType::FLOAT16) == VMC_KV_Q4_0);
}

// the TurboQuant attention node: set-up, per-rank head split, op_params
// decoding and every error the node raises before a launch
static void test_tq_bridge() {
    using official::TurboQuantKvBridge;
    KVCacheManager tq(cache_cfg("auto", "turboquant_3bit_nc"), ModelConfig{}, 4, 4, 128, 0, false, hostmem());
    tq.set_tq_boundary_layers({0});
    tq.allocate_gpu_blocks_for_group(0, 4);
    tq.allocate_gpu_blocks_for_group(1, 4);
    TurboQuantKvBridge b;
    b.initialize(cache_cfg("auto", "turboquant_3bit_nc"), 16, 4, 128, &tq, 0, 4, 1, ScalarType::FLOAT16);
    CHECK(b.num_attention_heads() == 16 && b.num_kv_heads() == 4 && b.head_dim() == 128);
    CHECK(b.tq_config().slot_size_aligned == 102 && b.tq_layer_enabled_count() == 3);
    CHECK(!b.kv_cache_ptr(0) && b.kv_cache_ptr(1) == tq.key_cache_ptr(1) && !b.kv_cache_ptr(4));
    CHECK(!vm_c_tq_bridge_layer_uses_turboquant(nullptr, 1));
    CHECK(!vm_c_tq_bridge_layer_uses_turboquant(&b, 0) && vm_c_tq_bridge_layer_uses_turboquant(&b, 2));
    TurboQuantKvBridge split;
    split.initialize(cache_cfg("auto", "turboquant_3bit_nc"), 16, 4, 128, &tq, 0, 4, 8);
    CHECK(split.num_attention_heads() == 2 && split.num_kv_heads() == 1);
    auto throws = [](const std::function<void()>& f, const char* what) {
        try {
            f();
        } catch (const std::runtime_error& e) {
            return std::string(e.what()).find(what) != std::string::npos;
        }
        return false;
    };
    CHECK(throws([&] { split.initialize(cache_cfg("auto", "turboquant_3bit_nc"), 16, 4, 128, &tq, 0, 4, 0); },
                 "tp_size must be positive"));
    CHECK(throws([&] { split.initialize(cache_cfg("auto", "turboquant_3bit_nc"), 4, 4, 128, &tq, 0, 4, 8); },
                 "num_attention_heads per rank is zero"));
    KVCacheManager plain(cache_cfg("fp16"), ModelConfig{}, 1, 4, 128, 0, false, hostmem());
    CHECK(throws([&] { split.initialize(cache_cfg("fp16"), 16, 4, 128, &plain, 0, 1); }, "is not TurboQuant"));
    // op_params {layer, kq_scale, bridge}
    auto params = [](int32_t layer, float scale, void* br) {
        std::vector<unsigned char> p(official::kTqAttnOpBytes);
        std::memcpy(p.data() + official::kTqAttnOpLayer, &layer, 4);
        std::memcpy(p.data() + official::kTqAttnOpScale, &scale, 4);
        std::memcpy(p.data() + official::kTqAttnOpBridge, &br, sizeof(br));
        return p;
    };
    // q as the head-split view [128, 16, 3], as one token [2048, 1], and as
    // [2048, 3] (third stride set, second extent > 1: read as head-split, so
    // 6144 wide, as the reference reads it)
    const int64_t ne3[4] = {128, 16, 3, 1}, ne2[4] = {2048, 1, 1, 1}, bad[4] = {128, 8, 3, 1};
    const int64_t flat3[4] = {2048, 3, 1, 1};
    const size_t nb3[4] = {2, 256, 4096, 12288}, nb2[4] = {2, 4096, 4096, 4096}, nbf[4] = {2, 4096, 12288, 12288};
    int x = 0;
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, nullptr).data(), &x, ne3, nb3, &x, &x, &x); },
                 "null bridge"));
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, &b).data(), &x, bad, nb3, &x, &x, &x); },
                 "q embedding dim mismatch: ne0=1024 expected=2048"));
    CHECK(throws([&] { official::turboquant_attn_op(params(0, 0.1f, &b).data(), &x, ne3, nb3, &x, &x, &x); },
                 "null kv cache for layer 0"));
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, &b).data(), &x, flat3, nbf, &x, &x, &x); },
                 "ne0=6144 expected=2048"));
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, &b).data(), &x, ne3, nb3, &x, &x, &x); },
                 "slot_mapping not set"));
    CHECK(throws([&] { official::turboquant_attn_op(params(2, 0.1f, &b).data(), &x, ne2, nb2, &x, &x, &x); },
                 "slot_mapping not set"));
    b.set_batch_metadata(nullptr, nullptr, nullptr, 3, 3, 4, 16, true, 3, 0, nullptr, nullptr, nullptr);
    CHECK(b.is_prefill() && b.num_prefill_tokens() == 3);
    b.mark_decode_mode(5);
    CHECK(!b.is_prefill() && b.num_decode_tokens() == 5 && b.num_tokens() == 5 && b.num_prefill_tokens() == 0);
    // batch metadata checked before any launch: a decode-only step must have
    // one token per request; a step with prefill tokens needs token_to_seq /
    // token_positions (the Engine's per-request block tables and lengths)
    const int64_t fake_slots = 0;
    b.set_batch_metadata(&fake_slots, nullptr, nullptr, 3, 2, 4, 16, false, 0, 3, nullptr, nullptr, nullptr);
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, &b).data(), &x, ne3, nb3, &x, &x, &x); },
                 "decode step of 3 tokens over 2 requests"));
    b.set_batch_metadata(&fake_slots, nullptr, nullptr, 3, 2, 4, 16, true, 3, 0, nullptr, nullptr, nullptr);
    CHECK(throws([&] { official::turboquant_attn_op(params(1, 0.1f, &b).data(), &x, ne3, nb3, &x, &x, &x); },
                 "prefill step without token_to_seq"));
    // the reference's workspace signature (kernels_turboquant.h:103): no
    // device memory for head_dim other than 128, one split, or no rows
    TQWorkspace ws;
    ws.ensure_decode(16, 64, 32, 0);
    ws.ensure_decode(16, 128, 1, 0);
    ws.ensure_decode(0, 128, 32, 0);
    CHECK(ws.decode_workspace == nullptr && ws.decode_bytes == 0);
}

int main() {
    const std::vector<std::pair<const char*, std::function<void()>>> tests = {
        {"free_queue", test_free_queue},
        {"allocation_order", test_allocation_order},
        {"prefix_cache", test_prefix_cache},
        {"layouts", test_layouts},
        {"token_io_nhd", [] { test_token_io("nhd"); }},
        {"token_io_hnd", [] { test_token_io("hnd"); }},
        {"swap", test_swap},
        {"metadata", test_metadata},
        {"errors", test_errors},
        {"tq_bridge", test_tq_bridge},
    };
    for (auto& t : tests) {
        const int before = g_fail;
        t.second();
        std::printf("%s %s\n", g_fail == before ? "ok  " : "FAIL", t.first);
    }
    return g_fail == 0 ? 0 : 1;
}
