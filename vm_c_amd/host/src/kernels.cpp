// kernels.cpp -- vm_c's kernel entry points (kernels_turboquant.h,
// kernels_cache.h, kernels_attention.h, kernels_flash_attn.h,
// kernels_fused_attn.h) over the C ABI
// of vmc_attn.h.  Argument checks that need no device live in the C ABI;
// this layer maps vm_c's string/enum conventions and turns failures into
// std::runtime_error.
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "vm_c/kernels_attention.hpp"
#include "vm_c/kernels_fused_attn.hpp"
#include "vm_c/kernels_turboquant.hpp"

namespace vm_c {

// ------------------------------------------------------------ TurboQuant

void TQConfig::compute_layout() {
    if (group_size != 0) {  // per-32-group variant: two parts of four blocks
        const int part = key_quant_bits == 4 ? 80 : 56;
        n_centroids = 0;
        mse_bytes = val_data_bytes = 16 * key_quant_bits;
        key_packed_size = value_packed_size = part;
        slot_size = slot_size_aligned = 2 * part;
        return;
    }
    n_centroids = 1 << key_quant_bits;
    if (key_fp8) {
        mse_bytes = head_dim;
        key_packed_size = head_dim;
    } else {
        mse_bytes = (head_dim * key_quant_bits + 7) / 8;
        key_packed_size = mse_bytes + 2;
    }
    val_data_bytes = (head_dim * value_quant_bits + 7) / 8;
    value_packed_size = val_data_bytes + 4;
    slot_size = key_packed_size + value_packed_size;
    slot_size_aligned = slot_size + (slot_size % 2);
}

TQConfig TQConfig::from_method(int head_dim_, const char* method, int gpu_device) {
    (void)gpu_device;
    TQConfig cfg;
    cfg.head_dim = head_dim_;
    const std::string m = method ? method : "";
    if (m == "turboquant_k8v4") {
        cfg.key_quant_bits = 8;
        cfg.value_quant_bits = 4;
        cfg.norm_correction = false;
        cfg.key_fp8 = true;
        cfg.fp8_e4b15 = false;
    } else if (m == "turboquant_k3v4_nc") {
        cfg.key_quant_bits = 3;
        cfg.value_quant_bits = 4;
    } else if (m == "turboquant_3bit_nc") {
        cfg.key_quant_bits = 3;
        cfg.value_quant_bits = 3;
    } else if (m == "turboquant_4bit_g32" || m == "turboquant_3bit_g32") {
        cfg.key_quant_bits = cfg.value_quant_bits = m == "turboquant_4bit_g32" ? 4 : 3;
        cfg.norm_correction = false;
        cfg.group_size = 32;
    }
    cfg.compute_layout();
    return cfg;
}

vmc_tq_config TQConfig::to_c() const {
    vmc_tq_config c;
    std::memset(&c, 0, sizeof(c));  // the padding before sign_seed too (callers compare bytes)
    c.head_dim = head_dim;
    c.key_quant_bits = key_quant_bits;
    c.value_quant_bits = value_quant_bits;
    c.norm_correction = norm_correction;
    c.key_fp8 = key_fp8;
    c.fp8_e4b15 = fp8_e4b15;
    c.mse_bytes = mse_bytes;
    c.key_packed_size = key_packed_size;
    c.val_data_bytes = val_data_bytes;
    c.value_packed_size = value_packed_size;
    c.slot_size = slot_size;
    c.slot_size_aligned = slot_size_aligned;
    c.n_centroids = n_centroids;
    c.max_num_kv_splits = max_num_kv_splits;
    c.group_size = group_size;
    c.sign_seed = sign_seed;
    return c;
}

void build_hadamard_on_host(float* out, int d) {
    const float c = 1.0f / std::sqrt((float)d);
    for (int i = 0; i < d; ++i)
        for (int j = 0; j < d; ++j) out[i * d + j] = (__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c;
}

void solve_lloyd_max_centroids(float* centroids_out, int d, int bits) {
    std::vector<float> mid((size_t)(1 << bits));
    VMC_CALL(vmc_tq_host_tables(d, bits, centroids_out, mid.data()));
}

namespace {
// fp32 -> fp16 bits, round to nearest even (host side, no compiler fp16 type)
uint16_t to_half_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
    if (ax < 0x38800000u) {  // subnormal half (or zero)
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 16777216.0f));
    }
    const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
}

template <typename T>
void* upload(const std::vector<T>& v) {
    void* p = nullptr;
    HIP_CHECK(hipMalloc(&p, v.size() * sizeof(T)));
    HIP_CHECK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    return p;
}
}  // namespace

void TQBuffers::init(int head_dim_, int centroid_bits_, int gpu_device) {
    if (initialized) free_buf();
    HIP_CHECK(hipSetDevice(gpu_device));
    head_dim = head_dim_;
    centroid_bits = centroid_bits_;
    const int d = head_dim_, n = 1 << centroid_bits_;
    std::vector<float> h((size_t)d * d), c(n), m(n - 1);
    build_hadamard_on_host(h.data(), d);
    VMC_CALL(vmc_tq_host_tables(d, centroid_bits_, c.data(), m.data()));
    std::vector<uint16_t> h16(h.size());
    for (size_t i = 0; i < h.size(); ++i) h16[i] = to_half_bits(h[i]);
    hadamard = upload(h);
    hadamard_fp16 = upload(h16);
    centroids = upload(c);
    midpoints = upload(m);
    initialized = true;
}

void TQBuffers::free_buf() {
    for (void** p : {&hadamard, &hadamard_fp16, &centroids, &midpoints}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    initialized = false;
}

void TQWorkspace::ensure_decode(int batch_size, int num_heads, int num_kv_heads, int head_dim,
                                int64_t max_num_blocks_per_req, int64_t block_size,
                                int max_num_kv_splits, int device) {
    const size_t need = vmc_turboquant_decode_workspace_size(batch_size, num_heads, num_kv_heads,
                                                             head_dim, max_num_blocks_per_req,
                                                             block_size, max_num_kv_splits);
    if (need <= decode_bytes) return;
    HIP_CHECK(hipSetDevice(device));
    if (decode_workspace) HIP_CHECK(hipFree(decode_workspace));
    decode_workspace = nullptr;
    decode_bytes = 0;
    HIP_CHECK(hipMalloc(&decode_workspace, need));
    decode_bytes = need;
    gpu_device = device;
}

void TQWorkspace::ensure_decode(int bhq, int head_dim, int num_kv_splits, int device) {
    // the decode's split partials are fp32 rows of head_dim + 4 floats, at
    // most two per launched workgroup and query head, with at most
    // batch x num_kv_splits workgroups (vmc_turboquant_decode_workspace_size)
    if (bhq <= 0 || num_kv_splits <= 1 || (head_dim != 128 && head_dim != 256)) return;
    const size_t need = (size_t)2 * (size_t)num_kv_splits * (size_t)bhq * (size_t)(head_dim + 4) * sizeof(float);
    if (need <= decode_bytes) return;
    HIP_CHECK(hipSetDevice(device));
    if (decode_workspace) HIP_CHECK(hipFree(decode_workspace));
    decode_workspace = nullptr;
    decode_bytes = 0;
    HIP_CHECK(hipMalloc(&decode_workspace, need));
    decode_bytes = need;
    gpu_device = device;
}

void TQWorkspace::free_buf() {
    if (decode_workspace) (void)hipFree(decode_workspace);
    decode_workspace = nullptr;
    decode_bytes = 0;
}

void turboquant_store(const void* key, const void* value, void* kv_cache,
                      const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                      int64_t block_size, const TQConfig& config, const TQBuffers& buffers,
                      TQWorkspace& workspace, hipStream_t stream, ScalarType dtype) {
    (void)buffers;
    (void)workspace;
    const vmc_tq_config c = config.to_c();
    VMC_CALL(vmc_turboquant_store(key, value, kv_cache, slot_mapping, num_tokens, num_kv_heads,
                                  head_dim, block_size, &c, vmc_dtype_of(dtype), stream));
}

void turboquant_decode_attention(void* output, const void* query, const void* kv_cache,
                                 const int32_t* block_tables, const int32_t* seq_lens,
                                 int batch_size, int num_heads, int num_kv_heads, int head_dim,
                                 float scale, int64_t block_size, int64_t max_num_blocks_per_req,
                                 const TQConfig& config, const TQBuffers& buffers,
                                 TQWorkspace& workspace, int max_num_kv_splits,
                                 hipStream_t stream, ScalarType dtype) {
    (void)buffers;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    workspace.ensure_decode(batch_size, num_heads, num_kv_heads, head_dim, max_num_blocks_per_req,
                            block_size, max_num_kv_splits, dev);
    const vmc_tq_config c = config.to_c();
    VMC_CALL(vmc_turboquant_decode_attention(
        output, query, kv_cache, block_tables, seq_lens, batch_size, num_heads, num_kv_heads,
        head_dim, scale, block_size, max_num_blocks_per_req, &c, vmc_dtype_of(dtype), max_num_kv_splits,
        workspace.decode_workspace, workspace.decode_bytes, stream));
}

// ------------------------------------------------------------ paged KV

void swap_blocks(void* src, void* dst, int64_t block_size_in_bytes, const int64_t* block_mapping,
                 int64_t num_blocks, int src_device, int dst_device, hipStream_t stream) {
    (void)src_device;
    (void)dst_device;
    auto* s = static_cast<const uint8_t*>(src);
    auto* d = static_cast<uint8_t*>(dst);
    for (int64_t i = 0; i < num_blocks; ++i) {
        const int64_t from = block_mapping[2 * i], to = block_mapping[2 * i + 1];
        HIP_CHECK(hipMemcpyAsync(d + to * block_size_in_bytes, s + from * block_size_in_bytes,
                                 (size_t)block_size_in_bytes, hipMemcpyDefault, stream));
    }
}

void reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                       const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                       int64_t block_size, int64_t cache_stride, const std::string& kv_cache_dtype,
                       const void* k_scale, const void* v_scale, ScalarType dtype,
                       hipStream_t stream, const std::string& layout) {
    if (kv_cache_dtype == "fp8_e4m3" || kv_cache_dtype == "fp8_e5m2") {
        // both strings store E4M3 bytes of x / scale (cache_kernels.cu:101-131)
        VMC_CALL(vmc_reshape_and_cache_fp8(key, value, key_cache, value_cache, slot_mapping, num_tokens,
                                           num_kv_heads, head_dim, block_size, cache_stride,
                                           static_cast<const float*>(k_scale), static_cast<const float*>(v_scale),
                                           vmc_dtype_of(dtype), vmc_layout_of(layout), stream));
        return;
    }
    // the scales only apply to fp8 caches (cache_kernels.cu:42-51)
    VMC_CALL(vmc_reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens,
                                   num_kv_heads, head_dim, block_size, cache_stride,
                                   vmc_kv_format_of(kv_cache_dtype, dtype), vmc_dtype_of(dtype),
                                   vmc_layout_of(layout), stream));
}

void reshape_and_cache_flash(const void* key, const void* value, void* key_cache, void* value_cache,
                             const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                             int64_t block_size, int64_t cache_stride, const std::string& kv_cache_dtype,
                             const void* k_scale, const void* v_scale, ScalarType dtype, hipStream_t stream,
                             const std::string& layout) {
    reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_kv_heads, head_dim,
                      block_size, cache_stride, kv_cache_dtype, k_scale, v_scale, dtype, stream, layout);
}

void convert_fp8(void* dst_cache, const void* src_cache, double scale, int64_t num_elements,
                 const std::string& kv_cache_dtype, ScalarType dtype, hipStream_t stream) {
    if (num_elements <= 0) return;  // cache_kernels.cu:193
    // "fp8_e4m3" -> E4M3, any other string -> E5M2 (cache_kernels.cu:196-211)
    VMC_CALL(vmc_convert_fp8(dst_cache, src_cache, scale, num_elements, kv_cache_dtype == "fp8_e4m3" ? 0 : 1,
                             vmc_dtype_of(dtype), stream));
}

void paged_attention_prefill(void* out, const void* query, const void* key_cache,
                             const void* value_cache, int num_tokens, int num_heads,
                             int num_kv_heads, int head_dim, float scale, int64_t block_size,
                             int64_t max_num_blocks_per_req, const int32_t* block_tables,
                             const int32_t* seq_lens, const int32_t* token_to_seq,
                             const int32_t* token_positions, int num_reqs,
                             const std::string& kv_cache_dtype, ScalarType dtype,
                             hipStream_t stream, const std::string& layout) {
    (void)seq_lens;
    (void)num_reqs;
    VMC_CALL(vmc_paged_attention_prefill(out, query, key_cache, value_cache, num_tokens, num_heads,
                                         num_kv_heads, head_dim, scale, (int)block_size,
                                         (int)max_num_blocks_per_req, block_tables, token_to_seq,
                                         token_positions, vmc_dtype_of(dtype),
                                         vmc_kv_format_of(kv_cache_dtype, dtype), vmc_layout_of(layout),
                                         1, nullptr, 0, stream));
}

void flash_attention_prefill_v2(void* output, const void* query, const void* key_cache,
                                const void* value_cache, int num_tokens, int num_heads,
                                int num_kv_heads, int head_dim, float scale, int64_t block_size,
                                int64_t max_num_blocks_per_req, const int32_t* block_tables,
                                const int32_t* seq_lens, const int32_t* token_to_seq,
                                const int32_t* token_positions, int num_reqs,
                                const std::string& kv_cache_dtype, ScalarType dtype,
                                hipStream_t stream, const std::string& layout) {
    VMC_CALL(vmc_flash_attention_prefill_v2(output, query, key_cache, value_cache, num_tokens, num_heads,
                                            num_kv_heads, head_dim, scale, (int)block_size,
                                            (int)max_num_blocks_per_req, block_tables, seq_lens,
                                            token_to_seq, token_positions, num_reqs, vmc_dtype_of(dtype),
                                            vmc_kv_format_of(kv_cache_dtype, dtype), vmc_layout_of(layout),
                                            stream));
}

namespace {
void check_params(const AttentionParams& p, const float* alibi_slopes) {
    if (alibi_slopes) throw std::runtime_error("paged attention: ALiBi is not supported");
    if (p.blocksparse_vert_stride > 1 || p.blocksparse_local_blocks > 0)
        throw std::runtime_error("paged attention: block-sparse attention is not supported");
}
}  // namespace

size_t paged_attention_v2_workspace_size(const AttentionParams& p) {
    return vmc_paged_decode_workspace_size(p.batch_size, p.num_heads, p.num_kv_heads, p.head_dim,
                                           p.max_num_blocks_per_req, p.block_size, 0);
}

void paged_attention_v1(void* out, const void* query, const void* key_cache,
                        const void* value_cache, const AttentionParams& p,
                        const int32_t* block_tables, const int32_t* seq_lens,
                        const float* alibi_slopes, const std::string& kv_cache_dtype,
                        const void* k_scale, const void* v_scale, hipStream_t stream,
                        const std::string& layout) {
    check_params(p, alibi_slopes);
    if (k_scale || v_scale) throw std::runtime_error("paged attention: fp8 k/v scales are not supported");
    // one pass per sequence: no split, no workspace
    VMC_CALL(vmc_paged_attention_decode(out, query, key_cache, value_cache, block_tables, seq_lens,
                                        p.batch_size, p.num_heads, p.num_kv_heads, p.head_dim,
                                        p.block_size, p.max_num_blocks_per_req, p.scale,
                                        vmc_dtype_of(p.dtype), vmc_kv_format_of(kv_cache_dtype, p.dtype),
                                        vmc_layout_of(layout), 1, nullptr, 0, stream));
}

void paged_attention_v2(void* out, void* exp_sums, void* max_logits, void* tmp_out,
                        const void* query, const void* key_cache, const void* value_cache,
                        const AttentionParams& p, const int32_t* block_tables,
                        const int32_t* seq_lens, const float* alibi_slopes,
                        const std::string& kv_cache_dtype, const void* k_scale,
                        const void* v_scale, hipStream_t stream, const std::string& layout) {
    (void)exp_sums;
    (void)max_logits;
    check_params(p, alibi_slopes);
    if (k_scale || v_scale) throw std::runtime_error("paged attention: fp8 k/v scales are not supported");
    VMC_CALL(vmc_paged_attention_decode(out, query, key_cache, value_cache, block_tables, seq_lens,
                                        p.batch_size, p.num_heads, p.num_kv_heads, p.head_dim,
                                        p.block_size, p.max_num_blocks_per_req, p.scale,
                                        vmc_dtype_of(p.dtype), vmc_kv_format_of(kv_cache_dtype, p.dtype),
                                        vmc_layout_of(layout), 0, tmp_out,
                                        paged_attention_v2_workspace_size(p), stream));
}

// ------------------------------------------------------------ prefill

void flash_attention_prefill_local(void* output, const void* query, const void* key,
                                   const void* value, int num_tokens, int num_heads,
                                   int num_kv_heads, int head_dim, float scale,
                                   const int32_t* token_to_seq, const int32_t* token_positions,
                                   ScalarType dtype, hipStream_t stream) {
    (void)token_to_seq;
    VMC_CALL(vmc_flash_attention_prefill(output, query, key, value, num_tokens, num_heads,
                                         num_kv_heads, head_dim, scale, token_positions,
                                         vmc_dtype_of(dtype), nullptr, nullptr, nullptr, 16,
                                         VMC_KV_F16, VMC_LAYOUT_NHD, stream));
}

void flash_attention_prefill_local_with_cache(
    void* output, const void* query, const void* key, const void* value, int num_tokens,
    int num_heads, int num_kv_heads, int head_dim, float scale, const int32_t* token_positions,
    ScalarType dtype, void* key_cache, void* value_cache, const int64_t* slot_mapping,
    int64_t block_size, const std::string& kv_cache_dtype, const std::string& layout,
    hipStream_t stream) {
    VMC_CALL(vmc_flash_attention_prefill(output, query, key, value, num_tokens, num_heads,
                                         num_kv_heads, head_dim, scale, token_positions,
                                         vmc_dtype_of(dtype), key_cache, value_cache, slot_mapping,
                                         block_size, vmc_kv_format_of(kv_cache_dtype, dtype),
                                         vmc_layout_of(layout), stream));
}

// ------------------------------------------------------------ fused norm + RoPE

void fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                              const void* q_norm_weight, const void* k_norm_weight,
                              const void* cos_sin_cache, const int64_t* position_ids,
                              void* key_cache, void* value_cache, const int64_t* slot_mapping,
                              int num_tokens, int num_heads, int num_kv_heads, int head_dim,
                              float rms_norm_eps, bool is_neox, int64_t block_size,
                              int64_t cache_stride, const std::string& kv_cache_dtype,
                              hipStream_t stream, ScalarType dtype, const std::string& layout) {
    // fused_attn_kernels.cu:243: the append needs both the cache and the slots
    const bool store = key_cache != nullptr && slot_mapping != nullptr;
    VMC_CALL(vmc_fused_qk_norm_rope_store(
        q_buf, k_buf, v_buf, q_norm_weight, k_norm_weight, cos_sin_cache, position_ids,
        store ? key_cache : nullptr, store ? value_cache : nullptr, store ? slot_mapping : nullptr,
        num_tokens, num_heads, num_kv_heads, head_dim, rms_norm_eps, is_neox ? 1 : 0, block_size,
        cache_stride, vmc_kv_format_of(kv_cache_dtype, dtype), vmc_layout_of(layout), nullptr,
        vmc_dtype_of(dtype), stream));
}

void fused_qk_norm_rope_store(void* q_buf, void* k_buf, const void* v_buf,
                              const void* q_norm_weight, const void* k_norm_weight,
                              const void* cos_sin_cache, const int64_t* position_ids,
                              void* kv_cache, const int64_t* slot_mapping, int num_tokens,
                              int num_heads, int num_kv_heads, int head_dim, float rms_norm_eps,
                              bool is_neox, int64_t block_size, const TQConfig& config,
                              hipStream_t stream, ScalarType dtype) {
    if (!kv_cache || !slot_mapping)
        throw std::runtime_error("fused_qk_norm_rope_store: TurboQuant append needs a cache and slots");
    const vmc_tq_config c = config.to_c();
    VMC_CALL(vmc_fused_qk_norm_rope_store(
        q_buf, k_buf, v_buf, q_norm_weight, k_norm_weight, cos_sin_cache, position_ids, kv_cache,
        nullptr, slot_mapping, num_tokens, num_heads, num_kv_heads, head_dim, rms_norm_eps,
        is_neox ? 1 : 0, block_size, 0, VMC_KV_F16, VMC_LAYOUT_NHD, &c, vmc_dtype_of(dtype),
        stream));
}

void fused_qk_norm_rope(void* q_buf, void* k_buf, const void* q_norm_weight,
                        const void* k_norm_weight, const void* cos_sin_cache,
                        const int64_t* position_ids, int num_tokens, int num_heads,
                        int num_kv_heads, int head_dim, float rms_norm_eps, bool is_neox,
                        hipStream_t stream, ScalarType dtype) {
    VMC_CALL(vmc_fused_qk_norm_rope_store(q_buf, k_buf, nullptr, q_norm_weight, k_norm_weight,
                                          cos_sin_cache, position_ids, nullptr, nullptr, nullptr,
                                          num_tokens, num_heads, num_kv_heads, head_dim,
                                          rms_norm_eps, is_neox ? 1 : 0, 0, 0, VMC_KV_F16,
                                          VMC_LAYOUT_NHD, nullptr, vmc_dtype_of(dtype), stream));
}

}  // namespace vm_c
