// vm_c/kernels_turboquant.hpp -- TurboQuant KV entry points on HIP.
//
// Same names, argument order and meaning as vm_c
// include/vm_c/cuda/kernels_turboquant.h:10-144; hipStream_t replaces
// cudaStream_t.  Underneath every call is the C ABI of vmc_attn.h.
//
// Differences a caller can see:
//   * TQBuffers holds the Hadamard matrix, centroids and midpoints on the
//     device for callers that read them; the gfx950 kernels do not need them
//     (the rotation is an in-register Walsh-Hadamard transform and the
//     codebook travels in the kernel arguments).
//   * TQWorkspace holds only the decode workspace (split partials); the store
//     is one fused kernel without scratch.  It is sized by ensure_decode;
//     TurboQuantBackend::ensure_workspace sizes it for max_num_seqs requests
//     of any length, so its decode calls never allocate.  A direct call that
//     needs more grows it before the launch (vm_c grew it inside the call,
//     turboquant_kernels.cu:704-741).
//   * The activation dtype is an argument (trailing, defaulted to fp16) of
//     turboquant_store and turboquant_decode_attention: vm_c reads it from
//     the process-wide gpu().compute_dtype() (turboquant_kernels.cu:808,
//     :966).  Norms, scales and zeros are stored in that dtype.
//   * "turboquant_k8v4" (fp8 keys): the decode reads no norm for fp8 keys;
//     the reference multiplies them by the two bytes at +mse_bytes, which
//     for this layout are the first V code bytes (turboquant_kernels.cu:
//     443-450), and that is not reproduced.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "vm_c/common.hpp"

namespace vm_c {

struct TQConfig {
    static constexpr int kMaxSupportedHeadDim = 256;

    int head_dim = 128;
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
    int max_num_kv_splits = 32;
    // Not in vm_c: the per-32-group variant of the benchmark configurations
    // ("turboquant_4bit_g32" / "turboquant_3bit_g32"; format in vmc_attn.h).
    int group_size = 0;        // 0: the reference layout
    uint64_t sign_seed = 0;    // rotation signs (0: all +1), the same for store and decode

    void compute_layout();
    // "turboquant_4bit_nc" (default), "turboquant_3bit_nc", "turboquant_k3v4_nc",
    // "turboquant_k8v4", and the variants "turboquant_4bit_g32",
    // "turboquant_3bit_g32"; gpu_device is accepted for signature compatibility
    static TQConfig from_method(int head_dim, const char* method, int gpu_device = 0);

    vmc_tq_config to_c() const;
};

struct TQBuffers {
    void* hadamard = nullptr;       // fp32 [d][d]
    void* hadamard_fp16 = nullptr;  // fp16 [d][d]
    void* centroids = nullptr;      // fp32 [2^bits]
    void* midpoints = nullptr;      // fp32 [2^bits - 1]
    int head_dim = 0;
    int centroid_bits = 0;
    bool initialized = false;

    void init(int head_dim, int centroid_bits, int gpu_device);
    void free_buf();
};

struct TQWorkspace {
    void* decode_workspace = nullptr;
    size_t decode_bytes = 0;
    int gpu_device = 0;

    // enough for batch_size x num_heads queries over max_num_blocks_per_req pages
    void ensure_decode(int batch_size, int num_heads, int num_kv_heads, int head_dim,
                       int64_t max_num_blocks_per_req, int64_t block_size,
                       int max_num_kv_splits, int gpu_device);
    // the reference's form (kernels_turboquant.h:103; its callers
    // attention_backend.cpp:129-132 and turboquant_kv_bridge.cpp:162-163):
    // enough for bhq = batch x num_heads query rows with num_kv_splits splits
    // each, at any context length -- a decode of that many rows allocates
    // nothing.  head_dim other than 128 and num_kv_splits <= 1 need none.
    void ensure_decode(int bhq, int head_dim, int num_kv_splits, int gpu_device);
    // turboquant_kernels.cu:704-741 grows four fp32 scratch buffers for its
    // multi-launch store; the fused HIP store needs none, so this only keeps
    // the reference's call sites compiling
    void ensure_store(int nh, int head_dim, int gpu_device) {
        (void)nh;
        (void)head_dim;
        (void)gpu_device;
    }
    void free_buf();
};

void turboquant_store(const void* key, const void* value, void* kv_cache,
                      const int64_t* slot_mapping, int num_tokens, int num_kv_heads,
                      int head_dim, int64_t block_size, const TQConfig& config,
                      const TQBuffers& buffers, TQWorkspace& workspace,
                      hipStream_t stream = nullptr, ScalarType dtype = ScalarType::FLOAT16);

void turboquant_decode_attention(void* output, const void* query, const void* kv_cache,
                                 const int32_t* block_tables, const int32_t* seq_lens,
                                 int batch_size, int num_heads, int num_kv_heads, int head_dim,
                                 float scale, int64_t block_size, int64_t max_num_blocks_per_req,
                                 const TQConfig& config, const TQBuffers& buffers,
                                 TQWorkspace& workspace, int max_num_kv_splits,
                                 hipStream_t stream = nullptr,
                                 ScalarType dtype = ScalarType::FLOAT16);

// Sylvester Hadamard matrix times 1/sqrt(d) (turboquant_kernels.cu:551-570)
void build_hadamard_on_host(float* out, int d);
// Lloyd-Max centroids for N(0, 1/d) (turboquant_kernels.cu:578-623)
void solve_lloyd_max_centroids(float* centroids_out, int d, int bits);

}  // namespace vm_c
