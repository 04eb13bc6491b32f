// tq_tables.cpp -- TurboQuant configuration and host constant tables.
//
// vmc_tq_config_from_method restates TQConfig::compute_layout / from_method
// (include/vm_c/cuda/kernels_turboquant.h:29-74).  The Lloyd-Max solver
// follows solve_lloyd_max_centroids (src/cuda/turboquant_kernels.cu:578-623)
// operation for operation in fp32, so the centroids carry the reference's
// exact bit patterns; midpoints are (c[i] + c[i+1]) * 0.5f (:662-664).  This
// file is compiled with -ffp-contract=off so no a*b+c is fused.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <mutex>
#include <vector>

#include "vmc_attn.h"
#include "vmc_tq.hpp"

namespace vmc {
namespace {

float gaussian_pdf(float x, float sigma2) {
    return (1.0f / sqrtf(2.0f * 3.14159265358979f * sigma2)) * expf(-x * x / (2.0f * sigma2));
}

void solve_lloyd_max(float* out, int d, int bits) {
    const int n = 1 << bits;
    const float sigma2 = 1.0f / (float)d;
    const float sigma = sqrtf(sigma2);
    const float lo = -3.5f * sigma, hi = 3.5f * sigma;
    std::vector<float> c(n);
    for (int i = 0; i < n; ++i) c[i] = lo + (hi - lo) * ((float)i + 0.5f) / (float)n;
    for (int iter = 0; iter < 200; ++iter) {
        std::vector<float> edges(n + 1);
        edges[0] = lo * 3.0f;
        for (int i = 0; i < n - 1; ++i) edges[i + 1] = (c[i] + c[i + 1]) * 0.5f;
        edges[n] = hi * 3.0f;
        std::vector<float> nc(n);
        bool converged = true;
        for (int i = 0; i < n; ++i) {
            const int n_trap = 200;
            const float a = edges[i], b = edges[i + 1];
            const float step = (b - a) / (float)n_trap;
            float num = 0.0f, den = 0.0f;
            for (int j = 0; j <= n_trap; ++j) {
                const float x = a + (float)j * step;
                const float p = gaussian_pdf(x, sigma2);
                const float w = (j == 0 || j == n_trap) ? 0.5f : 1.0f;
                den += w * p;
                num += w * x * p;
            }
            num *= step;
            den *= step;
            nc[i] = (den > 1e-15f) ? num / den : c[i];
            if (fabsf(nc[i] - c[i]) > 1e-10f) converged = false;
        }
        c = nc;
        if (converged) break;
    }
    std::sort(c.begin(), c.end());
    std::memcpy(out, c.data(), sizeof(float) * (size_t)n);
}

}  // namespace

const TQTables& tq_tables(int head_dim, int bits) {
    static std::mutex mu;
    static std::map<std::pair<int, int>, TQTables> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto key = std::make_pair(head_dim, bits);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    TQTables t;
    std::memset(&t, 0, sizeof(t));
    const int n = 1 << bits;
    solve_lloyd_max(t.centroids, head_dim, bits);
    for (int i = 0; i < n - 1; ++i) t.midpoints[i] = (t.centroids[i] + t.centroids[i + 1]) * 0.5f;
    t.n_centroids = n;
    t.rot_c = 1.0f / sqrtf((float)head_dim);
    return cache.emplace(key, t).first->second;
}

G32Signs g32_signs(unsigned long long seed) {
    auto mix = [](uint64_t x) {
        x += 0x9e3779b97f4a7c15ULL;
        x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
        x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
        return x ^ (x >> 31);
    };
    G32Signs s = {{0u, 0u, 0u, 0u}};
    if (seed == 0) return s;
    for (int k = 0; k < 2; ++k) {
        const uint64_t w = mix(mix(mix(seed) ^ 0x5349474eULL) ^ (uint64_t)k);
        s.w[2 * k] = (uint32_t)(w & 0xffffffffu);
        s.w[2 * k + 1] = (uint32_t)(w >> 32);
    }
    return s;
}

bool tq_config_valid(const vmc_tq_config* c) {
    if (!c) return false;
    if (c->key_fp8) {
        // turboquant_k8v4 (kernels_turboquant.h:29-55): head_dim fp8 key
        // bytes, 4-bit values, no norm (196-byte slots at head_dim 128)
        const int d = c->head_dim;
        if (d != 64 && d != 128 && d != 256) return false;
        const int slot = d + d / 2 + 4;
        return c->group_size == 0 && c->key_quant_bits == 8 && c->value_quant_bits == 4 &&
               c->norm_correction == 0 && c->mse_bytes == d && c->key_packed_size == d &&
               c->val_data_bytes == d / 2 && c->value_packed_size == d / 2 + 4 && c->slot_size == slot &&
               c->slot_size_aligned == slot + (slot % 2);
    }
    if (c->group_size != 0) {
        // per-32-group variant: head_dim 128, equal K/V bits, the fixed part sizes
        const int b = c->key_quant_bits;
        if (c->group_size != 32 || c->head_dim != 128 || (b != 3 && b != 4) || c->value_quant_bits != b)
            return false;
        const int part = b == 4 ? 80 : 56;
        return c->mse_bytes == 16 * b && c->key_packed_size == part && c->val_data_bytes == 16 * b &&
               c->value_packed_size == part && c->slot_size == 2 * part &&
               c->slot_size_aligned == 2 * part && c->n_centroids == 0 && c->norm_correction == 0;
    }
    if (c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256) return false;
    if (c->key_quant_bits != 3 && c->key_quant_bits != 4) return false;
    if (c->value_quant_bits != 3 && c->value_quant_bits != 4) return false;
    const int mse = (c->head_dim * c->key_quant_bits + 7) / 8;
    const int vdb = (c->head_dim * c->value_quant_bits + 7) / 8;
    const int slot = mse + 2 + vdb + 4;
    return c->mse_bytes == mse && c->key_packed_size == mse + 2 && c->val_data_bytes == vdb &&
           c->value_packed_size == vdb + 4 && c->slot_size == slot &&
           c->slot_size_aligned == slot + (slot % 2) && c->n_centroids == (1 << c->key_quant_bits);
}

}  // namespace vmc

extern "C" int vmc_tq_config_from_method(int head_dim, const char* method, vmc_tq_config* out) {
    if (!out || head_dim <= 0 || head_dim > 256) return VMC_EINVAL;
    vmc_tq_config c;
    std::memset(&c, 0, sizeof(c));
    c.head_dim = head_dim;
    c.norm_correction = 1;
    c.max_num_kv_splits = 32;
    const std::string m = method ? method : "";
    if (m == "turboquant_k8v4") {
        // fp8 keys; the reference picks e4b15 below sm_89 (no native fp8), e4m3
        // otherwise -- e4m3 here, fp8_e4b15 may be set by the caller
        c.key_quant_bits = 8;
        c.value_quant_bits = 4;
        c.norm_correction = 0;
        c.key_fp8 = 1;
        c.fp8_e4b15 = 0;
    } else if (m == "turboquant_k3v4_nc") {
        c.key_quant_bits = 3;
        c.value_quant_bits = 4;
    } else if (m == "turboquant_3bit_nc") {
        c.key_quant_bits = 3;
        c.value_quant_bits = 3;
    } else if (m.empty() || m == "turboquant_4bit_nc") {
        c.key_quant_bits = 4;
        c.value_quant_bits = 4;
    } else if ((m == "turboquant_4bit_g32" || m == "turboquant_3bit_g32") && head_dim == 128) {
        // per-32-group variant (no reference counterpart): see vmc_attn.h
        const int b = m == "turboquant_4bit_g32" ? 4 : 3;
        const int part = b == 4 ? 80 : 56;
        c.key_quant_bits = c.value_quant_bits = b;
        c.norm_correction = 0;
        c.n_centroids = 0;
        c.mse_bytes = c.val_data_bytes = 16 * b;
        c.key_packed_size = c.value_packed_size = part;
        c.slot_size = c.slot_size_aligned = 2 * part;
        c.group_size = 32;
        c.sign_seed = 0;
        std::memcpy(out, &c, sizeof(c));  // padding bytes included (zeroed)
        return VMC_OK;
    } else {
        return VMC_EINVAL;
    }
    c.n_centroids = 1 << c.key_quant_bits;
    c.mse_bytes = c.key_fp8 ? head_dim : (head_dim * c.key_quant_bits + 7) / 8;
    c.key_packed_size = c.key_fp8 ? head_dim : c.mse_bytes + 2;
    c.val_data_bytes = (head_dim * c.value_quant_bits + 7) / 8;
    c.value_packed_size = c.val_data_bytes + 4;
    c.slot_size = c.key_packed_size + c.value_packed_size;
    c.slot_size_aligned = c.slot_size + (c.slot_size % 2);
    std::memcpy(out, &c, sizeof(c));
    return VMC_OK;
}

extern "C" int vmc_tq_host_tables(int head_dim, int bits, float* centroids, float* midpoints) {
    if (head_dim <= 0 || (bits != 3 && bits != 4)) return VMC_EINVAL;
    const vmc::TQTables& t = vmc::tq_tables(head_dim, bits);
    const int n = 1 << bits;
    if (centroids) std::memcpy(centroids, t.centroids, sizeof(float) * (size_t)n);
    if (midpoints) std::memcpy(midpoints, t.midpoints, sizeof(float) * (size_t)(n - 1));
    return VMC_OK;
}

extern "C" const char* vmc_version(void) { return "vmc_attn 0.1.0 gfx950"; }
