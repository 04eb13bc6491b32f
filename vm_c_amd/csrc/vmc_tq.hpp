// vmc_tq.hpp -- TurboQuant constants shared by the store and decode kernels.
#pragma once

#include "vmc_attn.h"

namespace vmc {

// Passed to kernels by value (kernel-argument segment, scalar loads).
struct TQTables {
    float centroids[16];  // Lloyd-Max centroids for N(0, 1/d), ascending
    float midpoints[16];  // (c[i] + c[i+1]) / 2, n_centroids - 1 used
    int n_centroids;
    float rot_c;  // 1.0f / sqrtf(d): the scale of the reference Hadamard matrix
};

const TQTables& tq_tables(int head_dim, int bits);
bool tq_config_valid(const vmc_tq_config* c);

// Rotation signs of the per-32-group variant: bit i of the 128 (word i / 32)
// set = sign of dim i is -1; bit i % 64 of the splitmix64-mixed words
// (seed, stream 0x5349474e, i / 64); seed 0: all +1.
struct G32Signs {
    uint32_t w[4];
};
G32Signs g32_signs(unsigned long long seed);

}  // namespace vmc
