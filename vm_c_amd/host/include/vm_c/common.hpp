// vm_c/common.hpp -- shared host-side types of the vm_c attention API on HIP.
//
// ScalarType mirrors vm_c's DataType enum (include/vm_c/core/tensor.hpp:18-51);
// only the element types the attention path carries are used here.  Errors
// follow vm_c's convention (CUDA_CHECK, include/vm_c/cuda/gpu_arch.hpp:53-72):
// a failed call throws std::runtime_error naming the call site.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "vmc_attn.h"

namespace vm_c {

enum class DataType {
    FLOAT32 = 0,
    FLOAT16 = 1,
    BFLOAT16 = 2,
    FLOAT8_E4M3 = 3,
    FLOAT8_E5M2 = 4,
    INT8 = 5,
    INT32 = 6,
    INT64 = 7,
    UINT8 = 8,
};
using ScalarType = DataType;

inline size_t dtype_size(DataType t) {
    switch (t) {
        case DataType::FLOAT32:
        case DataType::INT32: return 4;
        case DataType::FLOAT16:
        case DataType::BFLOAT16: return 2;
        case DataType::INT64: return 8;
        default: return 1;
    }
}

[[noreturn]] void throw_status(int status, const char* what, const char* file, int line);
[[noreturn]] void throw_hip(hipError_t err, const char* what, const char* file, int line);

// the C ABI's element-type code of a ScalarType (throws for other types)
int vmc_dtype_of(ScalarType t);
// "fp16"/"bf16"/"auto"/"q8_0"/"q4_0" -> VMC_KV_*; "auto" takes the query type
int vmc_kv_format_of(const std::string& kv_cache_dtype, ScalarType query_dtype);
// "nhd"/"hnd" -> VMC_LAYOUT_*
int vmc_layout_of(const std::string& layout);

}  // namespace vm_c

#define VMC_CALL(expr)                                                        \
    do {                                                                      \
        const int rc_ = (expr);                                               \
        if (rc_ != VMC_OK) ::vm_c::throw_status(rc_, #expr, __FILE__, __LINE__); \
    } while (0)

#define HIP_CHECK(expr)                                                       \
    do {                                                                      \
        const hipError_t e_ = (expr);                                         \
        if (e_ != hipSuccess) ::vm_c::throw_hip(e_, #expr, __FILE__, __LINE__); \
    } while (0)
