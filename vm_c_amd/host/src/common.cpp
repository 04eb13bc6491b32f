// common.cpp -- error conversion and enum mapping for the vm_c host layer.
#include "vm_c/common.hpp"

#include <string>

namespace vm_c {

void throw_status(int status, const char* what, const char* file, int line) {
    const char* name = status == VMC_EINVAL ? "invalid argument"
                       : status == VMC_ENOMEM ? "workspace too small"
                       : status == VMC_EIO ? "HIP launch/runtime error"
                                           : "error";
    throw std::runtime_error(std::string(file) + ":" + std::to_string(line) + ": " + what +
                             " failed: " + name + " (" + std::to_string(status) + ")");
}

void throw_hip(hipError_t err, const char* what, const char* file, int line) {
    throw std::runtime_error(std::string(file) + ":" + std::to_string(line) + ": " + what +
                             " failed: " + hipGetErrorString(err));
}

int vmc_dtype_of(ScalarType t) {
    if (t == ScalarType::FLOAT16) return VMC_DTYPE_F16;
    if (t == ScalarType::BFLOAT16) return VMC_DTYPE_BF16;
    throw std::runtime_error("attention path: activations must be fp16 or bf16");
}

int vmc_kv_format_of(const std::string& s, ScalarType query_dtype) {
    if (s == "auto" || s.empty()) return vmc_dtype_of(query_dtype) == VMC_DTYPE_BF16 ? VMC_KV_BF16 : VMC_KV_F16;
    if (s == "fp16" || s == "float16" || s == "half") return VMC_KV_F16;
    if (s == "bf16" || s == "bfloat16") return VMC_KV_BF16;
    if (s == "q8_0") return VMC_KV_Q8_0;
    if (s == "q4_0") return VMC_KV_Q4_0;
    throw std::runtime_error("unsupported kv_cache_dtype '" + s + "' (fp16, bf16, q8_0, q4_0, auto)");
}

int vmc_layout_of(const std::string& layout) {
    if (layout.empty() || layout == "nhd") return VMC_LAYOUT_NHD;
    if (layout == "hnd") return VMC_LAYOUT_HND;
    throw std::runtime_error("unsupported kv cache layout '" + layout + "' (nhd, hnd)");
}

}  // namespace vm_c
