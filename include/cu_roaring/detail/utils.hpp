// Error helpers -- counterpart of include/cu_roaring/detail/utils.cuh:9-23.
// Library calls report failures by throwing std::runtime_error with the
// C-ABI's message (the reference's CUDA_CHECK contract).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "cu_roaring_abi.h"

namespace cu_roaring {

#define CU_ROARING_HIP_CHECK(call)                                                              \
    do {                                                                                        \
        hipError_t err__ = (call);                                                              \
        if (err__ != hipSuccess) {                                                              \
            throw std::runtime_error(std::string("HIP error at ") + __FILE__ + ":" +            \
                                     std::to_string(__LINE__) + ": " + hipGetErrorString(err__)); \
        }                                                                                       \
    } while (0)

inline void throw_on_error(int rc, const char* what)
{
    if (rc != CR_OK) throw std::runtime_error(std::string(what) + ": " + cr_last_error());
}

inline constexpr uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

}  // namespace cu_roaring
