// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/nexusquant_amd.h"

namespace nq {

// ----------------------------------------------------------------- host ----

void set_error(const char* fmt, ...);

#define NQ_CHECK_ARG(cond, ...)            \
    do {                                   \
        if (!(cond)) {                     \
            ::nq::set_error(__VA_ARGS__);  \
            return NQ_EINVAL;              \
        }                                  \
    } while (0)

// A dispatch's grid size is a 32-bit count of work-items per dimension, so a
// launch of `threads`-wide blocks takes at most this many blocks in one.
constexpr uint64_t max_blocks(uint32_t threads) { return 0xffffffffull / threads; }

#define NQ_CHECK_HIP(expr)                                                   \
    do {                                                                     \
        hipError_t _e = (expr);                                              \
        if (_e != hipSuccess) {                                              \
            ::nq::set_error("%s: %s", #expr, hipGetErrorString(_e));         \
            return NQ_EHIP;                                                  \
        }                                                                    \
    } while (0)

// --------------------------------------------------------------- device ----

// Quad (4-lane) permutes through DPP.  Encoded as quad_perm selectors.
constexpr int kQuadXor1 = 0xB1;  // [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;  // [2,3,0,1]

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __builtin_bit_cast(float, bits16 << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return __half2float(__builtin_bit_cast(__half, (unsigned short)bits16));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(unsigned short, __float2half_rn(f));
}

}  // namespace nq
