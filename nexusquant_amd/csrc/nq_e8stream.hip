// Symbol side of the reference's single-stream E8 container (encode_e8 /
// decode_e8, entropy_coder.py:360-431) on gfx950.  The rANS chain itself is
// nq_rans_encode / nq_rans_decode with one chunk spanning the stream.
//
//   nq_e8_stream_codes   lattice coordinates x = quantized / max(scale, 1e-8)
//                        (IEEE fp32, entropy_coder.py:380-383) as int8 2p codes
//                        clip(rint(2x), -L, L), and the half-integer flag of
//                        _lattice_to_symbols (:58-60): some |x - round(x)| > 0.25,
//                        which is rint(2x) odd, taken before the clip;
//   nq_e8_stream_values  codes back to fp32 values (c / 2) * fp32(scale_f16)
//                        (:418-420 with _symbols_to_lattice :78-86).
// A group of 8 coordinates shares scales[g] (or scales[0] when one scale is
// given, numpy's broadcast of a (1, 1) array).
#include "nq_common.h"

namespace nq {

__global__ __launch_bounds__(256) void e8_stream_codes_kernel(const float* __restrict__ q,
                                                              const float* __restrict__ scales, int64_t n_groups,
                                                              int32_t scale_stride, float lim,
                                                              int8_t* __restrict__ codes, uint32_t* has_half) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    bool odd = false;
    if (g < n_groups) {
        const float4 a = reinterpret_cast<const float4*>(q)[2 * g];
        const float4 b = reinterpret_cast<const float4*>(q)[2 * g + 1];
        const float s = __builtin_fmaxf(scales[g * scale_stride], 1e-8f);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = __builtin_rintf(2.0f * (x[j] / s));
            // integers of magnitude >= 2^24 are all even in fp32
            odd |= __builtin_fabsf(r) < 16777216.0f && ((int32_t)r & 1) != 0;
            const int32_t c = (int32_t)__builtin_fminf(__builtin_fmaxf(r, -lim), lim);
            const uint32_t byte = (uint32_t)(uint8_t)(int8_t)c;
            if (j < 4) lo |= byte << (8 * j);
            else hi |= byte << (8 * (j - 4));
        }
        reinterpret_cast<uint2*>(codes)[g] = make_uint2(lo, hi);
    }
    if (__any(odd) && (threadIdx.x & 63) == __builtin_ffsll(__ballot(odd)) - 1) atomicOr(has_half, 1u);
}

__global__ __launch_bounds__(256) void e8_stream_values_kernel(const int8_t* __restrict__ codes,
                                                               const __fp16* __restrict__ scales, int64_t n_groups,
                                                               int32_t scale_stride, float* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= n_groups) return;
    const uint2 c = reinterpret_cast<const uint2*>(codes)[g];
    const float s = (float)scales[g * scale_stride];
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t w = j < 4 ? c.x : c.y;
        const int8_t code = (int8_t)(uint8_t)(w >> (8 * (j & 3)));
        v[j] = (0.5f * (float)code) * s;
    }
    reinterpret_cast<float4*>(out)[2 * g] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(out)[2 * g + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

static int e8_stream_check(const char* what, const void* a, const void* scales, const void* b, int64_t n_groups,
                           int64_t n_scales) {
    NQ_CHECK_ARG(n_groups >= 0, "%s: negative size", what);
    NQ_CHECK_ARG(n_scales == 1 || n_scales == n_groups,
                 "%s: %lld scales for %lld groups (one per group of 8, or one in all)", what, (long long)n_scales,
                 (long long)n_groups);
    NQ_CHECK_ARG(a && scales && b, "%s: NULL pointer", what);
    NQ_CHECK_ARG(((uintptr_t)a & 7) == 0 && ((uintptr_t)b & 7) == 0, "%s: arrays must be 8-byte aligned", what);
    NQ_CHECK_ARG((n_groups + 255) / 256 < (1ll << 31), "%s: too many groups", what);
    return NQ_OK;
}

}  // namespace nq

extern "C" int nq_e8_stream_codes(const float* quantized, const float* scales, int64_t n_groups, int64_t n_scales,
                                  int32_t levels, int8_t* codes, uint32_t* has_half, void* stream) {
    using namespace nq;
    if (n_groups == 0) return NQ_OK;
    const int st = e8_stream_check("nq_e8_stream_codes", quantized, scales, codes, n_groups, n_scales);
    if (st != NQ_OK) return st;
    NQ_CHECK_ARG(((uintptr_t)quantized & 15) == 0, "nq_e8_stream_codes: quantized must be 16-byte aligned");
    NQ_CHECK_ARG(has_half != nullptr, "nq_e8_stream_codes: NULL has_half");
    NQ_CHECK_ARG(levels == 2 || levels == 4 || levels == 8 || levels == 16,
                 "nq_e8_stream_codes: levels must be 2, 4, 8 or 16 (got %d)", levels);
    hipLaunchKernelGGL(e8_stream_codes_kernel, dim3((uint32_t)((n_groups + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, quantized, scales, n_groups, n_scales == 1 ? 0 : 1, (float)levels, codes,
                       has_half);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_e8_stream_values(const int8_t* codes, const uint16_t* scales_f16, int64_t n_groups,
                                   int64_t n_scales, float* out, void* stream) {
    using namespace nq;
    if (n_groups == 0) return NQ_OK;
    const int st = e8_stream_check("nq_e8_stream_values", codes, scales_f16, out, n_groups, n_scales);
    if (st != NQ_OK) return st;
    NQ_CHECK_ARG(((uintptr_t)out & 15) == 0, "nq_e8_stream_values: out must be 16-byte aligned");
    hipLaunchKernelGGL(e8_stream_values_kernel, dim3((uint32_t)((n_groups + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, codes, reinterpret_cast<const __fp16*>(scales_f16), n_groups,
                       n_scales == 1 ? 0 : 1, out);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
