// Standalone relaxed-E8 primitives of nexusquant.kernels on gfx950:
//
//   nq_e8_nearest_point   the reference's E8 rule on [n, 8] fp32 groups
//                         (E8Lattice.nearest_point, e8_lattice.py:27-69);
//   nq_e8_quantize_perhead  per-row scale amax / (levels / 2), the rule on the
//                         zero-padded 8-groups, clamp to +-levels/2, times the
//                         scale (E8Lattice.quantize_perhead, e8_lattice.py:97-124).
//
// The rule is the one the fused quantizer applies (oracle/nq_spec.c
// nqs_e8_group): integer candidate rint(x), the first smallest-gap coordinate
// stepped one unit toward x when the coordinate sum is odd (+1 on a zero gap);
// half candidate rint(x - 0.5) + 0.5; the half candidate wins when
// sum |x - rint(x)| > 2 (even sum) or > 1 + 2 min |x - rint(x)| (odd sum),
// which is d_half < d_int written without the squares.  Divisions and the
// final product are IEEE fp32 as torch computes them.
#include "nq_common.h"

namespace nq {

// One 8-group in place: the lattice point (before any clamp).
__device__ __forceinline__ void e8_point(float (&x)[8]) {
    float r[8], a[8];
    int parity = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        r[j] = __builtin_rintf(x[j]);
        a[j] = __builtin_fabsf(x[j] - r[j]);
        parity += (int)r[j];
    }
    const bool odd = (parity & 1) != 0;
    int imin = 0;
    float amin = a[0];
#pragma unroll
    for (int j = 1; j < 8; ++j)
        if (a[j] < amin) {
            amin = a[j];
            imin = j;
        }
    const float asum = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    const float thr = odd ? __builtin_fmaf(2.0f, amin, 1.0f) : 2.0f;
    const bool use_half = asum > thr;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float step = (odd && j == imin) ? ((x[j] - r[j] >= 0.0f) ? 1.0f : -1.0f) : 0.0f;
        x[j] = use_half ? __builtin_rintf(x[j] - 0.5f) + 0.5f : r[j] + step;
    }
}

__global__ __launch_bounds__(256) void e8_nearest_kernel(const float* x, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    e8_point(v);
    reinterpret_cast<float4*>(out)[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(out)[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
}

// 16 lanes per row: amax over the row by a 16-lane reduction, then lane k
// takes the 8-groups k, k + 16, ... of the zero-padded row.
__global__ __launch_bounds__(256) void e8_perhead_kernel(const float* x, float* out, int64_t rows, int d,
                                                         float half) {
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int k = threadIdx.x & 15;
    const bool live = row < rows;  // the 16 lanes of a row agree
    const float* xr = x + (live ? row : 0) * d;
    float am = 0.0f;
    if (live)
        for (int j = k; j < d; j += 16) am = __builtin_fmaxf(am, __builtin_fabsf(xr[j]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) am = __builtin_fmaxf(am, __shfl_xor(am, o, 16));
    if (!live) return;
    am = __builtin_fmaxf(am, 1e-8f);          // clamp(min=1e-8)
    const float sc = am / half;               // amax / (levels / 2)
    const int groups = (d + 7) / 8;
    float* outr = out + row * d;
    for (int g = k; g < groups; g += 16) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = 8 * g + j;
            v[j] = c < d ? xr[c] / sc : 0.0f;  // zero padding after the division, as F.pad does
        }
        e8_point(v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = 8 * g + j;
            const float p = __builtin_fminf(__builtin_fmaxf(v[j], -half), half);
            if (c < d) outr[c] = p * sc;
        }
    }
}

}  // namespace nq

extern "C" int nq_e8_nearest_point(const float* x, float* out, int64_t n_groups, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(n_groups >= 0, "nq_e8_nearest_point: negative size");
    if (n_groups == 0) return NQ_OK;
    NQ_CHECK_ARG(x && out, "nq_e8_nearest_point: NULL pointer");
    NQ_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0,
                 "nq_e8_nearest_point: x and out must be 16-byte aligned");
    NQ_CHECK_ARG((n_groups + 255) / 256 < (1ll << 31), "nq_e8_nearest_point: too many groups");
    hipLaunchKernelGGL(e8_nearest_kernel, dim3((uint32_t)((n_groups + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, x, out, n_groups);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_e8_quantize_perhead(const float* x, float* out, int64_t rows, int32_t d, int32_t levels,
                                      void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(rows >= 0 && d > 0, "nq_e8_quantize_perhead: bad geometry (rows %lld, d %d)", (long long)rows, d);
    NQ_CHECK_ARG(levels >= 1, "nq_e8_quantize_perhead: levels must be positive (got %d)", levels);
    if (rows == 0) return NQ_OK;
    NQ_CHECK_ARG(x && out, "nq_e8_quantize_perhead: NULL pointer");
    NQ_CHECK_ARG((rows * 16 + 255) / 256 < (1ll << 31), "nq_e8_quantize_perhead: too many rows");
    hipLaunchKernelGGL(e8_perhead_kernel, dim3((uint32_t)((rows * 16 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, x, out, rows, d, 0.5f * (float)levels);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
