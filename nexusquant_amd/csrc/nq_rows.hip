// Row passthrough for layers kept at fp16 (boundary / explicitly protected
// layers): gather kept rows (truncation) or zero evicted rows (mask eviction),
// converting to fp16 with round-to-nearest-even.
// Reference: NexusQuantEvict.compress skip branch, pipeline.py:1204-1210;
// NexusQuantEvictTruncate.compress skip branch, pipeline.py:1359-1368.
// One thread writes 8 fp16 (16 bytes); rows are contiguous head_dim vectors.
#include "nq_common.h"

namespace nq {

struct RowsArgs {
    const uint64_t* src;
    const uint64_t* dst;
    const int32_t* gather;  // [batch, seq_out] or NULL
    const uint8_t* keep;    // [batch, seq_in] or NULL
    uint32_t heads, seq_in, seq_out, d, chunks_per_row;  // chunks of 8 elements
    uint64_t chunks;        // total chunks per tensor
};

template <int DT>
__global__ __launch_bounds__(256) void gather_rows_kernel(RowsArgs a) {
    const uint64_t c = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (c >= a.chunks) return;
    const uint32_t tensor = blockIdx.y;
    const uint64_t row = c / a.chunks_per_row;
    const uint32_t part = (uint32_t)(c - row * a.chunks_per_row);
    const uint32_t bh = (uint32_t)(row / a.seq_out);
    const uint32_t t_out = (uint32_t)(row - (uint64_t)bh * a.seq_out);
    const uint32_t b = bh / a.heads;
    uint32_t t_in = t_out;
    if (a.gather) {
        const int32_t gi = a.gather[(size_t)b * a.seq_out + t_out];
        t_in = gi < 0 ? 0u : ((uint32_t)gi >= a.seq_in ? a.seq_in - 1u : (uint32_t)gi);
    }
    const bool keep = a.keep ? a.keep[(size_t)b * a.seq_in + t_in] != 0 : true;
    const size_t in_off = ((size_t)bh * a.seq_in + t_in) * a.d + (size_t)part * 8;
    const size_t out_off = ((size_t)bh * a.seq_out + t_out) * a.d + (size_t)part * 8;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (keep) {
        if constexpr (DT == NQ_F16) {
            w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.src[tensor]) + in_off);
        } else {
            float v[8];
            if constexpr (DT == NQ_BF16) {
                uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.src[tensor]) + in_off);
                uint32_t rs[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[2 * k] = __builtin_bit_cast(float, rs[k] << 16);
                    v[2 * k + 1] = __builtin_bit_cast(float, rs[k] & 0xffff0000u);
                }
            } else {
                const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.src[tensor]) + in_off);
                float4 x0 = p[0], x1 = p[1];
                v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
                v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
            }
            w.x = f32_to_f16_bits(v[0]) | (f32_to_f16_bits(v[1]) << 16);
            w.y = f32_to_f16_bits(v[2]) | (f32_to_f16_bits(v[3]) << 16);
            w.z = f32_to_f16_bits(v[4]) | (f32_to_f16_bits(v[5]) << 16);
            w.w = f32_to_f16_bits(v[6]) | (f32_to_f16_bits(v[7]) << 16);
        }
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.dst[tensor]) + out_off) = w;
}

}  // namespace nq

extern "C" int nq_gather_rows(const uint64_t* src, const uint64_t* dst, int32_t n_tensors, int32_t dtype,
                              int32_t batch, int32_t heads, int32_t seq_in, int32_t seq_out, int32_t head_dim,
                              const int32_t* gather, const uint8_t* keep, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(src && dst, "nq_gather_rows: NULL pointer array");
    NQ_CHECK_ARG(n_tensors >= 0 && n_tensors <= 65535, "nq_gather_rows: n_tensors out of range");
    NQ_CHECK_ARG(head_dim > 0 && head_dim % 8 == 0, "nq_gather_rows: head_dim must be a multiple of 8");
    NQ_CHECK_ARG(dtype == NQ_F16 || dtype == NQ_BF16 || dtype == NQ_F32, "nq_gather_rows: bad dtype");
    NQ_CHECK_ARG(batch > 0 && heads > 0 && seq_in >= 0 && seq_out >= 0, "nq_gather_rows: bad shape");
    NQ_CHECK_ARG(gather || seq_in == seq_out, "nq_gather_rows: seq_out must equal seq_in without gather");
    if (n_tensors == 0 || seq_out == 0) return NQ_OK;
    RowsArgs a;
    a.src = src;
    a.dst = dst;
    a.gather = gather;
    a.keep = keep;
    a.heads = (uint32_t)heads;
    a.seq_in = (uint32_t)seq_in;
    a.seq_out = (uint32_t)seq_out;
    a.d = (uint32_t)head_dim;
    a.chunks_per_row = (uint32_t)(head_dim / 8);
    a.chunks = (uint64_t)batch * heads * seq_out * a.chunks_per_row;
    NQ_CHECK_ARG((a.chunks + 255) / 256 <= max_blocks(256), "nq_gather_rows: tensor too large");
    dim3 grid((uint32_t)((a.chunks + 255) / 256), (uint32_t)n_tensors);
    hipStream_t s = (hipStream_t)stream;
    switch (dtype) {
        case NQ_F16: hipLaunchKernelGGL(gather_rows_kernel<NQ_F16>, grid, dim3(256), 0, s, a); break;
        case NQ_BF16: hipLaunchKernelGGL(gather_rows_kernel<NQ_BF16>, grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(gather_rows_kernel<NQ_F32>, grid, dim3(256), 0, s, a); break;
    }
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
