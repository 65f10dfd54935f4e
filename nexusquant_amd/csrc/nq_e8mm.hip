// Fused dequantize + matrix product over the standalone E8 code format
// (int8 codes [K, H_pad], one fp32 scale per row):
//
//     out[k, j] = sum_{h < H} (codes[k, h] * scales[k]) * query[h, j]
//
// (nexusquant/kernels/e8_triton.py:373-444, 613-660), without materialising
// the decoded [K, H] tensor.
//
// gfx950 layout: 16x16x32 bf16 MFMAs with the codes as the A operand (16 rows
// of K x 32 of H) and the query as B (32 of H x 16 columns).  An int8 code is
// exact in bf16 (|c| <= 128 needs 8 significant bits); the fp32 query is split
// into three bf16 parts hi + mid + lo that carry its 24 significant bits, so
// every product is exact and the three MFMAs accumulate sum_h c * q in fp32.
// The row's scale multiplies the sum once at the end.  A workgroup holds one
// 16-column tile of the query in registers (3 parts per 32-row K step) and
// its four waves stream 16-row tiles of codes.
#include "nq_rowmath.h"

namespace nq {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

struct DmmArgs {
    const int8_t* codes;
    const float* scales;
    const float* query;
    float* out;
    int64_t k_rows;
    int32_t h_pad, h, q_cols;
    uint32_t row_tiles;  // ceil(k_rows / 16)
};

constexpr int kTiles = 2;  // 16-row tiles per wave and round: 2 is 4 % faster than 1 on codes read from HBM, 4 is slower
constexpr uint32_t kMaxBlocks = 1024;  // row blocks per column tile: each wave streams ~16 tiles

// K slot s of lane group kq in K step ks is column h(ks, kq, s): with V16,
// 64 (ks / 2) + 16 kq + 8 (ks % 2) + s, so a lane's two K steps of a pair read
// 16 consecutive code bytes in one load (H_pad a multiple of 16, an even
// number of steps); else 32 ks + 8 kq + s, 8 bytes per step.
template <bool V16>
__device__ __forceinline__ int kcol(int ks, int kq, int s) {
    return V16 ? 64 * (ks >> 1) + 16 * kq + 8 * (ks & 1) + s : 32 * ks + 8 * kq + s;
}

template <int KS, bool V16>
__global__ __launch_bounds__(256) void e8_dequant_matmul_kernel(DmmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, kq = lane >> 4;
    const int col = (int)blockIdx.y * 16 + n;
    const bool col_ok = col < a.q_cols;

    // B operands: lane l holds query rows kcol(ks, kq, 0 .. 7) of column col,
    // as three bf16 parts (rows >= H and columns >= Q_cols are zero)
    bf16x8v qb[KS][3];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int h = kcol<V16>(ks, kq, s);
            const float x = (h < a.h && col_ok) ? a.query[(size_t)h * a.q_cols + col] : 0.0f;
            const __bf16 p0 = (__bf16)x;
            const float r1 = x - (float)p0;
            const __bf16 p1 = (__bf16)r1;
            const __bf16 p2 = (__bf16)(r1 - (float)p1);
            qb[ks][0][s] = p0;
            qb[ks][1][s] = p1;
            qb[ks][2][s] = p2;
        }

    // bytes of this lane's code words that are padding (columns >= H) are
    // cleared before conversion
    uint2 keep[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int h0 = kcol<V16>(ks, kq, 0);
        uint32_t m[2] = {0u, 0u};
#pragma unroll
        for (int b = 0; b < 8; ++b)
            if (h0 + b < a.h) m[b >> 2] |= 0xffu << (8 * (b & 3));
        keep[ks] = make_uint2(m[0], m[1]);
    }

    // each wave takes kTiles consecutive 16-row tiles per round, all their code
    // and scale loads issued before the first is used
    for (uint32_t t0 = (blockIdx.x * 4u + (uint32_t)wave) * kTiles; t0 < a.row_tiles; t0 += gridDim.x * 4u * kTiles) {
        uint2 w[kTiles][KS];
        float sc[kTiles][4];
#pragma unroll
        for (int u = 0; u < kTiles; ++u) {
            const int64_t row = (int64_t)(t0 + u) * 16 + n;  // A row of this lane
            const bool row_ok = row < a.k_rows;
            if constexpr (V16) {
#pragma unroll
                for (int ks = 0; ks < KS; ks += 2) {
                    const int h0 = kcol<true>(ks, kq, 0);  // 16 bytes: steps ks and ks + 1
                    uint4 v = make_uint4(0u, 0u, 0u, 0u);
                    if (row_ok && h0 < a.h_pad) v = *reinterpret_cast<const uint4*>(a.codes + row * a.h_pad + h0);
                    w[u][ks] = make_uint2(v.x, v.y);
                    if (ks + 1 < KS) w[u][ks + 1] = make_uint2(v.z, v.w);
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int h0 = kcol<false>(ks, kq, 0);
                    w[u][ks] = make_uint2(0u, 0u);
                    if (row_ok && h0 < a.h_pad) w[u][ks] = *reinterpret_cast<const uint2*>(a.codes + row * a.h_pad + h0);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t rr = (int64_t)(t0 + u) * 16 + 4 * kq + i;
                sc[u][i] = rr < a.k_rows ? a.scales[rr] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < kTiles; ++u) {
            const int64_t r0 = (int64_t)(t0 + u) * 16;
            f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                // int8 -> exact bf16: c + 128 under the fp32 exponent of 2^23
                // (v_perm), minus 2^23 + 128, then the high half of the fp32
                const uint32_t x[2] = {(w[u][ks].x & keep[ks].x) ^ 0x80808080u, (w[u][ks].y & keep[ks].y) ^ 0x80808080u};
                bf16x8v av;
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const uint32_t bits = __builtin_amdgcn_perm(x[b >> 2], 0x4b000000u, 0x03010004u + (uint32_t)(b & 3));
                    av[b] = (__bf16)(__builtin_bit_cast(float, bits) - 8388736.0f);
                }
#pragma unroll
                for (int p = 0; p < 3; ++p) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, qb[ks][p], acc, 0, 0, 0);
            }
            // lane l holds rows r0 + 4 kq + i of column col
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t rr = r0 + 4 * kq + i;
                if (rr < a.k_rows && col_ok) a.out[rr * a.q_cols + col] = acc[i] * sc[u][i];
            }
        }
    }
}

template <int KS>
static void launch_e8mm(bool v16, dim3 grid, hipStream_t s, const DmmArgs& a) {
    if constexpr (KS % 2 == 0) {
        if (v16) {
            hipLaunchKernelGGL((e8_dequant_matmul_kernel<KS, true>), grid, dim3(256), 0, s, a);
            return;
        }
    }
    hipLaunchKernelGGL((e8_dequant_matmul_kernel<KS, false>), grid, dim3(256), 0, s, a);
}

}  // namespace nq

extern "C" int nq_e8_dequant_matmul(const int8_t* codes, const float* scales, const float* query, float* out,
                                    int64_t k_rows, int32_t h_pad, int32_t h, int32_t q_cols, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(k_rows >= 0 && q_cols >= 0, "nq_e8_dequant_matmul: negative size");
    NQ_CHECK_ARG(h > 0 && h_pad >= h && h_pad % 8 == 0,
                 "nq_e8_dequant_matmul: need 0 < H <= H_pad and H_pad a multiple of 8 (H %d, H_pad %d)", h, h_pad);
    NQ_CHECK_ARG(h_pad <= 256, "nq_e8_dequant_matmul: H_pad %d above 256", h_pad);
    if (k_rows == 0 || q_cols == 0) return NQ_OK;
    NQ_CHECK_ARG(codes && scales && query && out, "nq_e8_dequant_matmul: NULL pointer");
    NQ_CHECK_ARG(((uintptr_t)codes & 7) == 0, "nq_e8_dequant_matmul: codes must be 8-byte aligned");
    const int64_t tiles = (k_rows + 15) / 16;
    NQ_CHECK_ARG(tiles < (1ll << 31), "nq_e8_dequant_matmul: too many rows");
    DmmArgs a;
    a.codes = codes;
    a.scales = scales;
    a.query = query;
    a.out = out;
    a.k_rows = k_rows;
    a.h_pad = h_pad;
    a.h = h;
    a.q_cols = q_cols;
    a.row_tiles = (uint32_t)tiles;
    const uint32_t col_tiles = (uint32_t)((q_cols + 15) / 16);
    NQ_CHECK_ARG(col_tiles <= 65535u, "nq_e8_dequant_matmul: Q_cols %d too large", q_cols);
    // a bounded grid whose waves loop over row tiles: the query split in the
    // prologue is paid once per ~16 tiles (8192 blocks of 2 tiles ran 25 %
    // slower)
    uint32_t row_blocks = (uint32_t)((tiles + 4 * kTiles - 1) / (4 * kTiles));
    const uint32_t cap = kMaxBlocks / col_tiles > 0 ? kMaxBlocks / col_tiles : 1u;
    if (row_blocks > cap) row_blocks = cap;
    const dim3 grid(row_blocks, col_tiles);
    int ks = (h + 31) / 32;
    // 16-byte code loads when every row starts 16-byte aligned; their K steps
    // come in pairs, so the count rounds up to even (columns >= H are masked)
    const bool v16 = h_pad % 16 == 0 && ((uintptr_t)codes & 15) == 0;
    if (v16) ks = (ks + 1) & ~1;
    hipStream_t s = (hipStream_t)stream;
    switch (ks) {
        case 1: launch_e8mm<1>(false, grid, s, a); break;
        case 2: launch_e8mm<2>(v16, grid, s, a); break;
        case 3: launch_e8mm<3>(false, grid, s, a); break;
        case 4: launch_e8mm<4>(v16, grid, s, a); break;
        case 5: launch_e8mm<5>(false, grid, s, a); break;
        case 6: launch_e8mm<6>(v16, grid, s, a); break;
        case 7: launch_e8mm<7>(false, grid, s, a); break;
        default: launch_e8mm<8>(v16, grid, s, a); break;
    }
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
