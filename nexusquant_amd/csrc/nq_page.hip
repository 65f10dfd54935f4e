// Page codec of the vLLM compressor format (int8 codes 2p, fp16 row scales,
// int32 absolute positions) for gfx950: page decode and nibble packing.
//
// Page decode keeps the quantizer's quad-per-row layout (lane q of a quad owns
// chunks of 8 coordinates 32c + 8q .. +7).  The integer codes become exact
// fp16 values, the inverse Walsh-Hadamard runs on them in packed fp16 (every
// partial sum is an integer of magnitude <= 16 * D / 2 <= 2048, exact in fp16),
// and each coordinate is scaled once by fl(fl(scale / 2) * h_D); keys leave the
// top butterfly stage to the merged step with forward RoPE at the stored
// position.  oracle/nq_spec.c (nqs_page_decode) restates this order.
#include <algorithm>
#include "nq_rowmath.h"

namespace nq {

struct PageArgs {
    const uint64_t* codes;
    const uint64_t* scales;
    const uint64_t* positions;
    const uint64_t* out;
    const float* rope_cos;
    const float* rope_sin;
    const float* rope_dm;
    const float* rope_dp;
    uint32_t rows;   // heads * tokens per page
    uint32_t tokens;
    uint32_t tiles;  // ceil(rows / 64)
    uint32_t rope_n_pos;
    float hscale;
};

// Four int8 codes (one dword) -> two fp16 pairs, exactly.  XOR 0x80 biases
// the byte to c + 128; v_perm places it under the fp16 exponent of 1024
// (0x64 high byte), giving 1024 + c + 128, and one packed add removes 1152.
__device__ __forceinline__ void codes_to_f16(uint32_t w, half2v& lo, half2v& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const half2v bias = {(__fp16)-1152.0f, (__fp16)-1152.0f};
    lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(u, 0x64646464u, 0x00050004u)) + bias;
    hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(u, 0x64646464u, 0x00070006u)) + bias;
}

template <int D>
__device__ __forceinline__ uint32_t page_position(const PageArgs& a, uint32_t page, uint32_t row) {
    const int32_t p = reinterpret_cast<const int32_t*>(a.positions[page])[row % a.tokens];
    // the host validates positions against the table; clamp so none reads outside it
    return p < 0 ? 0u : ((uint32_t)p >= a.rope_n_pos ? a.rope_n_pos - 1u : (uint32_t)p);
}

template <int D, bool IS_KEY>
__global__ __launch_bounds__(256) void page_decode_kernel(PageArgs a) {
    constexpr int C = D / 32;
    const int q = threadIdx.x & 3;
    const uint32_t page = blockIdx.x / a.tiles;
    const uint32_t row_raw = (blockIdx.x % a.tiles) * 64u + (threadIdx.x >> 2);
    const bool active = row_raw < a.rows;
    const uint32_t row = active ? row_raw : a.rows - 1u;  // idle quads recompute a valid row

    const int8_t* crow = reinterpret_cast<const int8_t*>(a.codes[page]) + (size_t)row * D;
    half2v h[C][4];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint2 w = *reinterpret_cast<const uint2*>(crow + 32 * c + 8 * q);
        codes_to_f16(w.x, h[c][0], h[c][1]);
        codes_to_f16(w.y, h[c][2], h[c][3]);
    }
    const float sc = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.scales[page])[row]);
    const float g = quad_sign(q) * ((0.5f * sc) * a.hscale);  // sign of the quad stages folded in

    fwht_row_f16<C, !IS_KEY>(h, q);
    float x[C][8];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[c][2 * k] = __builtin_fmaf((float)h[c][k].x, g, 0.0f);
            x[c][2 * k + 1] = __builtin_fmaf((float)h[c][k].y, g, 0.0f);
        }
    if constexpr (IS_KEY) {
        float dm[C / 2][8], dp[C / 2][8];
        load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, page_position<D>(a, page, row), q, dm, dp);
        rope_stage_merged<C>(x, dm, dp);
    }
    if (!active) return;
    // fp32 first, then fp16 (the empty asm keeps the backend from fusing the
    // last fma with the conversion into a single rounding)
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) asm("" : "+v"(x[c][i]));
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out[page]) + (size_t)row * D;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        half2v o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = half2v{(__fp16)x[c][2 * k], (__fp16)x[c][2 * k + 1]};
        uint4 w;
        w.x = __builtin_bit_cast(uint32_t, o[0]);
        w.y = __builtin_bit_cast(uint32_t, o[1]);
        w.z = __builtin_bit_cast(uint32_t, o[2]);
        w.w = __builtin_bit_cast(uint32_t, o[3]);
        *reinterpret_cast<uint4*>(orow + 32 * c + 8 * q) = w;
    }
}

// Logits of queries against one page's fp32 keys (the decoded keys before the
// fp16 rounding): logits[h, i, t] = (q[h, i] . k[h, t]) / scale_divisor.
template <int D, int QDT>
__global__ __launch_bounds__(256) void page_logits_kernel(PageArgs a, const void* query, uint32_t q_len,
                                                          float scale_divisor, float* logits) {
    constexpr int C = D / 32;
    const int q = threadIdx.x & 3;
    const uint32_t row_raw = blockIdx.x * 64u + (threadIdx.x >> 2);
    const bool active = row_raw < a.rows;
    const uint32_t row = active ? row_raw : a.rows - 1u;
    const int8_t* crow = reinterpret_cast<const int8_t*>(a.codes[0]) + (size_t)row * D;
    half2v h[C][4];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint2 w = *reinterpret_cast<const uint2*>(crow + 32 * c + 8 * q);
        codes_to_f16(w.x, h[c][0], h[c][1]);
        codes_to_f16(w.y, h[c][2], h[c][3]);
    }
    const float sc = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.scales[0])[row]);
    const float g = quad_sign(q) * ((0.5f * sc) * a.hscale);
    fwht_row_f16<C, false>(h, q);
    float x[C][8];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[c][2 * k] = __builtin_fmaf((float)h[c][k].x, g, 0.0f);
            x[c][2 * k + 1] = __builtin_fmaf((float)h[c][k].y, g, 0.0f);
        }
    float dm[C / 2][8], dp[C / 2][8];
    load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, page_position<D>(a, 0, row), q, dm, dp);
    rope_stage_merged<C>(x, dm, dp);

    const uint32_t head = row / a.tokens, t = row % a.tokens;
    for (uint32_t i = 0; i < q_len; ++i) {
        const size_t qb = ((size_t)head * q_len + i) * D;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float qv[8];
            load8<QDT>(query, (int64_t)(qb + 32 * c + 8 * q), qv);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(qv[j], x[c][j], acc);
        }
        acc += dpp_f32<kQuadXor1>(acc);
        acc += dpp_f32<kQuadXor2>(acc);
        if (active && q == 0) logits[((size_t)head * q_len + i) * a.tokens + t] = acc / scale_divisor;
    }
}

// ------------------------------------------------------------ nibbles ----

__device__ __forceinline__ uint32_t nibble_of(int8_t c) {
    const int v = (int)c + 8;
    return (uint32_t)(v < 0 ? 0 : (v > 15 ? 15 : v));
}

// Both nibble kernels stride over the grid, which the host caps at
// kNibbleBlocks blocks: inputs of more than 2^32 elements need no wider grid.
constexpr int64_t kNibbleBlocks = 1 << 20;

__global__ __launch_bounds__(256) void nibble_pack_kernel(const int8_t* codes, int64_t rows, int32_t d,
                                                          uint8_t* packed) {
    const int32_t pd = (d + 1) / 2;
    const int64_t n = rows * pd;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / pd;
        const int32_t j = (int32_t)(i - r * pd);
        const int8_t* row = codes + r * d;
        const uint32_t lo = nibble_of(row[2 * j]);
        const uint32_t hi = 2 * j + 1 < d ? nibble_of(row[2 * j + 1]) : 0u;  // the pad nibble is 0
        packed[i] = (uint8_t)(lo | (hi << 4));
    }
}

__global__ __launch_bounds__(256) void nibble_unpack_kernel(const uint8_t* packed, int64_t rows, int32_t pd,
                                                            int32_t d, int8_t* codes) {
    const int64_t n = rows * d;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / d;
        const int32_t k = (int32_t)(i - r * d);
        const uint32_t b = packed[r * pd + k / 2];
        codes[i] = (int8_t)((int)((k & 1) ? (b >> 4) : (b & 15u)) - 8);
    }
}

template <int D>
static hipError_t launch_page_decode(bool key, const PageArgs& a, uint32_t n_pages, hipStream_t s) {
    const dim3 grid(n_pages * a.tiles);
    if (key) hipLaunchKernelGGL((page_decode_kernel<D, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((page_decode_kernel<D, false>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace nq

extern "C" int nq_page_decode(const nq_page_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_page_decode: desc is NULL");
    NQ_CHECK_ARG(d->n_pages >= 0 && d->n_pages <= 65535, "nq_page_decode: n_pages %d out of range", d->n_pages);
    if (d->n_pages == 0) return NQ_OK;
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_page_decode: head_dim %d unsupported (64, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->heads > 0 && d->tokens >= 0, "nq_page_decode: bad geometry");
    NQ_CHECK_ARG(d->codes && d->scales && d->out, "nq_page_decode: codes, scales and out are required");
    const uint64_t rows = (uint64_t)d->heads * d->tokens;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq_page_decode: %llu rows per page exceeds 2^31",
                 (unsigned long long)rows);
    if (rows == 0) return NQ_OK;
    NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                 "nq_page_decode: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
    if (d->is_key) {
        NQ_CHECK_ARG(d->positions != nullptr, "nq_page_decode: keys need positions");
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin && d->rope_n_pos > 0 && d->rope_n_pos < (1ll << 31),
                     "nq_page_decode: keys need RoPE tables");
    }
    const uint64_t tiles = (rows + 63) / 64;
    NQ_CHECK_ARG(tiles * (uint64_t)d->n_pages <= max_blocks(256), "nq_page_decode: grid too large");
    PageArgs a = {};
    a.codes = d->codes;
    a.scales = d->scales;
    a.positions = d->positions;
    a.out = d->out;
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.rows = (uint32_t)rows;
    a.tokens = (uint32_t)d->tokens;
    a.tiles = (uint32_t)tiles;
    a.rope_n_pos = (uint32_t)(d->is_key ? d->rope_n_pos : 1);
    a.hscale = d->hadamard_scale;
    hipStream_t s = (hipStream_t)stream;
    const bool key = d->is_key != 0;
    hipError_t e;
    switch (d->head_dim) {
        case 64: e = launch_page_decode<64>(key, a, (uint32_t)d->n_pages, s); break;
        case 128: e = launch_page_decode<128>(key, a, (uint32_t)d->n_pages, s); break;
        default: e = launch_page_decode<256>(key, a, (uint32_t)d->n_pages, s); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

extern "C" int nq_page_logits(const nq_page_desc* d, const void* query, int32_t q_dtype, int32_t q_len,
                              float scale_divisor, float* logits, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_page_logits: desc is NULL");
    NQ_CHECK_ARG(d->n_pages == 1, "nq_page_logits: one page per call (got %d)", d->n_pages);
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_page_logits: head_dim %d unsupported (64, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(q_dtype == NQ_F16 || q_dtype == NQ_BF16 || q_dtype == NQ_F32,
                 "nq_page_logits: unknown query dtype %d", q_dtype);
    NQ_CHECK_ARG(d->heads > 0 && d->tokens >= 0 && q_len >= 0, "nq_page_logits: bad geometry");
    const uint64_t rows = (uint64_t)d->heads * d->tokens;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq_page_logits: too many rows");
    if (rows == 0 || q_len == 0) return NQ_OK;
    NQ_CHECK_ARG(d->codes && d->scales && d->positions && query && logits,
                 "nq_page_logits: codes, scales, positions, query and logits are required");
    NQ_CHECK_ARG(d->rope_cos && d->rope_sin && d->rope_n_pos > 0 && d->rope_n_pos < (1ll << 31),
                 "nq_page_logits: keys need RoPE tables");
    NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                 "nq_page_logits: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
    PageArgs a = {};
    a.codes = d->codes;
    a.scales = d->scales;
    a.positions = d->positions;
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.rows = (uint32_t)rows;
    a.tokens = (uint32_t)d->tokens;
    a.tiles = (uint32_t)((rows + 63) / 64);
    a.rope_n_pos = (uint32_t)d->rope_n_pos;
    a.hscale = d->hadamard_scale;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(a.tiles);
#define NQ_LOGITS(DIM, QT) \
    hipLaunchKernelGGL((page_logits_kernel<DIM, QT>), grid, dim3(256), 0, s, a, query, (uint32_t)q_len, scale_divisor, logits)
#define NQ_LOGITS_DT(DIM)                                              \
    do {                                                               \
        if (q_dtype == NQ_F16) NQ_LOGITS(DIM, NQ_F16);                 \
        else if (q_dtype == NQ_BF16) NQ_LOGITS(DIM, NQ_BF16);          \
        else NQ_LOGITS(DIM, NQ_F32);                                   \
    } while (0)
    switch (d->head_dim) {
        case 64: NQ_LOGITS_DT(64); break;
        case 128: NQ_LOGITS_DT(128); break;
        default: NQ_LOGITS_DT(256); break;
    }
#undef NQ_LOGITS_DT
#undef NQ_LOGITS
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_nibble_pack(const int8_t* codes, int64_t rows, int32_t d, uint8_t* packed, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(rows >= 0 && rows <= (1ll << 40) && d > 0, "nq_nibble_pack: bad geometry");
    const int64_t n = rows * ((d + 1) / 2);
    if (n == 0) return NQ_OK;
    NQ_CHECK_ARG(codes && packed, "nq_nibble_pack: NULL pointer");
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, kNibbleBlocks);
    hipLaunchKernelGGL(nibble_pack_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, codes, rows, d,
                       packed);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_nibble_unpack(const uint8_t* packed, int64_t rows, int32_t packed_cols, int32_t d, int8_t* codes,
                                void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(rows >= 0 && rows <= (1ll << 40) && d > 0 && packed_cols > 0 && d <= 2 * (int64_t)packed_cols,
                 "nq_nibble_unpack: bad geometry (d %d, packed_cols %d)", d, packed_cols);
    const int64_t n = rows * d;
    if (n == 0) return NQ_OK;
    NQ_CHECK_ARG(codes && packed, "nq_nibble_unpack: NULL pointer");
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, kNibbleBlocks);
    hipLaunchKernelGGL(nibble_unpack_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, packed, rows,
                       packed_cols, d, codes);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
