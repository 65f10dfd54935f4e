// Packed-code kernels for gfx950: dequantize to the fp16 reconstruction,
// convert to int8 2p codes (the reference's vLLM page format,
// vllm_backend.py:267-338), the temporal delta stream of those codes
// (compression_accounting.py:49-62) and its inverse (:70-77).
//
// Rows use the quantizer's quad layout (lane q owns chunks c of coordinates
// 32c + 8q .. +7; its symbol slots are the q-th run of C slots of the row), so
// dequantization repeats the quantizer's reconstruction arithmetic exactly.
#include "nq_rowmath.h"

namespace nq {

struct CodecArgs {
    const uint64_t* syms;
    const uint64_t* cosets;
    const uint64_t* scales;
    const uint64_t* out;
    const float* rope_cos;
    const float* rope_sin;
    const float* rope_dm;
    const float* rope_dp;
    uint32_t heads, seq, n_tensors, bh, work, per_xcd;
    float hscale;
};

// Lattice points of this lane's C groups from the packed row.
template <int D, int L>
__device__ __forceinline__ void unpack_points(const CodecArgs& a, uint32_t tensor, size_t row, int q,
                                             float (&p)[D / 32][8], int (&coset)[D / 32], float& scale) {
    constexpr int C = D / 32;
    constexpr int B = SymBits<L>::value;
    constexpr int NB = C * B;
    constexpr int HL = L / 2;
    constexpr int ROW_BYTES = D / 8 * B;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.syms[tensor]) + row * ROW_BYTES + q * NB;
    uint8_t bytes[NB];
    if constexpr (NB % 4 == 0) {
#pragma unroll
        for (int k = 0; k < NB; k += 4) {
            uint32_t w = *reinterpret_cast<const uint32_t*>(src + k);
            bytes[k] = (uint8_t)w;
            bytes[k + 1] = (uint8_t)(w >> 8);
            bytes[k + 2] = (uint8_t)(w >> 16);
            bytes[k + 3] = (uint8_t)(w >> 24);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NB; k += 2) {
            uint16_t w = *reinterpret_cast<const uint16_t*>(src + k);
            bytes[k] = (uint8_t)w;
            bytes[k + 1] = (uint8_t)(w >> 8);
        }
    }
    const uint8_t* cb = reinterpret_cast<const uint8_t*>(a.cosets[tensor]) + row * (D / 64);
    uint32_t cbits;
    if constexpr (D == 64) cbits = *cb;
    else if constexpr (D == 128) cbits = *reinterpret_cast<const uint16_t*>(cb);
    else cbits = *reinterpret_cast<const uint32_t*>(cb);
    scale = reinterpret_cast<const float*>(a.scales[tensor])[row];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        uint64_t v = 0;
#pragma unroll
        for (int m = 0; m < B; ++m) v |= (uint64_t)bytes[c * B + m] << (8 * m);
        coset[c] = (int)((cbits >> (4 * c + q)) & 1u);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int sym = (int)((v >> (B * j)) & ((1u << B) - 1u));
            float x = (float)(sym - HL);
            if (coset[c]) {
                if constexpr ((HL & 1) == 0) x = __builtin_fminf(x + 0.5f, (float)HL);
                else x = __builtin_fmaxf(x - 0.5f, (float)-HL);
            }
            p[c][j] = x;
        }
    }
}

template <int D, int L, bool IS_KEY, int DR>
__global__ __launch_bounds__(256) void dequant_kernel(CodecArgs a) {
    constexpr int C = D / 32;
    constexpr int RC = RopeChunks<D, DR>::value;
    const int q = threadIdx.x & 3;
    const uint32_t w = (blockIdx.x & 7u) * a.per_xcd + (blockIdx.x >> 3);
    if (w >= a.work) return;
    const uint32_t tensor = w % a.n_tensors;
    const uint32_t rest = w / a.n_tensors;
    const uint32_t bh = rest % a.bh;
    const uint32_t t_raw = (rest / a.bh) * 64u + (threadIdx.x >> 2);
    const bool active = t_raw < a.seq;
    const uint32_t t = active ? t_raw : a.seq - 1u;
    const size_t row = (size_t)bh * a.seq + t;

    float x[C][8];
    int coset[C];
    float scale;
    unpack_points<D, L>(a, tensor, row, q, x, coset, scale);
    const float g = quad_sign(q) * (a.hscale * scale);
    // keys with DR == D: the top Hadamard stage merges with forward RoPE, as in
    // the quantizer (the sum of exact partial transforms is the same number)
    constexpr bool MERGED = IS_KEY && DR == D;
    constexpr bool EXACT_F16 = D * (L / 2) <= 1024;
    if constexpr (EXACT_F16) {
        half2v hp[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                hp[c][k] = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(x[c][2 * k], x[c][2 * k + 1]));
        fwht_row_f16<C, !MERGED>(hp, q);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x[c][2 * k] = __builtin_fmaf((float)hp[c][k].x, g, 0.0f);
                x[c][2 * k + 1] = __builtin_fmaf((float)hp[c][k].y, g, 0.0f);
            }
    } else {
        fwht_row<C, !MERGED>(x, q);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = x[c][i] * g;
    }
    if constexpr (MERGED) {
        float dm[RC][8], dp[RC][8];
        load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, t, q, dm, dp);
        rope_stage_merged<C>(x, dm, dp);
    } else if constexpr (IS_KEY) {
        float cs[RC][8], sn[RC][8];
        load_rope<D, DR, RC>(a.rope_cos, a.rope_sin, t, q, cs, sn);
        apply_rope<D, DR, RC, false>(x, q, cs, sn);
    }
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) asm("" : "+v"(x[c][i]));  // keep the fp32 rounding (see quantizer)
    if (!active) return;
    half2v* dst = reinterpret_cast<half2v*>(reinterpret_cast<uint16_t*>(a.out[tensor]) + row * DR);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        if (32 * c >= DR) continue;
        uint4 o;
        half2v h0 = {(__fp16)x[c][0], (__fp16)x[c][1]}, h1 = {(__fp16)x[c][2], (__fp16)x[c][3]};
        half2v h2 = {(__fp16)x[c][4], (__fp16)x[c][5]}, h3 = {(__fp16)x[c][6], (__fp16)x[c][7]};
        o.x = __builtin_bit_cast(uint32_t, h0);
        o.y = __builtin_bit_cast(uint32_t, h1);
        o.z = __builtin_bit_cast(uint32_t, h2);
        o.w = __builtin_bit_cast(uint32_t, h3);
        *reinterpret_cast<uint4*>(dst + (32 * c + 8 * q) / 2) = o;
    }
}

// ---------------------------------------------------------------------------
// int8 2p codes straight from the packed symbols, in integer arithmetic.  A
// symbol s decodes to the lattice coordinate x = s - L/2, moved half a step in
// the half coset: up and capped at L/2 when L/2 is even, down and floored at
// -L/2 when it is odd (unpack_points above); the code is the int8 byte of 2x.
// Four codes per dword: with y = 2s + 128 - L (+1 or -1 in the half coset)
// every byte lies in [0, 256), so one shift-add forms them without carries and
// an XOR with 0x80 removes the bias; the bytes whose symbol passes the cap
// (floor) are then replaced by it.  Exact for every symbol value (s < 32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ constexpr uint32_t splat8(uint32_t b) { return (b & 0xffu) * 0x01010101u; }

template <int L>
__device__ __forceinline__ uint32_t two_p_bytes(uint32_t s, bool half) {
    constexpr bool UP = ((L / 2) & 1) == 0;
    const uint32_t bias = half ? (UP ? 129u - L : 127u - L) : 128u - L;
    const uint32_t v = ((s << 1) + splat8(bias)) ^ 0x80808080u;
    uint32_t g;  // bit 7 of the bytes the cap (floor) replaces: s >= L (s == 0), half coset only
    if constexpr (UP) g = (s + splat8(half ? 128u - L : 96u)) & 0x80808080u;
    else g = ~(s + splat8(half ? 127u : 128u)) & 0x80808080u;
    const uint32_t m = g | (g - (g >> 7));  // 0xff in those bytes
    constexpr uint32_t bound = splat8(UP ? (uint32_t)L : (uint32_t)-L);
    return (v & ~m) | (bound & m);
}

// Four B-bit fields (bits 0, B, 2B, 3B of x) moved to bytes 0..3.
template <int B>
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
    constexpr uint32_t M = (1u << B) - 1u;
    constexpr uint32_t M2 = (1u << (2 * B)) - 1u;
    x = (x & M2) | ((x << (16 - 2 * B)) & (M2 << 16));  // fields 2, 3 to bit 16
    return (x & (M | (M << 16))) | ((x << (8 - B)) & ((M << 8) | (M << 24)));
}

// 32 bits of a little-endian run of ND dwords from bit `bit` on (zeros past the end).
template <int bit, int ND>
__device__ __forceinline__ uint32_t window32(const uint32_t (&d)[ND]) {
    constexpr int k = bit / 32, sh = bit % 32;
    if constexpr (sh == 0) return d[k];
    else if constexpr (k + 1 < ND) return __builtin_amdgcn_alignbit(d[k + 1], d[k], sh);
    else return d[k] >> sh;
}

// int8 2p of this lane's C groups of one row into an LDS row (D bytes in
// coordinate order): group c covers coordinates 32c + 8q .. +7, and its 8
// B-bit symbols are bits [8Bc, 8Bc + 8B) of the lane's run of C * B symbol
// bytes, turned into bytes 4 at a time.
template <int D, int L, int c = 0>
__device__ __forceinline__ void groups_to_row(const uint32_t (&d)[(D / 32 * SymBits<L>::value + 3) / 4], uint32_t cbits,
                                              int q, uint8_t* lds_row) {
    constexpr int C = D / 32;
    constexpr int B = SymBits<L>::value;
    if constexpr (c < C) {
        const bool half = ((cbits >> (4 * c + q)) & 1u) != 0;
        uint32_t lo, hi;
        if constexpr (B == 4) {
            const uint32_t w = d[c];
            const uint32_t ev = w & 0x0f0f0f0fu, od = (w >> 4) & 0x0f0f0f0fu;  // symbols 0 2 4 6 / 1 3 5 7
            lo = __builtin_amdgcn_perm(od, ev, 0x05010400u);
            hi = __builtin_amdgcn_perm(od, ev, 0x07030602u);
        } else {
            lo = spread4<B>(window32<8 * B * c>(d));
            hi = spread4<B>(window32<8 * B * c + 4 * B>(d));
        }
        *reinterpret_cast<uint2*>(lds_row + 32 * c + 8 * q) = make_uint2(two_p_bytes<L>(lo, half), two_p_bytes<L>(hi, half));
        groups_to_row<D, L, c + 1>(d, cbits, q, lds_row);
    }
}

// The packed symbols (this lane's run of C * B bytes) and coset bits of one row.
template <int D, int L>
struct RowSyms {
    static constexpr int NB = D / 32 * SymBits<L>::value;
    uint32_t d[(NB + 3) / 4];
    uint32_t cbits;

    __device__ __forceinline__ void load(const CodecArgs& a, uint32_t tensor, size_t row, int q) {
        constexpr int ND = (NB + 3) / 4;
        const uint8_t* src = reinterpret_cast<const uint8_t*>(a.syms[tensor]) + row * (D / 8 * SymBits<L>::value) + q * NB;
        if constexpr (NB % 4 == 0) {
#pragma unroll
            for (int k = 0; k < ND; ++k) d[k] = reinterpret_cast<const uint32_t*>(src)[k];
        } else {  // NB = 6 or 10 (head_dim 64): 2-byte aligned
#pragma unroll
            for (int k = 0; k < ND; ++k) {
                const uint32_t lo16 = reinterpret_cast<const uint16_t*>(src)[2 * k];
                const uint32_t hi16 = 4 * k + 2 < NB ? reinterpret_cast<const uint16_t*>(src)[2 * k + 1] : 0u;
                d[k] = lo16 | (hi16 << 16);
            }
        }
        const uint8_t* cb = reinterpret_cast<const uint8_t*>(a.cosets[tensor]) + row * (D / 64);
        if constexpr (D == 64) cbits = *cb;
        else if constexpr (D == 128) cbits = *reinterpret_cast<const uint16_t*>(cb);
        else cbits = *reinterpret_cast<const uint32_t*>(cb);
    }
};

template <int D, int L>
__device__ __forceinline__ void codes_to_row(const CodecArgs& a, uint32_t tensor, size_t row, int q, uint8_t* lds_row) {
    RowSyms<D, L> rs;
    rs.load(a, tensor, row, q);
    groups_to_row<D, L>(rs.d, rs.cbits, q, lds_row);
}

// Byte-wise wrapping subtraction of four int8 lanes.
__device__ __forceinline__ uint32_t sub_bytes(uint32_t a, uint32_t b) {
    return ((a | 0x80808080u) - (b & 0x7f7f7f7fu)) ^ ((a ^ ~b) & 0x80808080u);
}

constexpr uint32_t kInt8Tiles = 8;  // 64-token tiles per block of int8_codes_kernel

// One block per kInt8Tiles consecutive 64-token tiles of one (tensor, batch x
// head) stream.  Per tile, each quad decodes one token row into an LDS tile
// (row stride D + 16 bytes, so the 8-byte writes of a wave's 16 rows spread
// over all banks); the block then streams the tile out in 16-byte chunks,
// contiguous across the tile.  DELTA: LDS row 0 holds the token before the
// tile and each chunk is stored minus the chunk above it.  Lanes 0-3 decode
// that token for the block's first tile (zeros at token 0); for the next ones
// the threads that stored the previous tile's last row write it to row 0 once
// every thread has read the tile, so each row is decoded once.  The symbol
// loads of the next tile are issued before the current tile is decoded.
template <int D, int L, bool DELTA>
__global__ __launch_bounds__(256) void int8_codes_kernel(CodecArgs a) {
    constexpr int STRIDE = D + 16;
    constexpr int CPR = D / 16;  // 16-byte chunks per row
    __shared__ __align__(16) uint8_t tile[65 * STRIDE];
    const int q = threadIdx.x & 3;
    const uint32_t w = (blockIdx.x & 7u) * a.per_xcd + (blockIdx.x >> 3);
    if (w >= a.work) return;  // whole block
    const uint32_t tensor = w % a.n_tensors;
    const uint32_t rest = w / a.n_tensors;
    const uint32_t bh = rest % a.bh;
    const uint32_t t_begin = (rest / a.bh) * (64u * kInt8Tiles);
    const uint32_t t_end = min(t_begin + 64u * kInt8Tiles, a.seq);
    const size_t row0 = (size_t)bh * a.seq;  // the stream's token 0
    const uint32_t r = threadIdx.x >> 2;
    if constexpr (DELTA) {
        if (threadIdx.x < 4) {
            if (t_begin > 0) {
                codes_to_row<D, L>(a, tensor, row0 + t_begin - 1, q, tile);
            } else {
#pragma unroll
                for (int c = 0; c < D / 32; ++c) *reinterpret_cast<uint2*>(tile + 32 * c + 8 * q) = make_uint2(0u, 0u);
            }
        }
    }
    int8_t* dst = reinterpret_cast<int8_t*>(a.out[tensor]) + row0 * D;
    // this thread's row of the next tile is loaded while the current one is
    // decoded and stored (rows past the stream read its last row, unused)
    RowSyms<D, L> next;
    next.load(a, tensor, row0 + min(t_begin + r, a.seq - 1u), q);
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += 64) {
        const uint32_t n_rows = min(64u, t_end - t0);
        const RowSyms<D, L> cur = next;
        if (t0 + 64 < t_end) next.load(a, tensor, row0 + min(t0 + 64 + r, a.seq - 1u), q);
        if (r < n_rows) groups_to_row<D, L>(cur.d, cur.cbits, q, tile + (r + 1) * STRIDE);
        __syncthreads();
        uint4 last = make_uint4(0u, 0u, 0u, 0u);
        int last_cc = -1;  // this thread's chunk of the tile's row 63, if it stored one
        for (uint32_t k = threadIdx.x; k < n_rows * CPR; k += 256) {
            const uint32_t rr = k / CPR, cc = k % CPR;
            const uint4 v = *reinterpret_cast<const uint4*>(tile + (rr + 1) * STRIDE + 16 * cc);
            uint4 o = v;
            if constexpr (DELTA) {
                const uint4 p = *reinterpret_cast<const uint4*>(tile + rr * STRIDE + 16 * cc);
                o = make_uint4(sub_bytes(v.x, p.x), sub_bytes(v.y, p.y), sub_bytes(v.z, p.z), sub_bytes(v.w, p.w));
                if (rr == 63) {
                    last = v;
                    last_cc = (int)cc;
                }
            }
            *reinterpret_cast<uint4*>(dst + (size_t)t0 * D + 16 * k) = o;
        }
        __syncthreads();  // the tile is read: rows 1..64 (and row 0) may be overwritten
        if constexpr (DELTA) {
            if (last_cc >= 0) *reinterpret_cast<uint4*>(tile + 16 * last_cc) = last;
        }
    }
}

// ---------------------------------------------------------------------------
// Raw int8 token deltas and their inverse over [stream][token][coord] bytes.
// A thread owns one W-byte word of a token row (W = 16, 4 or 1 as the row
// width allows); int8 lanes wrap like numpy's int8 arithmetic.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t add_bytes(uint32_t a, uint32_t b) {
    return ((a & 0x7f7f7f7fu) + (b & 0x7f7f7f7fu)) ^ ((a ^ b) & 0x80808080u);
}

template <int W> struct Bytes;
template <> struct Bytes<1> {
    using T = uint8_t;
    static __device__ __forceinline__ T add(T a, T b) { return (T)(a + b); }
    static __device__ __forceinline__ T sub(T a, T b) { return (T)(a - b); }
    static __device__ __forceinline__ T zero() { return 0; }
};
template <> struct Bytes<4> {
    using T = uint32_t;
    static __device__ __forceinline__ T add(T a, T b) { return add_bytes(a, b); }
    static __device__ __forceinline__ T sub(T a, T b) { return sub_bytes(a, b); }
    static __device__ __forceinline__ T zero() { return 0u; }
};
template <> struct Bytes<16> {
    using T = uint4;
    static __device__ __forceinline__ T add(T a, T b) {
        return make_uint4(add_bytes(a.x, b.x), add_bytes(a.y, b.y), add_bytes(a.z, b.z), add_bytes(a.w, b.w));
    }
    static __device__ __forceinline__ T sub(T a, T b) {
        return make_uint4(sub_bytes(a.x, b.x), sub_bytes(a.y, b.y), sub_bytes(a.z, b.z), sub_bytes(a.w, b.w));
    }
    static __device__ __forceinline__ T zero() { return make_uint4(0u, 0u, 0u, 0u); }
};

struct DeltaGeom {
    uint32_t seq;        // token rows per stream
    uint32_t row_words;  // W-byte words per token row
    uint32_t chunk_len;  // token rows per scan chunk (the last chunk may be shorter)
    uint32_t n_chunks;
    uint32_t n_threads;  // streams * n_chunks * row_words
};

// out[s, t] = x[s, t] - x[s, t - 1] for t > 0, x[s, 0] at t = 0.  out must not
// alias x: the previous row is read by another thread.
template <int W>
__global__ __launch_bounds__(256) void delta_encode_kernel(const uint64_t* src, const uint64_t* out, uint32_t n_words,
                                                           uint32_t row_words, uint32_t seq) {
    using B = Bytes<W>;
    using T = typename B::T;
    const T* __restrict__ x = reinterpret_cast<const T*>(src[blockIdx.y]);
    T* __restrict__ o = reinterpret_cast<T*>(out[blockIdx.y]);
    const uint32_t stride = gridDim.x * 256u;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n_words; i += stride) {
        T v = x[i];
        if ((i / row_words) % seq != 0) v = B::sub(v, x[i - row_words]);
        o[i] = v;
    }
}

// Word `word` of the token rows of (stream, chunk).
__device__ __forceinline__ void delta_column(const DeltaGeom& g, uint32_t i, uint32_t& stream, uint32_t& chunk,
                                             uint32_t& word) {
    word = i % g.row_words;
    const uint32_t sc = i / g.row_words;
    chunk = sc % g.n_chunks;
    stream = sc / g.n_chunks;
}

__device__ __forceinline__ uint32_t chunk_last_row(const DeltaGeom& g, uint32_t chunk) {
    return min(g.seq, (chunk + 1u) * g.chunk_len) - 1u;
}

// Pass 1 of a chunked scan: the wrapping sum of each chunk's deltas, stored
// at the chunk's last row of out.
template <int W>
__global__ __launch_bounds__(256) void delta_chunk_totals_kernel(const uint64_t* deltas, const uint64_t* out,
                                                                 DeltaGeom g) {
    using B = Bytes<W>;
    using T = typename B::T;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= g.n_threads) return;
    uint32_t stream, chunk, word;
    delta_column(g, i, stream, chunk, word);
    const size_t base = (size_t)stream * g.seq * g.row_words + word;
    const T* in = reinterpret_cast<const T*>(deltas[blockIdx.y]) + base;
    T* o = reinterpret_cast<T*>(out[blockIdx.y]) + base;
    const uint32_t t0 = chunk * g.chunk_len, t1 = chunk_last_row(g, chunk) + 1u;
    constexpr int U = 8;
    T acc = B::zero();
    uint32_t t = t0;
    for (; t + U <= t1; t += U) {
        T d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = in[(size_t)(t + u) * g.row_words];
#pragma unroll
        for (int u = 0; u < U; ++u) acc = B::add(acc, d[u]);
    }
    for (; t < t1; ++t) acc = B::add(acc, in[(size_t)t * g.row_words]);
    o[(size_t)(t1 - 1u) * g.row_words] = acc;
}

// Pass 2: running sums of the chunk totals, one workgroup per (stream, word)
// column: thread j loads the totals of chunks [j*per, (j+1)*per) (per <= 16),
// the 256 partial sums are scanned in LDS, and each chunk's last row then
// holds the inclusive prefix through that row.
template <int W>
__global__ __launch_bounds__(256) void delta_chunk_prefix_kernel(const uint64_t* out, DeltaGeom g) {
    using B = Bytes<W>;
    using T = typename B::T;
    constexpr int PER = 16;
    __shared__ T part[256];
    const uint32_t col = blockIdx.x;
    const uint32_t word = col % g.row_words, stream = col / g.row_words;
    T* o = reinterpret_cast<T*>(out[blockIdx.y]) + (size_t)stream * g.seq * g.row_words + word;
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (g.n_chunks + 255u) / 256u;
    const uint32_t k0 = tid * per;
    T v[PER];
    T sum = B::zero();
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const uint32_t k = k0 + (uint32_t)u;
        if ((uint32_t)u < per && k < g.n_chunks) {
            v[u] = o[(size_t)chunk_last_row(g, k) * g.row_words];
            sum = B::add(sum, v[u]);
        }
    }
    part[tid] = sum;
    __syncthreads();
    for (uint32_t off = 1; off < 256u; off <<= 1) {
        const T x = tid >= off ? part[tid - off] : B::zero();
        __syncthreads();
        part[tid] = B::add(part[tid], x);
        __syncthreads();
    }
    T acc = tid > 0 ? part[tid - 1] : B::zero();
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const uint32_t k = k0 + (uint32_t)u;
        if ((uint32_t)u < per && k < g.n_chunks) {
            acc = B::add(acc, v[u]);
            o[(size_t)chunk_last_row(g, k) * g.row_words] = acc;
        }
    }
}

// Pass 3 (the whole scan when n_chunks == 1): prefix sums of a chunk's rows,
// starting from the previous chunk's last row.  With several chunks the last
// row of each chunk already holds its final value (passes 1-2) and is left as
// it is, so no thread writes a row another thread reads.
template <int W>
__global__ __launch_bounds__(256) void delta_chunk_scan_kernel(const uint64_t* deltas, const uint64_t* out,
                                                               DeltaGeom g) {
    using B = Bytes<W>;
    using T = typename B::T;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= g.n_threads) return;
    uint32_t stream, chunk, word;
    delta_column(g, i, stream, chunk, word);
    const size_t base = (size_t)stream * g.seq * g.row_words + word;
    const T* in = reinterpret_cast<const T*>(deltas[blockIdx.y]) + base;
    T* o = reinterpret_cast<T*>(out[blockIdx.y]) + base;
    const uint32_t t0 = chunk * g.chunk_len;
    const uint32_t t1 = g.n_chunks > 1 ? chunk_last_row(g, chunk) : g.seq;
    T acc = chunk > 0 ? o[(size_t)(t0 - 1u) * g.row_words] : B::zero();
    constexpr int U = 8;
    uint32_t t = t0;
    for (; t + U <= t1; t += U) {
        T d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = in[(size_t)(t + u) * g.row_words];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc = B::add(acc, d[u]);
            o[(size_t)(t + u) * g.row_words] = acc;
        }
    }
    for (; t < t1; ++t) {
        acc = B::add(acc, in[(size_t)t * g.row_words]);
        o[(size_t)t * g.row_words] = acc;
    }
}

// Word width of a row of `coords` bytes.
static int delta_word_bytes(int32_t coords) { return coords % 16 == 0 ? 16 : coords % 4 == 0 ? 4 : 1; }

template <int W>
static hipError_t launch_delta_encode(const uint64_t* src, const uint64_t* out, uint32_t n_tensors, uint32_t n_words,
                                      uint32_t row_words, uint32_t seq, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>(((uint64_t)n_words + 255) / 256, 8192);
    hipLaunchKernelGGL(delta_encode_kernel<W>, dim3(blocks, n_tensors), dim3(256), 0, s, src, out, n_words, row_words,
                       seq);
    return hipGetLastError();
}

template <int W>
static hipError_t launch_delta_decode(const uint64_t* deltas, const uint64_t* out, uint32_t n_tensors,
                                      uint32_t streams, DeltaGeom g, hipStream_t s) {
    const uint32_t cols = streams * g.row_words;
    if (g.n_chunks > 1) {
        hipLaunchKernelGGL(delta_chunk_totals_kernel<W>, dim3((g.n_threads + 255) / 256, n_tensors), dim3(256), 0, s,
                           deltas, out, g);
        hipLaunchKernelGGL(delta_chunk_prefix_kernel<W>, dim3(cols, n_tensors), dim3(256), 0, s, out, g);
    }
    hipLaunchKernelGGL(delta_chunk_scan_kernel<W>, dim3((g.n_threads + 255) / 256, n_tensors), dim3(256), 0, s,
                       deltas, out, g);
    return hipGetLastError();
}

template <int D, int L, int DR>
static hipError_t launch_codec(int kind, bool key, const CodecArgs& a, hipStream_t s) {
    dim3 grid(a.per_xcd * 8u);
    if (kind == 0) {
        if (key) hipLaunchKernelGGL((dequant_kernel<D, L, true, DR>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((dequant_kernel<D, L, false, DR>), grid, dim3(256), 0, s, a);
    } else {
        // int8 codes: blocks of kInt8Tiles tiles of one stream
        CodecArgs b = a;
        b.work = (uint32_t)((((uint64_t)a.seq + 64u * kInt8Tiles - 1) / (64u * kInt8Tiles)) * a.bh * a.n_tensors);
        b.per_xcd = (b.work + 7u) / 8u;
        dim3 grid8(b.per_xcd * 8u);
        if (kind == 1) hipLaunchKernelGGL((int8_codes_kernel<D, L, false>), grid8, dim3(256), 0, s, b);
        else hipLaunchKernelGGL((int8_codes_kernel<D, L, true>), grid8, dim3(256), 0, s, b);
    }
    return hipGetLastError();
}

template <int D, int DR = D>
static hipError_t codec_levels(int L, int kind, bool key, const CodecArgs& a, hipStream_t s) {
    switch (L) {
        case 2: return launch_codec<D, 2, DR>(kind, key, a, s);
        case 4: return launch_codec<D, 4, DR>(kind, key, a, s);
        case 8: return launch_codec<D, 8, DR>(kind, key, a, s);
        default: return launch_codec<D, 16, DR>(kind, key, a, s);
    }
}

static int run_codec(const nq_codes_desc* d, int kind, void* stream) {
    NQ_CHECK_ARG(d != nullptr, "nq codes: desc is NULL");
    NQ_CHECK_ARG(d->n_tensors >= 0 && d->n_tensors <= 65535, "nq codes: n_tensors out of range");
    if (d->n_tensors == 0 || d->seq == 0) return NQ_OK;
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 96 || d->head_dim == 128 || d->head_dim == 256,
                 "nq codes: head_dim %d unsupported (64, 96, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->levels == 2 || d->levels == 4 || d->levels == 8 || d->levels == 16,
                 "nq codes: levels must be 2, 4, 8 or 16");
    NQ_CHECK_ARG(d->batch > 0 && d->heads > 0 && d->seq > 0, "nq codes: bad geometry");
    NQ_CHECK_ARG(d->syms && d->cosets && d->scales && d->out, "nq codes: NULL pointer array");
    if (kind == 0 && d->is_key) {
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin && d->rope_n_pos >= d->seq, "nq_dequantize: RoPE table too short");
        NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                     "nq_dequantize: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
        NQ_CHECK_ARG(d->rope_sin_minus_cos == nullptr || d->head_dim != 96,
                     "nq_dequantize: head_dim 96 keys take cos / sin tables only");
    }
    const uint64_t rows = (uint64_t)d->batch * d->heads * d->seq;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq codes: too many rows");
    CodecArgs a;
    a.syms = d->syms;
    a.cosets = d->cosets;
    a.scales = d->scales;
    a.out = d->out;
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.heads = (uint32_t)d->heads;
    a.seq = (uint32_t)d->seq;
    a.n_tensors = (uint32_t)d->n_tensors;
    a.bh = (uint32_t)d->batch * (uint32_t)d->heads;
    const uint64_t work = (uint64_t)((d->seq + 63) / 64) * a.bh * a.n_tensors;
    NQ_CHECK_ARG(work + 8 <= max_blocks(256), "nq codes: grid too large");
    a.work = (uint32_t)work;
    a.per_xcd = (uint32_t)((work + 7) / 8);
    a.hscale = d->hadamard_scale;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    switch (d->head_dim) {
        case 64: e = codec_levels<64>(d->levels, kind, d->is_key != 0, a, s); break;
        case 96: e = codec_levels<128, 96>(d->levels, kind, d->is_key != 0, a, s); break;
        case 128: e = codec_levels<128>(d->levels, kind, d->is_key != 0, a, s); break;
        default: e = codec_levels<256>(d->levels, kind, d->is_key != 0, a, s); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

}  // namespace nq

extern "C" int nq_dequantize(const nq_codes_desc* desc, void* stream) { return nq::run_codec(desc, 0, stream); }

extern "C" int nq_codes_to_int8(const nq_codes_desc* desc, int32_t delta, void* stream) {
    return nq::run_codec(desc, delta ? 2 : 1, stream);
}

extern "C" int nq_delta_encode(const uint64_t* src, const uint64_t* out, int32_t n_tensors, int32_t streams,
                               int32_t seq, int32_t coords, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(src && out, "nq_delta_encode: NULL pointer array");
    NQ_CHECK_ARG(n_tensors >= 0 && n_tensors <= 65535 && streams >= 0 && seq >= 0 && coords > 0,
                 "nq_delta_encode: bad shape");
    if (n_tensors == 0 || streams == 0 || seq == 0) return NQ_OK;
    const int W = delta_word_bytes(coords);
    const uint64_t row_words = (uint64_t)coords / W;
    const uint64_t n_words = (uint64_t)streams * seq * row_words;
    NQ_CHECK_ARG(n_words < (1ull << 32) - (1ull << 22), "nq_delta_encode: tensor too large (%llu words of %d bytes)",
                 (unsigned long long)n_words, W);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (W == 16) e = launch_delta_encode<16>(src, out, n_tensors, (uint32_t)n_words, (uint32_t)row_words, seq, s);
    else if (W == 4) e = launch_delta_encode<4>(src, out, n_tensors, (uint32_t)n_words, (uint32_t)row_words, seq, s);
    else e = launch_delta_encode<1>(src, out, n_tensors, (uint32_t)n_words, (uint32_t)row_words, seq, s);
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

extern "C" int nq_delta_decode(const uint64_t* deltas, const uint64_t* out, int32_t n_tensors, int32_t streams,
                               int32_t seq, int32_t coords, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(deltas && out, "nq_delta_decode: NULL pointer array");
    NQ_CHECK_ARG(n_tensors >= 0 && n_tensors <= 65535 && streams >= 0 && seq >= 0 && coords > 0,
                 "nq_delta_decode: bad shape");
    if (n_tensors == 0 || streams == 0 || seq == 0) return NQ_OK;
    const int W = delta_word_bytes(coords);
    DeltaGeom g;
    g.seq = (uint32_t)seq;
    g.row_words = (uint32_t)(coords / W);
    const uint64_t cols = (uint64_t)streams * g.row_words;
    NQ_CHECK_ARG(cols < (1ull << 31), "nq_delta_decode: too many streams");
    // Split the token axis into chunks when the columns alone would leave the
    // chip idle: about 2^17 threads in flight, chunks of at least 16 rows and
    // at most 4096 chunks (16 per thread of the prefix workgroup).
    constexpr uint64_t kTargetThreads = 1u << 17;
    uint64_t n_chunks = 1;
    if (cols < kTargetThreads) {
        n_chunks = std::min<uint64_t>((kTargetThreads + cols - 1) / cols, ((uint64_t)seq + 15) / 16);
        n_chunks = std::max<uint64_t>(1, std::min<uint64_t>(n_chunks, 4096));
    }
    g.chunk_len = (uint32_t)(((uint64_t)seq + n_chunks - 1) / n_chunks);
    g.n_chunks = (uint32_t)(((uint64_t)seq + g.chunk_len - 1) / g.chunk_len);
    NQ_CHECK_ARG(cols * g.n_chunks < (1ull << 32) - 256, "nq_delta_decode: too many columns");
    g.n_threads = (uint32_t)(cols * g.n_chunks);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (W == 16) e = launch_delta_decode<16>(deltas, out, n_tensors, streams, g, s);
    else if (W == 4) e = launch_delta_decode<4>(deltas, out, n_tensors, streams, g, s);
    else e = launch_delta_decode<1>(deltas, out, n_tensors, streams, g, s);
    NQ_CHECK_HIP(e);
    return NQ_OK;
}
