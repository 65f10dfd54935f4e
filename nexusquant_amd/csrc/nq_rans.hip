// Chunked rANS entropy coding of int8 lattice codes (c = 2p) on gfx950.
//
// The coder is the reference's (entropy_coder.py:163-345): 32-bit state in
// [2^16, 2^32), 16-bit renormalisation, frequencies summing to 2^12, symbols
// encoded in reverse and the word list reversed, so decoding runs forward.
// The stream is cut into chunks of `chunk` symbols; one lane codes one chunk
// with its own state, so each chunk's words are exactly what the reference
// encoder writes for that chunk's symbols on its own.
//
// Symbols: with half-integer points present (has_half) s = c + L (alphabet
// 2L + 1), otherwise s = c/2 + L/2 (alphabet L + 1) (entropy_coder.py:35-75).
#include "nq_common.h"

namespace nq {

constexpr uint32_t kRansM = 1u << 12;
constexpr uint32_t kRansL = 1u << 16;
constexpr int kRansMaxAlpha = 64;

__device__ __forceinline__ int rans_symbol(int8_t c, int L, int has_half) {
    return has_half ? (int)c + L : ((int)c >> 1) + L / 2;
}

__device__ __forceinline__ int8_t rans_code(int s, int L, int has_half) {
    return (int8_t)(has_half ? s - L : 2 * (s - L / 2));
}

__device__ __forceinline__ int hist_bin(int8_t c, int L) {
    const int b = (int)c + L;
    return b < 0 ? 0 : (b > 2 * L ? 2 * L : b);  // codes outside [-L, L] are not valid input
}

// histogram of c + L over [0, 2L] (the host folds it when no code is odd)
__global__ __launch_bounds__(256) void rans_hist_kernel(const int8_t* codes, int64_t n, int L, uint32_t* hist) {
    __shared__ uint32_t h[kRansMaxAlpha];
    if (threadIdx.x < kRansMaxAlpha) h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t stride = (int64_t)gridDim.x * 256 * 16;
    for (int64_t base = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16; base < n; base += stride) {
        if (base + 16 <= n) {
            const uint4 w = *reinterpret_cast<const uint4*>(codes + base);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) atomicAdd(&h[hist_bin((int8_t)(ws[k] >> (8 * j)), L)], 1u);
        } else {
            for (int64_t i = base; i < n; ++i) atomicAdd(&h[hist_bin(codes[i], L)], 1u);
        }
    }
    __syncthreads();
    if (threadIdx.x <= 2 * L && h[threadIdx.x]) atomicAdd(&hist[threadIdx.x], h[threadIdx.x]);
}

struct RansArgs {
    const int8_t* codes;
    int8_t* out_codes;
    const uint16_t* freq;
    uint16_t* scratch;       // [n_chunks][rans_stride(chunk)] words, each chunk's stream right-aligned
    uint32_t* n_words;       // [n_chunks]
    const uint64_t* offset;  // [n_chunks + 1] word offsets in the compacted stream (decode)
    const uint16_t* words;   // compacted stream (decode)
    int64_t n;
    int64_t n_chunks;
    int chunk, L, has_half, alphabet;
};

// words per chunk in the encoder's scratch: the chunk's worst case (one word
// per symbol plus the two state words), rounded to 4 words so every chunk's
// right end is 8-byte aligned
__host__ __device__ __forceinline__ int64_t rans_stride(int chunk) { return ((int64_t)chunk + 2 + 3) & ~(int64_t)3; }

// x / d for x < d * 2^20, d in [1, 4096]: the fp32 quotient is within 1 of the
// true one, and one remainder test corrects it
__device__ __forceinline__ uint32_t rans_div(uint32_t x, uint32_t d, float rcp, uint32_t& r) {
    uint32_t q = (uint32_t)((float)x * rcp);
    int32_t rem = (int32_t)(x - q * d);
    if (rem < 0) {
        --q;
        rem += (int32_t)d;
    } else if (rem >= (int32_t)d) {
        ++q;
        rem -= (int32_t)d;
    }
    r = (uint32_t)rem;
    return q;
}

// One lane per chunk, one wave per block (so the chunks spread over every CU).
// Codes are read 16 at a time from the chunk's end backwards; emitted words
// collect in a 64-bit buffer and leave in 8-byte stores.
__global__ __launch_bounds__(64) void rans_encode_kernel(RansArgs a) {
    __shared__ uint32_t fc[kRansMaxAlpha];  // f | cf << 16
    __shared__ float rcp[kRansMaxAlpha];
    if (threadIdx.x == 0) {
        uint32_t acc = 0;
        for (int s = 0; s < a.alphabet; ++s) {
            const uint32_t f = a.freq[s];
            fc[s] = f | (acc << 16);
            rcp[s] = f ? 1.0f / (float)f : 0.0f;
            acc += f;
        }
    }
    __syncthreads();
    const int64_t ch = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (ch >= a.n_chunks) return;
    const int64_t c0 = ch * a.chunk;
    const int64_t c1 = c0 + a.chunk < a.n ? c0 + a.chunk : a.n;
    uint16_t* const end = a.scratch + (ch + 1) * rans_stride(a.chunk);
    uint16_t* out = end;  // next 4-word group goes just below
    uint64_t buf = 0;
    int nbuf = 0;
    uint32_t n_emit = 0;
    auto emit = [&](uint32_t wd) {
        buf = (buf << 16) | wd;
        ++n_emit;
        if (++nbuf == 4) {
            out -= 4;
            *reinterpret_cast<uint64_t*>(out) = buf;
            nbuf = 0;
        }
    };
    uint32_t state = kRansL;
    auto code_one = [&](int8_t c) {
        int s = rans_symbol(c, a.L, a.has_half);
        s = s < 0 ? 0 : (s >= a.alphabet ? a.alphabet - 1 : s);  // codes outside [-L, L] are not valid input
        const uint32_t e = fc[s];
        const uint32_t fs = e & 0xffffu, cs = e >> 16;
        if ((uint64_t)state >= ((uint64_t)fs << 20)) {  // at most one word: state >> 16 < 2^16 <= fs << 20
            emit(state & 0xffffu);
            state >>= 16;
        }
        uint32_t r;
        const uint32_t q = rans_div(state, fs, rcp[s], r);
        state = q * kRansM + r + cs;
    };
    // 16-byte blocks [b, b + 16) from the one holding c1 - 1 down to the one holding c0
    int64_t b = ((c1 - 1) / 16) * 16;
    auto load_block = [&](int64_t bb) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (bb + 16 <= a.n) {
            v = *reinterpret_cast<const uint4*>(a.codes + bb);
        } else {  // the array's last, partial block
            uint8_t t[16] = {};
            for (int k = 0; k < 16 && bb + k < a.n; ++k) t[k] = (uint8_t)a.codes[bb + k];
            v = *reinterpret_cast<const uint4*>(t);
        }
        return v;
    };
    uint4 cur = load_block(b);
    for (; b + 16 > c0; b -= 16) {
        const uint4 nxt = b - 16 >= 0 && b - 16 + 16 > c0 ? load_block(b - 16) : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t wv[4] = {cur.x, cur.y, cur.z, cur.w};
        const int k_hi = (int)((c1 - 1 < b + 15 ? c1 - 1 : b + 15) - b);
        const int k_lo = (int)((c0 > b ? c0 : b) - b);
        if (k_hi == 15 && k_lo == 0) {
#pragma unroll
            for (int k = 15; k >= 0; --k) code_one((int8_t)(wv[k >> 2] >> (8 * (k & 3))));
        } else {
            for (int k = k_hi; k >= k_lo; --k) code_one((int8_t)(wv[k >> 2] >> (8 * (k & 3))));
        }
        cur = nxt;
    }
    emit(state & 0xffffu);
    emit(state >> 16);
    // the last 0..3 words, just below the stored groups: the earliest emitted
    // (the buffer's highest) at the highest address
    for (int k = 0; k < nbuf; ++k) out[-1 - k] = (uint16_t)(buf >> (16 * (nbuf - 1 - k)));
    a.n_words[ch] = n_emit;
}

// copy each chunk's right-aligned words to its compacted offset; one wave per chunk
__global__ __launch_bounds__(256) void rans_compact_kernel(const uint16_t* scratch, const uint32_t* n_words,
                                                           const uint64_t* offset, int64_t n_chunks, int chunk,
                                                           uint16_t* words) {
    const int64_t ch = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (ch >= n_chunks) return;
    const int lane = threadIdx.x & 63;
    const uint32_t nw = n_words[ch];
    const uint16_t* src = scratch + (ch + 1) * rans_stride(chunk) - nw;
    uint16_t* dst = words + offset[ch];
    for (uint32_t i = lane; i < nw; i += 64) dst[i] = src[i];
}

// One lane per chunk, one wave per block.  A 4096-entry LDS table maps a slot
// to code byte | (slot - cf[s]) << 8 | (f[s] - 1) << 20 for its symbol s.  A
// symbol needs at most one word (the state is >= 16 before renormalisation);
// words are read 4 at a time (aligned 8-byte loads inside the stream, single
// words at its very end), and decoded codes leave 16 at a time when the
// chunk's start is 16-aligned.
__global__ __launch_bounds__(64) void rans_decode_kernel(RansArgs a) {
    __shared__ uint32_t tab[kRansM];
    __shared__ uint16_t cf[kRansMaxAlpha + 1];
    if (threadIdx.x == 0) {
        uint32_t acc = 0;
        for (int s = 0; s < a.alphabet; ++s) {
            cf[s] = (uint16_t)acc;
            acc += a.freq[s];
        }
        cf[a.alphabet] = (uint16_t)acc;
    }
    __syncthreads();
    for (int s = 0; s < a.alphabet; ++s) {
        const uint32_t lo = cf[s], hi = cf[s + 1] < kRansM ? cf[s + 1] : kRansM;
        const uint32_t code = (uint8_t)rans_code(s, a.L, a.has_half);
        const uint32_t fm1 = (hi > lo ? hi - lo : 1u) - 1u;
        for (uint32_t k = lo + threadIdx.x; k < hi; k += 64) tab[k] = code | ((k - lo) << 8) | (fm1 << 20);
    }
    __syncthreads();
    const int64_t ch = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (ch >= a.n_chunks) return;
    const int64_t c0 = ch * a.chunk;
    const uint32_t n_sym = (uint32_t)((c0 + a.chunk < a.n ? c0 + a.chunk : a.n) - c0);
    const uint64_t w0 = a.offset[ch];
    const uint32_t len = (uint32_t)(a.offset[ch + 1] - w0);
    const uint64_t total = a.offset[a.n_chunks];
    // sequential word reader: gbuf holds the next gleft words of the aligned
    // 4-word group starting at word g (groups past the stream's end read as 0)
    auto load_group = [&](uint64_t g) -> uint64_t {
        if (g + 4 <= total) return *reinterpret_cast<const uint64_t*>(a.words + g);
        uint64_t v = 0;
        for (uint64_t k = 0; g + k < total; ++k) v |= (uint64_t)a.words[g + k] << (16 * k);
        return v;
    };
    uint64_t g = w0 & ~(uint64_t)3;
    uint64_t gbuf = load_group(g) >> (16 * (uint32_t)(w0 & 3));
    uint32_t gleft = 4u - (uint32_t)(w0 & 3);
    auto next_word = [&]() -> uint32_t {
        if (gleft == 0) {
            g += 4;
            gbuf = load_group(g);
            gleft = 4;
        }
        const uint32_t v = (uint32_t)gbuf & 0xffffu;
        gbuf >>= 16;
        --gleft;
        return v;
    };
    uint32_t pos = 2;
    uint32_t state = kRansL;
    if (len >= 2) {
        const uint32_t hi = next_word();
        state = (hi << 16) | next_word();
    }
    auto step = [&]() -> uint32_t {
        const uint32_t e = tab[state & (kRansM - 1u)];
        state = ((e >> 20) + 1u) * (state >> 12) + ((e >> 8) & 0xfffu);
        if (state < kRansL && pos < len) {
            state = (state << 16) | next_word();
            ++pos;
        }
        return e & 0xffu;
    };
    int8_t* out = a.out_codes + c0;
    uint32_t i = 0;
    if ((((uintptr_t)out) & 15) == 0) {
        for (; i + 16 <= n_sym; i += 16) {
            uint32_t ob[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t v = step();
                v |= step() << 8;
                v |= step() << 16;
                v |= step() << 24;
                ob[q] = v;
            }
            *reinterpret_cast<uint4*>(out + i) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
        }
    }
    for (; i < n_sym; ++i) out[i] = (int8_t)step();
}

// exclusive scan of n_words into offset[0..n_chunks]: one block; per round
// every thread sums 32 consecutive counts, one block-wide scan of the 1024
// sums, then every thread writes its 32 offsets
__global__ __launch_bounds__(1024) void rans_scan_kernel(const uint32_t* n_words, int64_t n_chunks, uint64_t* offset) {
    __shared__ uint64_t s[1024];
    constexpr int kPer = 32;
    uint64_t carry = 0;
    for (int64_t b0 = 0; b0 < n_chunks; b0 += 1024 * kPer) {
        const int64_t i0 = b0 + (int64_t)threadIdx.x * kPer;
        uint32_t cnt[kPer];
        if (i0 + kPer <= n_chunks && ((reinterpret_cast<uintptr_t>(n_words + i0) & 15) == 0)) {
#pragma unroll
            for (int k = 0; k < kPer; k += 4) {
                const uint4 v = *reinterpret_cast<const uint4*>(n_words + i0 + k);
                cnt[k] = v.x;
                cnt[k + 1] = v.y;
                cnt[k + 2] = v.z;
                cnt[k + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPer; ++k) cnt[k] = i0 + k < n_chunks ? n_words[i0 + k] : 0u;
        }
        uint64_t sum = 0;
#pragma unroll
        for (int k = 0; k < kPer; ++k) sum += cnt[k];
        s[threadIdx.x] = sum;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const uint64_t add = threadIdx.x >= (unsigned)o ? s[threadIdx.x - o] : 0;
            __syncthreads();
            s[threadIdx.x] += add;
            __syncthreads();
        }
        uint64_t run = carry + s[threadIdx.x] - sum;  // exclusive prefix of this thread's first count
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            if (i0 + k < n_chunks) offset[i0 + k] = run;
            run += cnt[k];
        }
        carry += s[1023];
        __syncthreads();
    }
    if (threadIdx.x == 0) offset[n_chunks] = carry;
}

}  // namespace nq

using namespace nq;

extern "C" int nq_rans_histogram(const int8_t* codes, int64_t n, int32_t levels, uint32_t* hist, void* stream) {
    NQ_CHECK_ARG(levels == 2 || levels == 4 || levels == 8 || levels == 16,
                 "nq_rans_histogram: levels must be 2, 4, 8 or 16 (got %d)", levels);
    NQ_CHECK_ARG(n >= 0 && (n == 0 || (codes && hist)), "nq_rans_histogram: bad arguments");
    NQ_CHECK_ARG(((uintptr_t)codes & 15) == 0, "nq_rans_histogram: codes must be 16-byte aligned");
    if (n == 0) return NQ_OK;
    int64_t blocks = (n + 256 * 16 - 1) / (256 * 16);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(rans_hist_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, codes, n, levels,
                       hist);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

static int rans_check(const char* who, int64_t n, int32_t chunk, int32_t levels, int32_t has_half,
                      const uint16_t* freq, int32_t alphabet) {
    NQ_CHECK_ARG(levels == 2 || levels == 4 || levels == 8 || levels == 16, "%s: levels must be 2, 4, 8 or 16", who);
    NQ_CHECK_ARG(alphabet == (has_half ? 2 * levels + 1 : levels + 1), "%s: alphabet %d does not match levels %d%s",
                 who, alphabet, levels, has_half ? " (half-integer codes)" : "");
    NQ_CHECK_ARG(chunk >= 1 && chunk <= (1 << 24), "%s: chunk %d out of range", who, chunk);
    NQ_CHECK_ARG(n >= 0 && freq != nullptr, "%s: bad arguments", who);
    return NQ_OK;
}

extern "C" int64_t nq_rans_scratch_words(int64_t n, int32_t chunk) {
    if (n <= 0 || chunk <= 0) return 0;
    return (n + chunk - 1) / chunk * rans_stride(chunk);
}

extern "C" int nq_rans_encode(const int8_t* codes, int64_t n, int32_t levels, int32_t has_half, const uint16_t* freq,
                              int32_t alphabet, int32_t chunk, uint16_t* scratch, uint32_t* n_words,
                              uint64_t* offset, void* stream) {
    const int st = rans_check("nq_rans_encode", n, chunk, levels, has_half, freq, alphabet);
    if (st != NQ_OK) return st;
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    NQ_CHECK_ARG(n == 0 || (codes && scratch && n_words && offset), "nq_rans_encode: NULL buffer");
    NQ_CHECK_ARG(((uintptr_t)codes & 15) == 0 && ((uintptr_t)scratch & 7) == 0,
                 "nq_rans_encode: codes must be 16-byte and scratch 8-byte aligned");
    NQ_CHECK_ARG((n_chunks + 63) / 64 < (1ll << 31), "nq_rans_encode: too many chunks");
    hipStream_t s = (hipStream_t)stream;
    if (n_chunks > 0) {
        RansArgs a = {};
        a.codes = codes;
        a.freq = freq;
        a.scratch = scratch;
        a.n_words = n_words;
        a.n = n;
        a.n_chunks = n_chunks;
        a.chunk = chunk;
        a.L = levels;
        a.has_half = has_half;
        a.alphabet = alphabet;
        hipLaunchKernelGGL(rans_encode_kernel, dim3((uint32_t)((n_chunks + 63) / 64)), dim3(64), 0, s, a);
        NQ_CHECK_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(rans_scan_kernel, dim3(1), dim3(1024), 0, s, n_words, n_chunks, offset);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_rans_compact(const uint16_t* scratch, const uint32_t* n_words, const uint64_t* offset,
                               int64_t n, int32_t chunk, uint16_t* words, void* stream) {
    NQ_CHECK_ARG(chunk >= 1 && n >= 0, "nq_rans_compact: bad arguments");
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    if (n_chunks == 0) return NQ_OK;
    NQ_CHECK_ARG(scratch && n_words && offset && words, "nq_rans_compact: NULL buffer");
    NQ_CHECK_ARG((n_chunks + 3) / 4 < (1ll << 31), "nq_rans_compact: too many chunks");
    hipLaunchKernelGGL(rans_compact_kernel, dim3((uint32_t)((n_chunks + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       scratch, n_words, offset, n_chunks, chunk, words);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_rans_decode(const uint16_t* words, const uint64_t* offset, int64_t n, int32_t levels,
                              int32_t has_half, const uint16_t* freq, int32_t alphabet, int32_t chunk,
                              int8_t* codes, void* stream) {
    const int st = rans_check("nq_rans_decode", n, chunk, levels, has_half, freq, alphabet);
    if (st != NQ_OK) return st;
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    if (n_chunks == 0) return NQ_OK;
    NQ_CHECK_ARG(words && offset && codes, "nq_rans_decode: NULL buffer");
    NQ_CHECK_ARG(((uintptr_t)words & 7) == 0 && ((uintptr_t)codes & 15) == 0,
                 "nq_rans_decode: words must be 8-byte and codes 16-byte aligned");
    NQ_CHECK_ARG((n_chunks + 63) / 64 < (1ll << 31), "nq_rans_decode: too many chunks");
    RansArgs a = {};
    a.out_codes = codes;
    a.freq = freq;
    a.words = words;
    a.offset = offset;
    a.n = n;
    a.n_chunks = n_chunks;
    a.chunk = chunk;
    a.L = levels;
    a.has_half = has_half;
    a.alphabet = alphabet;
    hipLaunchKernelGGL(rans_decode_kernel, dim3((uint32_t)((n_chunks + 63) / 64)), dim3(64), 0,
                       (hipStream_t)stream, a);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
