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
    uint16_t* scratch;       // [n_chunks][chunk + 2] words, each chunk's stream right-aligned
    uint32_t* n_words;       // [n_chunks]
    const uint64_t* offset;  // [n_chunks + 1] word offsets in the compacted stream (decode)
    const uint16_t* words;   // compacted stream (decode)
    int64_t n;
    int64_t n_chunks;
    int chunk, L, has_half, alphabet;
};

__device__ __forceinline__ void rans_tables(const RansArgs& a, uint16_t* f, uint16_t* cf) {
    if (threadIdx.x == 0) {
        uint32_t acc = 0;
        for (int s = 0; s < a.alphabet; ++s) {
            f[s] = a.freq[s];
            cf[s] = (uint16_t)acc;
            acc += a.freq[s];
        }
        cf[a.alphabet] = (uint16_t)acc;
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void rans_encode_kernel(RansArgs a) {
    __shared__ uint16_t f[kRansMaxAlpha], cf[kRansMaxAlpha + 1];
    rans_tables(a, f, cf);
    const int64_t ch = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (ch >= a.n_chunks) return;
    const int64_t c0 = ch * a.chunk;
    const int64_t c1 = c0 + a.chunk < a.n ? c0 + a.chunk : a.n;
    uint16_t* end = a.scratch + ch * (int64_t)(a.chunk + 2) + (a.chunk + 2);
    uint16_t* out = end;
    uint32_t state = kRansL;
    for (int64_t i = c1 - 1; i >= c0; --i) {
        int s = rans_symbol(a.codes[i], a.L, a.has_half);
        s = s < 0 ? 0 : (s >= a.alphabet ? a.alphabet - 1 : s);  // codes outside [-L, L] are not valid input
        const uint32_t fs = f[s], cs = cf[s];
        if ((uint64_t)state >= ((uint64_t)fs << 20)) {  // at most one word: state >> 16 < 2^16 <= fs << 20
            *--out = (uint16_t)(state & 0xffffu);
            state >>= 16;
        }
        state = (state / fs) * kRansM + (state % fs) + cs;
    }
    *--out = (uint16_t)(state & 0xffffu);
    *--out = (uint16_t)(state >> 16);
    a.n_words[ch] = (uint32_t)(end - out);
}

// copy each chunk's right-aligned words to its compacted offset; one wave per chunk
__global__ __launch_bounds__(256) void rans_compact_kernel(const uint16_t* scratch, const uint32_t* n_words,
                                                           const uint64_t* offset, int64_t n_chunks, int chunk,
                                                           uint16_t* words) {
    const int64_t ch = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (ch >= n_chunks) return;
    const int lane = threadIdx.x & 63;
    const uint32_t nw = n_words[ch];
    const uint16_t* src = scratch + ch * (int64_t)(chunk + 2) + (chunk + 2) - nw;
    uint16_t* dst = words + offset[ch];
    for (uint32_t i = lane; i < nw; i += 64) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void rans_decode_kernel(RansArgs a) {
    __shared__ uint16_t f[kRansMaxAlpha], cf[kRansMaxAlpha + 1];
    __shared__ uint8_t c2s[kRansM];
    rans_tables(a, f, cf);
    for (int s = 0; s < a.alphabet; ++s)
        for (uint32_t k = cf[s] + threadIdx.x; k < cf[s + 1]; k += 256) c2s[k] = (uint8_t)s;
    __syncthreads();
    const int64_t ch = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (ch >= a.n_chunks) return;
    const int64_t c0 = ch * a.chunk;
    const int64_t c1 = c0 + a.chunk < a.n ? c0 + a.chunk : a.n;
    const uint16_t* w = a.words + a.offset[ch];
    const uint64_t len = a.offset[ch + 1] - a.offset[ch];
    uint64_t pos = 2;
    uint32_t state = len >= 2 ? ((uint32_t)w[0] << 16) | w[1] : kRansL;
    for (int64_t i = c0; i < c1; ++i) {
        const uint32_t slot = state & (kRansM - 1u);
        const int s = c2s[slot];
        state = (uint32_t)f[s] * (state >> 12) + slot - cf[s];
        while (state < kRansL && pos < len) state = (state << 16) | w[pos++];
        a.out_codes[i] = rans_code(s, a.L, a.has_half);
    }
}

// exclusive scan of n_words into offset[0..n_chunks] (one block, chunked)
__global__ __launch_bounds__(1024) void rans_scan_kernel(const uint32_t* n_words, int64_t n_chunks, uint64_t* offset) {
    __shared__ uint64_t s[1024];
    uint64_t carry = 0;
    for (int64_t b0 = 0; b0 < n_chunks; b0 += 1024) {
        const int64_t i = b0 + threadIdx.x;
        const uint64_t v = i < n_chunks ? n_words[i] : 0;
        s[threadIdx.x] = v;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const uint64_t add = threadIdx.x >= (unsigned)o ? s[threadIdx.x - o] : 0;
            __syncthreads();
            s[threadIdx.x] += add;
            __syncthreads();
        }
        if (i < n_chunks) offset[i] = carry + s[threadIdx.x] - v;
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
    return (n + chunk - 1) / chunk * (int64_t)(chunk + 2);
}

extern "C" int nq_rans_encode(const int8_t* codes, int64_t n, int32_t levels, int32_t has_half, const uint16_t* freq,
                              int32_t alphabet, int32_t chunk, uint16_t* scratch, uint32_t* n_words,
                              uint64_t* offset, void* stream) {
    const int st = rans_check("nq_rans_encode", n, chunk, levels, has_half, freq, alphabet);
    if (st != NQ_OK) return st;
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    NQ_CHECK_ARG(n == 0 || (codes && scratch && n_words && offset), "nq_rans_encode: NULL buffer");
    NQ_CHECK_ARG((n_chunks + 255) / 256 < (1ll << 31), "nq_rans_encode: too many chunks");
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
        hipLaunchKernelGGL(rans_encode_kernel, dim3((uint32_t)((n_chunks + 255) / 256)), dim3(256), 0, s, a);
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
    NQ_CHECK_ARG((n_chunks + 255) / 256 < (1ll << 31), "nq_rans_decode: too many chunks");
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
    hipLaunchKernelGGL(rans_decode_kernel, dim3((uint32_t)((n_chunks + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
