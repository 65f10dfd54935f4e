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
#include <algorithm>

#include "nq_common.h"

namespace nq {

constexpr uint32_t kRansM = 1u << 12;
constexpr uint32_t kRansL = 1u << 16;
constexpr int kRansMaxAlpha = 64;

__device__ __forceinline__ int8_t rans_code(int s, int L, int has_half) {
    return (int8_t)(has_half ? s - L : 2 * (s - L / 2));
}

__device__ __forceinline__ int hist_bin(int8_t c, int L) {
    const int b = (int)c + L;
    return b < 0 ? 0 : (b > 2 * L ? 2 * L : b);  // codes outside [-L, L] are not valid input
}

// histogram of c + L over [0, 2L] (the host folds it when no code is odd).
// Lattice codes are peaked around 0, so a wave's 64 lanes mostly hit a few
// bins: each of 16 lane groups (lane % 16) counts into its own copy of the
// bins, so at most 4 lanes of a wave meet on one address.  Copy c's bin b is
// word c * hs + b, in bank (c * hs + b) mod 64.  With hs = 17 (17 bins, levels
// 8) the busy central bins of different copies fall in different banks; with
// hs = 65 (the earlier layout) copy c + 1's bin b - 1 shared copy c's bin b's
// bank, and one instruction's busiest bank held about 7 lanes instead of 4.
// Levels 16 (33 bins) keep hs = 65.  (One copy per lane measured the same.)
constexpr int kHistCopies = 16;
constexpr int kHistStride = kRansMaxAlpha + 1;

__global__ __launch_bounds__(256) void rans_hist_kernel(const int8_t* codes, int64_t n, int L, uint32_t* hist) {
    __shared__ uint32_t h_all[kHistCopies * kHistStride];
    for (int i = threadIdx.x; i < kHistCopies * kHistStride; i += 256) h_all[i] = 0;
    __syncthreads();
    const int hs = 2 * L + 1 <= 17 ? 17 : kHistStride;  // words between copies
    uint32_t* const h = h_all + (threadIdx.x & (kHistCopies - 1)) * hs;
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
    if (threadIdx.x <= 2 * L) {
        uint32_t t = 0;
#pragma unroll
        for (int c = 0; c < kHistCopies; ++c) t += h_all[c * hs + threadIdx.x];
        if (t) atomicAdd(&hist[threadIdx.x], t);
    }
}

// Histogram for alphabets of at most 9 bins (levels 2 and 4), without an
// atomic per code: each lane counts in one 64-bit register, 7 bits per bin
// (bin b at bit 7b), adding 1 << 7b per code, and empties it into 32-bit
// totals every 64 codes, before any 7-bit counter can pass 127.  The totals are
// summed across each wave and added once per wave and bin.  The per-code
// kernel above was bound by the LDS atomic rate, not by HBM.
constexpr int kHistSmallBins = 9;
constexpr int kHistSmallLoads = 4;  // 16-byte loads per lane in flight: 64 codes between flushes
                                    // (8 in flight, flushed every 4, measured the same)

__global__ __launch_bounds__(256) void rans_hist_small_kernel(const int8_t* codes, int64_t n, int L, uint32_t* hist) {
    __shared__ uint32_t h[kHistSmallBins];
    if (threadIdx.x < kHistSmallBins) h[threadIdx.x] = 0;
    __syncthreads();
    uint32_t tot[kHistSmallBins];
#pragma unroll
    for (int b = 0; b < kHistSmallBins; ++b) tot[b] = 0;
    const int bias = 7 * L;
    auto count16 = [&](const uint4& w, uint64_t& acc) {
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int c = (int)(ws[k] << (24 - 8 * j)) >> 24;
                c = min(max(c, -L), L);  // codes outside [-L, L] are not valid input
                acc += 1ull << (7 * c + bias);
            }
    };
    auto flush = [&](uint64_t acc) {
#pragma unroll
        for (int b = 0; b < kHistSmallBins; ++b) tot[b] += (uint32_t)(acc >> (7 * b)) & 127u;
    };
    const uint4* const v = reinterpret_cast<const uint4*>(codes);
    const int64_t n16 = n / 16;
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; g + (kHistSmallLoads - 1) * stride < n16; g += kHistSmallLoads * stride) {
        uint4 w[kHistSmallLoads];
#pragma unroll
        for (int u = 0; u < kHistSmallLoads; ++u) w[u] = v[g + u * stride];
        uint64_t acc = 0;
#pragma unroll
        for (int u = 0; u < kHistSmallLoads; ++u) count16(w[u], acc);
        flush(acc);
    }
    for (; g < n16; g += stride) {
        uint64_t acc = 0;
        count16(v[g], acc);
        flush(acc);
    }
    // the last n % 16 codes, one each to the first threads of block 0
    if (blockIdx.x == 0 && threadIdx.x < n - 16 * n16) {
        const int c = min(max((int)codes[16 * n16 + threadIdx.x], -L), L);
        flush(1ull << (7 * c + bias));
    }
#pragma unroll
    for (int b = 0; b < kHistSmallBins; ++b) {
        uint32_t t = tot[b];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
        if ((threadIdx.x & 63) == 0 && t) atomicAdd(&h[b], t);
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

// One lane per chunk, one wave per block (so the chunks spread over every CU).
// A chunk is a chain of dependent state updates: with few chunks the time is
// the chain's latency per symbol, with many (a whole role's codes as one
// stream) the instructions per symbol, so both the chain and the count are
// kept short.
//  - The codes of a whole chunk whose length is a multiple of 64 are read
//    64 at a time (four 16-byte loads per lane), one group ahead, from the
//    chunk's end backwards; other chunks read 16 at a time.
//  - The table is indexed by the raw code byte (256 entries, the symbol
//    mapping and its clamp folded in), so a lookup is one byte select and the
//    LDS reads; entries (f, cf, 1/f, and the renorm bound f * 2^20 - 1) are
//    looked up 8 codes ahead of the chain, so no LDS latency lies on it and
//    the lookahead costs 40 VGPRs (16 codes ahead took 80 and a wave of
//    occupancy).
//  - Emitted words go to a per-lane LDS ring (below) and leave in 32-byte
//    blocks; nothing inside a group of 64 waits on memory.
// Per-symbol encoder constants.  rcp is 1/f rounded up in fp64: for x < f 2^20
// it gives q = trunc(x * rcp) = floor(x / f) exactly (x * rcp exceeds x / f by
// at most 2^-32, less than the 1/f gap to the next integer, and the rounded
// product stays below it), so the update q M + (x - q f) + cf is
// q (M - f) + x + cf with a 24-bit multiply and no correction.
struct RansEnc {
    uint32_t xmax, mmf, cf;  // renorm bound f 2^20 - 1, M - f, cumulative frequency
    double rcp;
};
// In LDS the integer fields and 1/f sit in two arrays (16- and 8-byte
// entries): the code bytes in use (around 0 and 255) then fall in distinct
// banks, where 32-byte entries put bytes 8 apart on the same banks.
struct __attribute__((aligned(16))) RansEncInt {
    uint32_t xmax, mmf, cf, pad;
};

__device__ __forceinline__ double rcp_up(uint32_t f) {
    double r = 1.0 / (double)f;
    if (__builtin_fma(r, (double)f, -1.0) < 0.0) r = __longlong_as_double(__double_as_longlong(r) + 1);
    return r;
}

// Emitted words go to a per-lane ring of 32 words in LDS, written at the
// lane's current slot on every symbol and kept (the slot moves down) only when
// the step emitted one: no branch and no buffer shuffling per symbol.  After
// every 16 symbols a lane with 16 or more words pending stores the oldest 16
// (32 bytes, already in stream order) below its previous ones; at most 31 are
// ever pending, so the slot written next never holds an unstored word.
constexpr int kEncRingStride = 18;  // dwords per lane: 32 words + 8 bytes, 8-byte aligned rows
constexpr int64_t kEncWideChunks = 256 * 2 * 4 * 64;  // two 4-wave blocks per CU
constexpr int kEncGroup = 64;  // codes per load group of a whole chunk (read one group ahead)

// W waves per block share the byte table: one wave for streams of few chunks
// (so they spread over every CU), four when there are chunks for at least two
// such blocks per CU (LDS then holds more waves per CU).
template <int W>
__global__ __launch_bounds__(64 * W) void rans_encode_kernel(RansArgs a) {
    // the encoder constants of every code byte value: byte b (a signed code c)
    // codes symbol c + L, or c / 2 + L / 2 without half-integer points; bytes
    // outside [-L, L] (not valid input) take the nearest valid symbol, so any
    // byte stays inside the table
    __shared__ RansEncInt tab_i[256];
    __shared__ double tab_r[256];
    __shared__ uint32_t fcf[kRansMaxAlpha];  // f | cf << 16 per symbol
    __shared__ __align__(16) uint32_t ring_all[64 * W * kEncRingStride];
    if (threadIdx.x < 64) {
        // cumulative frequencies: an exclusive scan over the first wave (alphabet <= 64)
        const int t = threadIdx.x;
        const uint32_t f = t < a.alphabet ? a.freq[t] : 0u;
        uint32_t inc = f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_up(inc, o, 64);
            inc += t >= o ? v : 0u;
        }
        if (t < a.alphabet) fcf[t] = f | (inc - f) << 16;
    }
    __syncthreads();
    for (int b = threadIdx.x; b < 256; b += 64 * W) {
        const int c = (int)(int8_t)(uint8_t)b;
        const int sym = min(max(a.has_half ? c + a.L : (c >> 1) + a.L / 2, 0), a.alphabet - 1);
        const uint32_t f = fcf[sym] & 0xffffu, cf = fcf[sym] >> 16;
        RansEncInt e;
        // state >= f * 2^20 as a 32-bit test: f * 2^20 - 1 wraps to 2^32 - 1
        // at f = 4096 (never renormalise); f = 0 (not valid input) gives 0
        e.xmax = f ? (f << 20) - 1u : 0u;
        e.mmf = kRansM - f;
        e.cf = cf;
        e.pad = 0;
        tab_i[b] = e;
        tab_r[b] = f ? rcp_up(f) : 0.0;
    }
    __syncthreads();
    const int64_t ch = (int64_t)blockIdx.x * (64 * W) + threadIdx.x;
    if (ch >= a.n_chunks) return;
    const int64_t c0 = ch * a.chunk;
    const int64_t c1 = c0 + a.chunk < a.n ? c0 + a.chunk : a.n;
    uint16_t* const end = a.scratch + (ch + 1) * rans_stride(a.chunk);
    uint16_t* out = end;  // next 16-word block goes just below
    uint16_t* const ring = reinterpret_cast<uint16_t*>(ring_all + threadIdx.x * kEncRingStride);
    int wp = -1;  // the lane's next free slot (mod 32); counts down as words are emitted
    int fl = 0;   // slot one above the oldest pending word: slots wp + 1 .. fl - 1 are pending
    uint32_t state = kRansL;
    auto lookup = [&](uint32_t word, int k) -> RansEnc {
        const uint32_t b = (word >> (8 * k)) & 255u;
        const RansEncInt t = tab_i[b];
        return RansEnc{t.xmax, t.mmf, t.cf, tab_r[b]};
    };
    auto code_one = [&](const RansEnc& e) {
        // at most one word: state >> 16 < 2^16 <= f << 20
        const bool ren = state > e.xmax;
        // off the chain: the low word goes to the current slot, kept if emitted
        ring[wp & 31] = (uint16_t)state;
        wp -= ren ? 1 : 0;
        state = ren ? state >> 16 : state;
        const uint32_t q = (uint32_t)((double)state * e.rcp);  // floor(state / f), q < 2^20
        state = __umul24(q, e.mmf) + state + e.cf;             // q (M - f) < 2^32
    };
    // after 16 symbols: store the oldest 16 pending words (slots fl - 16 .. fl - 1,
    // ascending = stream order) below the stored ones
    auto flush16 = [&]() {
        if (fl - wp > 16) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(ring + ((fl - 16) & 31));
            uint2 w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) w[k] = *reinterpret_cast<const uint2*>(src + 2 * k);
            out -= 16;
#pragma unroll
            for (int k = 0; k < 4; ++k) *reinterpret_cast<uint2*>(out + 4 * k) = w[k];
            fl -= 16;
        }
    };
    // the 16 codes of one 16-byte block, highest first, 8 table entries at a time
    auto code16 = [&](uint4 v) {
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 1; h >= 0; --h) {
            RansEnc e[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) e[k] = lookup(wv[2 * h + (k >> 2)], k & 3);
#pragma unroll
            for (int k = 7; k >= 0; --k) code_one(e[k]);
        }
    };
    if (a.chunk % kEncGroup == 0 && c1 - c0 == a.chunk) {
        constexpr int G = kEncGroup / 16;  // 16-byte loads per group
        const uint4* p = reinterpret_cast<const uint4*>(a.codes + c0);
        int sb = a.chunk / kEncGroup - 1;
        uint4 cur[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            cur[j] = p[G * sb + j];
            // keeps the first group's loads apart from the loop's, so they are not
            // merged into one load at the loop top
            asm("" : "+v"(cur[j].x), "+v"(cur[j].y), "+v"(cur[j].z), "+v"(cur[j].w));
        }
        // table entries run 8 codes ahead of the chain: the entry of the code
        // 8 places later is looked up right after each code, where it fills the
        // chain's dependency stalls (e[k & 7] holds code k's entry when it is coded)
        RansEnc e[8];
        {
            const uint32_t wv[4] = {cur[G - 1].x, cur[G - 1].y, cur[G - 1].z, cur[G - 1].w};
#pragma unroll
            for (int k = 8; k < 16; ++k) e[k & 7] = lookup(wv[k >> 2], k & 3);
        }
        for (; sb >= 0; --sb) {
            const int nb = sb > 0 ? sb - 1 : 0;  // the last pass reloads group 0 (in bounds, unused)
            uint4 nxt[G];
#pragma unroll
            for (int j = 0; j < G; ++j) nxt[j] = p[G * nb + j];
#pragma unroll
            for (int j = G - 1; j >= 0; --j) {
                const uint32_t cw[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
                const uint4 nv = j > 0 ? cur[j - 1] : nxt[G - 1];
                const uint32_t nw[4] = {nv.x, nv.y, nv.z, nv.w};
#pragma unroll
                for (int k = 15; k >= 0; --k) {
                    code_one(e[k & 7]);
                    e[k & 7] = k >= 8 ? lookup(cw[(k - 8) >> 2], (k - 8) & 3) : lookup(nw[(k + 8) >> 2], (k + 8) & 3);
                }
                flush16();
            }
#pragma unroll
            for (int j = 0; j < G; ++j) cur[j] = nxt[j];
        }
    } else {
        // 16-byte blocks [b, b + 16) from the one holding c1 - 1 down to the one holding c0
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
        int64_t b = ((c1 - 1) / 16) * 16;
        uint4 cur = load_block(b);
        for (; b + 16 > c0; b -= 16) {
            const uint4 nxt = b - 16 >= 0 && b - 16 + 16 > c0 ? load_block(b - 16) : make_uint4(0u, 0u, 0u, 0u);
            const int k_hi = (int)((c1 - 1 < b + 15 ? c1 - 1 : b + 15) - b);
            const int k_lo = (int)((c0 > b ? c0 : b) - b);
            if (k_hi == 15 && k_lo == 0) {
                code16(cur);
            } else {
                const uint32_t wv[4] = {cur.x, cur.y, cur.z, cur.w};
                for (int k = k_hi; k >= k_lo; --k) code_one(lookup(wv[k >> 2], k & 3));
            }
            flush16();
            cur = nxt;
        }
    }
    // the final state, high word last (the decoder reads it first)
    ring[wp & 31] = (uint16_t)state;
    --wp;
    ring[wp & 31] = (uint16_t)(state >> 16);
    --wp;
    // the 0..17 pending words, just below the stored blocks in stream order
    const int pend = fl - wp - 1;
    for (int k = 0; k < pend; ++k) out[-1 - k] = ring[(fl - 1 - k) & 31];
    a.n_words[ch] = (uint32_t)(end - out) + (uint32_t)pend;
}

// copy each chunk's right-aligned words to its compacted offset.
// A wave takes `group` (<= 64) consecutive chunks: its lanes load their word
// counts and offsets, then their chunks' first and last words, and the wave
// copies the chunks one after the other, reading each chunk's count, offset and
// edge words back from its lane, so these cost two memory latencies per group,
// and a chunk's copy waits only on its own pair loads.  The waves
// stride over the groups with a grid the chip holds at once; the host shrinks
// the group until there are enough groups to give every wave one.
// Stores are 4-byte: a word before the destination's first 4-byte boundary and
// a last odd word go alone; the pairs between them come from aligned 4-byte
// source loads, funnel-shifted when source and destination differ in parity.
// Scratch rows span a multiple of 4 words, so every load stays in its row:
// with an odd source start the pair loads begin one word early, at or after the
// row's start, and the word count past the head is then odd, so they end on
// the row's last word.
constexpr uint32_t kCompactBlocks = 2048;  // 256 CUs x 8 blocks of 4 waves
constexpr int64_t kCompactWaves = 4 * (int64_t)kCompactBlocks;
constexpr int kCompactUnroll = 8;          // pairs per lane per piece: 1024 words, a 4096-code chunk at ~3 bits

__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)x, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
    return (uint64_t)hi << 32 | lo;
}

__global__ __launch_bounds__(256) void rans_compact_kernel(const uint16_t* scratch, const uint32_t* n_words,
                                                           const uint64_t* offset, int64_t n_chunks, int chunk,
                                                           int group, uint16_t* words) {
    const int lane = threadIdx.x & 63;
    const int64_t n_groups = (n_chunks + group - 1) / group;
    const int64_t stride = rans_stride(chunk);
    for (int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); g < n_groups; g += (int64_t)gridDim.x * 4) {
        const int64_t c0 = g * group;
        uint32_t my_nw = 0;
        uint64_t my_off = 0;
        if (lane < group && c0 + lane < n_chunks) {
            my_nw = n_words[c0 + lane];
            my_off = offset[c0 + lane];
        }
        // each lane's chunk's first and last words, for a lone head or tail store
        uint32_t my_edge = 0;
        if (my_nw) {
            const int64_t s0 = (c0 + lane + 1) * stride - my_nw;
            my_edge = (uint32_t)scratch[s0] | (uint32_t)scratch[s0 + my_nw - 1] << 16;
        }
        // wait here, once per group: past the loop's stores the compiler
        // can no longer count these loads and would wait on every store
        __builtin_amdgcn_s_waitcnt(0);
        const int cnt = (int)(n_chunks - c0 < group ? n_chunks - c0 : group);
        for (int c = 0; c < cnt; ++c) {
            const uint32_t nw = (uint32_t)__builtin_amdgcn_readlane((int)my_nw, c);
            if (nw == 0) continue;
            const uint64_t dst0 = readlane_u64(my_off, c);
            const int64_t src0 = (c0 + c + 1) * stride - nw;
            const uint32_t head = (uint32_t)(dst0 & 1);
            const uint32_t pairs = (nw - head) >> 1;
            const uint32_t tail = (nw - head) & 1;
            const uint32_t edge = (uint32_t)__builtin_amdgcn_readlane((int)my_edge, c);
            const int64_t q0 = src0 + head;  // source word of the first pair
            const uint32_t sh = (uint32_t)(q0 & 1);
            const uint32_t* s32 = reinterpret_cast<const uint32_t*>(scratch + (q0 & ~(int64_t)1));
            uint32_t* d32 = reinterpret_cast<uint32_t*>(words + dst0 + head);
            // all of a piece's loads go out before its stores; loads past the
            // last pair repeat the last pair's, so none is conditional
            for (uint32_t b = 0; b < pairs; b += 64 * kCompactUnroll) {
                uint32_t v[kCompactUnroll];
#pragma unroll
                for (int j = 0; j < kCompactUnroll; ++j) {
                    const uint32_t i = min(b + lane + 64 * j, pairs - 1);
                    const uint32_t lo = s32[i], hi = s32[i + sh];
                    v[j] = __builtin_amdgcn_alignbit(hi, lo, 16 * sh);  // lo when sh = 0
                }
#pragma unroll
                for (int j = 0; j < kCompactUnroll; ++j) {
                    const uint32_t i = b + lane + 64 * j;
                    if (i < pairs) d32[i] = v[j];
                }
            }
            if (lane == 0 && head) words[dst0] = (uint16_t)edge;
            if (lane == 1 && tail) words[dst0 + nw - 1] = (uint16_t)(edge >> 16);
        }
    }
}

// One lane per chunk, one wave per block.  Two 4096-entry LDS tables map a
// slot to f[s] | (slot - cf[s]) << 13 and to the code byte of its symbol s.  A
// symbol needs at most one word (the state is >= 16 before renormalisation).
// The chain per symbol is one table read and a multiply-add; everything else
// is kept off it:
//  - each lane's stream words pass through a private 64-word ring in LDS.  At
//    the start of every 16 symbols a lane writes the words it loaded one
//    step earlier and, if fewer than 32 unread words remain, loads the next
//    batch (16 words in one-wave blocks, 32 in the wide blocks, which then
//    load half as often), so no load is waited on inside a step and the ring
//    always holds the (at most 16) words a step reads.  A wave whose lanes can
//    only reach words inside the stream loads without the end-of-stream test,
//    on a branch the whole wave takes;
//  - the word a renormalisation would take is read from the ring alongside
//    the table entry, before it is known to be needed;
//  - 16 decoded codes leave in one 16-byte store, issued a step late and after
//    that step's loads, so that the next wait on loads does not also wait for
//    it.
constexpr int kRingStride = 34;  // dwords per lane: 64 words + 4 bytes, 8-byte aligned rows
// the ring is written in 8-byte groups and read in 16-bit words: both through
// may_alias types, so the compiler keeps every read after the writes it follows
typedef uint16_t __attribute__((may_alias)) ring_word_t;
typedef uint64_t __attribute__((may_alias)) ring_group_t;

// W waves per block share the slot tables.  The tables and one wave's rings
// take 20.6 KB and 8.7 KB of LDS, so one-wave blocks fit 5 to a CU; a long
// stream's chains (more than the chip holds at once) run in blocks of 6 waves,
// 2 to a CU, 12 waves in all.  A short stream keeps one wave per block, so its
// few chains spread over every CU.
constexpr int kDecodeWaves = 6;

template <int W>
__global__ __launch_bounds__(64 * W) void rans_decode_kernel(RansArgs a) {
    __shared__ uint32_t tab[kRansM];
    __shared__ uint8_t code_of[kRansM];
    __shared__ uint16_t cf[kRansMaxAlpha + 1];
    __shared__ __attribute__((aligned(8))) uint32_t ring_all[64 * W * kRingStride];
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
        const uint8_t code = (uint8_t)rans_code(s, a.L, a.has_half);
        const uint32_t f = hi > lo ? hi - lo : 1u;  // f <= 4096: 13 bits
        for (uint32_t k = lo + threadIdx.x; k < hi; k += 64 * W) {
            tab[k] = f | ((k - lo) << 13);
            code_of[k] = code;
        }
    }
    __syncthreads();
    const int64_t ch = (int64_t)blockIdx.x * (64 * W) + threadIdx.x;
    if (ch >= a.n_chunks) return;  // no barrier follows
    const int64_t c0 = ch * a.chunk;
    const uint32_t n_sym = (uint32_t)((c0 + a.chunk < a.n ? c0 + a.chunk : a.n) - c0);
    const uint64_t w0 = a.offset[ch];
    const uint32_t len = (uint32_t)(a.offset[ch + 1] - w0);
    const uint64_t total = a.offset[a.n_chunks];
    // words are numbered from g0, the 4-aligned word at or below the chunk's
    // first; 4-word group k holds words 4k .. 4k + 3 and sits in ring slots
    // 4 (k % 16) ..
    const uint64_t g0 = w0 & ~(uint64_t)3;
    uint32_t* const ring = ring_all + threadIdx.x * kRingStride;
    const ring_word_t* const ring16 = reinterpret_cast<const ring_word_t*>(ring);
    auto load_group = [&](uint32_t k) -> uint64_t {  // groups past the stream's end read as 0
        const uint64_t g = g0 + 4ull * k;
        if (g + 4 <= total) return *reinterpret_cast<const uint64_t*>(a.words + g);
        uint64_t v = 0;
        for (uint64_t j = 0; g + j < total; ++j) v |= (uint64_t)a.words[g + j] << (16 * j);
        return v;
    };
    // Words this lane can load: rpos never passes the chunk's end (renormalising
    // stops there) nor 2 + n_sym, and a batch is loaded only while fewer than 32
    // words are unread, so every load stays below g0 + rmax + 32 + kBatch (and
    // the first 32 words).  A wave all of whose lanes stay inside the stream
    // skips the per-group end test.
    constexpr uint32_t kBatch = W > 1 ? 32 : 16;  // words per prefetch
    const uint32_t rmax = (uint32_t)(w0 & 3) + (len < n_sym + 2 ? len : n_sym + 2);
    const uint64_t lane_end = g0 + (rmax + 32 + kBatch > 32 ? rmax + 32 + kBatch : 32);
    const bool wave_inside = __builtin_amdgcn_ballot_w64(lane_end > total) == 0;
    auto put_group = [&](uint32_t k, uint64_t v) { *reinterpret_cast<ring_group_t*>(ring + 2 * (k & 15u)) = v; };
    uint32_t written = 8;  // groups in the ring: the first 8, all loads issued before the first write
    {
        uint64_t first[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) first[k] = load_group(k);
#pragma unroll
        for (int k = 0; k < 8; ++k) put_group(k, first[k]);
    }
    uint32_t rpos = (uint32_t)(w0 & 3);   // next word to read
    const uint32_t rend = rpos + len;     // one past the chunk's last word
    uint32_t state = kRansL;
    if (len >= 2) {
        state = ((uint32_t)ring16[rpos] << 16) | ring16[rpos + 1];
        rpos += 2;
    }
    uint32_t nw = ring16[rpos & 63u];  // the word a renormalisation takes next
    // renormalise below lim: 2^16 while the chunk has words left, else never
    uint32_t lim = rpos < rend ? kRansL : 0u;
    // opaque to the compiler, which would otherwise split state < lim back into
    // two tests joined by a scalar AND on the chain
    auto set_lim = [&]() {
        lim = rpos < rend ? kRansL : 0u;
        asm("" : "+v"(lim));
    };
    auto step = [&]() -> uint32_t {
        const uint32_t slot = state & (kRansM - 1u);
        const uint32_t e = tab[slot];
        const uint32_t code = code_of[slot];
        state = __umul24(e & 0x1fffu, state >> 12) + (e >> 13);  // f (state >> 12) + slot - cf
        const bool need = state < lim;
        state = need ? (state << 16) | nw : state;
        rpos += need ? 1u : 0u;
        set_lim();
        nw = ring16[rpos & 63u];
        return code;
    };
    constexpr int PG = kBatch / 4;
    uint64_t pf[PG];       // groups loaded for the next step
    bool inflight = false;
    auto refill = [&]() {
        if (inflight) {
#pragma unroll
            for (int j = 0; j < PG; ++j) put_group(written + j, pf[j]);
            written += PG;
            inflight = false;
            nw = ring16[rpos & 63u];  // its slot may have just been written
        }
    };
    auto prefetch = [&]() {
        if (4 * written - rpos < 32) {
            if (wave_inside) {
#pragma unroll
                for (int j = 0; j < PG; ++j)
                    pf[j] = *reinterpret_cast<const uint64_t*>(a.words + g0 + 4ull * (written + j));
            } else {
#pragma unroll
                for (int j = 0; j < PG; ++j) pf[j] = load_group(written + j);
            }
            inflight = true;
        }
    };
    int8_t* out = a.out_codes + c0;
    uint32_t i = 0;
    if ((((uintptr_t)out) & 15) == 0) {
        uint4 prev = make_uint4(0u, 0u, 0u, 0u);
        for (; i + 16 <= n_sym; i += 16) {
            refill();
            prefetch();
            if (i) *reinterpret_cast<uint4*>(out + i - 16) = prev;
            uint32_t ob[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t v = step();
                v |= step() << 8;
                v |= step() << 16;
                v |= step() << 24;
                ob[q] = v;
            }
            prev = make_uint4(ob[0], ob[1], ob[2], ob[3]);
        }
        if (i) *reinterpret_cast<uint4*>(out + i - 16) = prev;
    }
    // the rest one code at a time; every 16 codes the ring is topped up to at
    // least 16 unread words first
    for (; i < n_sym; ++i) {
        if ((i & 15u) == 0) {
            refill();
            if (4 * written - rpos < 16) {
                prefetch();
                refill();
            }
        }
        out[i] = (int8_t)step();
    }
}

// Chunk offsets = exclusive prefix sums of the word counts, in three launches
// over segments of kScanSeg = 1024 x kScanPer counts (one 1024-thread block
// each, every thread owning kScanPer consecutive counts): pass 1 sums each
// segment, pass 2 (one block) scans the segment sums into segment bases, and
// pass 3 scans within each segment from its base.  No workspace: a segment's
// total, and then its base, live in offset[first chunk of the segment] until
// the last pass reads that slot and overwrites it with the chunk's own offset.
constexpr int kScanPer = 4;                                   // counts per thread
constexpr int64_t kScanSeg = 1024 * (int64_t)kScanPer;        // counts per segment (one block)

// inclusive scan of one value per thread of a 1024-thread block; *total gets
// the block's sum.  Uses lds[0 .. 32].
__device__ __forceinline__ uint64_t block_incl_scan(uint64_t v, uint64_t* lds, uint64_t* total) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint64_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) lds[wave] = x;
    __syncthreads();
    if (t < 16) {
        const uint64_t w = lds[t];
        uint64_t r = w;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const uint64_t y = __shfl_up(r, o, 64);
            if (t >= o) r += y;
        }
        lds[16 + t] = r - w;
        if (t == 15) lds[32] = r;
    }
    __syncthreads();
    const uint64_t res = x + lds[16 + wave];
    *total = lds[32];
    __syncthreads();
    return res;
}

// pass 1: each segment's total into offset[its first chunk]
__global__ __launch_bounds__(1024) void rans_seg_sum_kernel(const uint32_t* n_words, int64_t n_chunks,
                                                            uint64_t* offset) {
    __shared__ uint64_t lds[33];
    const int64_t seg0 = (int64_t)blockIdx.x * kScanSeg;
    uint64_t sum = 0;
#pragma unroll 4
    for (int k = 0; k < kScanPer; ++k) {
        const int64_t i = seg0 + (int64_t)k * 1024 + threadIdx.x;
        if (i < n_chunks) sum += n_words[i];
    }
    uint64_t tot;
    (void)block_incl_scan(sum, lds, &tot);
    if (threadIdx.x == 0) offset[seg0] = tot;
}

// pass 2 (one block): the segment totals into exclusive bases, in place, and
// the stream's word count into offset[n_chunks]
__global__ __launch_bounds__(1024) void rans_seg_base_kernel(int64_t n_chunks, uint64_t* offset) {
    __shared__ uint64_t lds[33];
    const int64_t n_seg = (n_chunks + kScanSeg - 1) / kScanSeg;
    uint64_t carry = 0;
    for (int64_t b0 = 0; b0 < n_seg; b0 += 1024) {
        const int64_t b = b0 + threadIdx.x;
        const uint64_t v = b < n_seg ? offset[b * kScanSeg] : 0;
        uint64_t tot;
        const uint64_t incl = block_incl_scan(v, lds, &tot);
        if (b < n_seg) offset[b * kScanSeg] = carry + incl - v;
        carry += tot;
    }
    if (threadIdx.x == 0) offset[n_chunks] = carry;
}

// pass 3: thread t of segment b writes the offsets of its kScanPer consecutive chunks
__global__ __launch_bounds__(1024) void rans_seg_scan_kernel(const uint32_t* n_words, int64_t n_chunks,
                                                             uint64_t* offset) {
    __shared__ uint64_t lds[33];
    __shared__ uint64_t s_base;
    const int64_t seg0 = (int64_t)blockIdx.x * kScanSeg;
    if (threadIdx.x == 0) s_base = offset[seg0];
    const int64_t i0 = seg0 + (int64_t)threadIdx.x * kScanPer;
    uint32_t cnt[kScanPer];
    if (i0 + kScanPer <= n_chunks && ((reinterpret_cast<uintptr_t>(n_words + i0) & 15) == 0)) {
#pragma unroll
        for (int k = 0; k < kScanPer; k += 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(n_words + i0 + k);
            cnt[k] = v.x;
            cnt[k + 1] = v.y;
            cnt[k + 2] = v.z;
            cnt[k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) cnt[k] = i0 + k < n_chunks ? n_words[i0 + k] : 0u;
    }
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanPer; ++k) sum += cnt[k];
    uint64_t tot;
    const uint64_t incl = block_incl_scan(sum, lds, &tot);  // its barriers order s_base before the writes
    uint64_t run = s_base + incl - sum;
#pragma unroll
    for (int k = 0; k < kScanPer; ++k) {
        if (i0 + k < n_chunks) offset[i0 + k] = run;
        run += cnt[k];
    }
}

}  // namespace nq

using namespace nq;

extern "C" int nq_rans_histogram(const int8_t* codes, int64_t n, int32_t levels, uint32_t* hist, void* stream) {
    NQ_CHECK_ARG(levels == 2 || levels == 4 || levels == 8 || levels == 16,
                 "nq_rans_histogram: levels must be 2, 4, 8 or 16 (got %d)", levels);
    NQ_CHECK_ARG(n >= 0 && (n == 0 || (codes && hist)), "nq_rans_histogram: bad arguments");
    NQ_CHECK_ARG(n <= (int64_t)0xffffffffll,
                 "nq_rans_histogram: %lld codes in one call; the uint32 bins take at most 2^32 - 1 (count in pieces)",
                 (long long)n);
    NQ_CHECK_ARG(((uintptr_t)codes & 15) == 0, "nq_rans_histogram: codes must be 16-byte aligned");
    if (n == 0) return NQ_OK;
    int64_t blocks = (n + 256 * 16 - 1) / (256 * 16);
    if (blocks > 4096) blocks = 4096;
    if (2 * levels + 1 <= kHistSmallBins)
        hipLaunchKernelGGL(rans_hist_small_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, codes, n,
                           levels, hist);
    else
        hipLaunchKernelGGL(rans_hist_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, codes, n,
                           levels, hist);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

static int rans_check(const char* who, int64_t n, int32_t chunk, int32_t levels, int32_t has_half,
                      const uint16_t* freq, int32_t alphabet) {
    NQ_CHECK_ARG(levels == 2 || levels == 4 || levels == 8 || levels == 16, "%s: levels must be 2, 4, 8 or 16", who);
    NQ_CHECK_ARG(alphabet == (has_half ? 2 * levels + 1 : levels + 1), "%s: alphabet %d does not match levels %d%s",
                 who, alphabet, levels, has_half ? " (half-integer codes)" : "");
    // chunk is at most INT32_MAX by its type: the encoder's and decoder's
    // per-chunk counters (word counts, ring positions) are 32-bit unsigned and
    // stay below 2^32 for chunk + 64 words
    NQ_CHECK_ARG(chunk >= 1, "%s: chunk %d out of range", who, chunk);
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
        if (n_chunks >= kEncWideChunks)
            hipLaunchKernelGGL(rans_encode_kernel<4>, dim3((uint32_t)((n_chunks + 255) / 256)), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(rans_encode_kernel<1>, dim3((uint32_t)((n_chunks + 63) / 64)), dim3(64), 0, s, a);
        const uint32_t n_seg = (uint32_t)((n_chunks + kScanSeg - 1) / kScanSeg);
        hipLaunchKernelGGL(rans_seg_sum_kernel, dim3(n_seg), dim3(1024), 0, s, n_words, n_chunks, offset);
        hipLaunchKernelGGL(rans_seg_base_kernel, dim3(1), dim3(1024), 0, s, n_chunks, offset);
        hipLaunchKernelGGL(rans_seg_scan_kernel, dim3(n_seg), dim3(1024), 0, s, n_words, n_chunks, offset);
    } else if (offset) {
        hipLaunchKernelGGL(rans_seg_base_kernel, dim3(1), dim3(1024), 0, s, n_chunks, offset);  // offset[0] = 0
    }
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}

extern "C" int nq_rans_compact(const uint16_t* scratch, const uint32_t* n_words, const uint64_t* offset,
                               int64_t n, int32_t chunk, uint16_t* words, void* stream) {
    NQ_CHECK_ARG(chunk >= 1 && n >= 0, "nq_rans_compact: bad arguments");
    const int64_t n_chunks = (n + chunk - 1) / chunk;
    if (n_chunks == 0) return NQ_OK;
    NQ_CHECK_ARG(scratch && n_words && offset && words, "nq_rans_compact: NULL buffer");
    NQ_CHECK_ARG(((uintptr_t)scratch & 7) == 0 && ((uintptr_t)words & 3) == 0,
                 "nq_rans_compact: scratch must be 8-byte and words 4-byte aligned");
    int group = 64;
    while (group > 1 && n_chunks < group * kCompactWaves) group >>= 1;
    const int64_t n_groups = (n_chunks + group - 1) / group;
    const uint32_t blocks = (uint32_t)std::min<int64_t>((n_groups + 3) / 4, kCompactBlocks);
    hipLaunchKernelGGL(rans_compact_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, scratch, n_words,
                       offset, n_chunks, chunk, group, words);
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
    if (n_chunks >= (int64_t)64 * kDecodeWaves * 2 * 256)  // two blocks for each of 256 CUs
        hipLaunchKernelGGL(rans_decode_kernel<kDecodeWaves>,
                           dim3((uint32_t)((n_chunks + 64 * kDecodeWaves - 1) / (64 * kDecodeWaves))),
                           dim3(64 * kDecodeWaves), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(rans_decode_kernel<1>, dim3((uint32_t)((n_chunks + 63) / 64)), dim3(64), 0,
                           (hipStream_t)stream, a);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
