// Keep-mask construction on gfx950: BOS + recent window + top-k of the
// evictable prefix + protected positions, and the ascending kept-index list.
//
// One 1024-thread block per batch row.  The row's order-preserving 32-bit keys
// are staged in LDS, 16384 positions per window (a row of at most one window
// is staged once; longer rows are re-staged per pass and window), with every
// thread's 16 loads in flight at once.  Thread t owns the 16 consecutive
// positions 16t .. 16t+15 of a window.
//  1. The k-th largest key of the prefix is found by an MSB-first radix select
//     (4 passes of 8 bits into a 256-bin LDS histogram); the bin holding it is
//     picked by one block scan of the bins in descending order.
//  2. One stable pass per window marks keys above the threshold and the first
//     (lowest-position) keys equal to it: a block scan of the threads' counts
//     of threshold-equal keys ranks them, and keeps the first `want`.
//  3. Protected positions are set in the window's LDS flags, which are then
//     written out and compacted into the kept-index list with one more block
//     scan: kept positions ascending from the front, evicted positions
//     descending from the back.
// Ties at the threshold therefore keep the lowest positions; torch.topk leaves
// their order unspecified.
#include "nq_common.h"

namespace nq {

constexpr int kSelThreads = 1024;
constexpr int kPer = 16;                   // consecutive positions per thread in a window
constexpr int kWin = kSelThreads * kPer;   // positions per LDS window

__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive block scan of one value per thread; returns the inclusive prefix
// and writes the block total to *total.  Uses lds[0 .. 1023 + 32].
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* lds, uint32_t* total) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    // wave-level inclusive scan with shuffles
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) lds[wave] = x;
    __syncthreads();
    if (t < 16) {
        uint32_t w = lds[t];
        uint32_t s = w;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            uint32_t y = __shfl_up(s, off, 64);
            if (t >= off) s += y;
        }
        lds[16 + t] = s - w;  // exclusive prefix of wave totals
        if (t == 15) lds[32] = s;
    }
    __syncthreads();
    uint32_t res = x + lds[16 + wave];
    *total = lds[32];
    __syncthreads();
    return res;
}

struct SelectArgs {
    const float* importance;  // [batch, seq]
    uint8_t* keep;            // [batch, seq]
    int32_t* kept_idx;        // [batch, seq] kept positions ascending, then evicted descending
    int32_t* n_kept;          // [batch]
    const int32_t* protected_pos;
    int32_t n_protected;
    int32_t seq, prefix, k, window;
};

__global__ __launch_bounds__(kSelThreads) void keep_mask_kernel(SelectArgs a) {
    __shared__ __align__(16) uint32_t s_key[kWin];   // order keys of one window
    __shared__ __align__(16) uint8_t s_keep[kWin];   // keep flags of one window
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scan_lds[64];
    __shared__ uint32_t sel[2];
    const int row = blockIdx.x;
    const int t = threadIdx.x;
    const float* imp = a.importance + (size_t)row * a.seq;
    const int lo = 1, hi = a.prefix;  // candidates: positions 1 .. prefix-1
    const int n_win = (a.seq + kWin - 1) / kWin;
    // keys of window w into s_key: coalesced loads, all of a thread's in flight
    auto stage = [&](int w) {
        const int base = w * kWin;
        uint32_t v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = base + j * kSelThreads + t;
            v[j] = i < a.seq ? order_key(imp[i]) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) s_key[j * kSelThreads + t] = v[j];
    };
    // this thread's 16 consecutive keys of the staged window
    auto my_keys = [&](uint32_t (&u)[kPer]) {
        const uint4* src = reinterpret_cast<const uint4*>(s_key + kPer * t);
#pragma unroll
        for (int q = 0; q < kPer / 4; ++q) {
            const uint4 x = src[q];
            u[4 * q] = x.x;
            u[4 * q + 1] = x.y;
            u[4 * q + 2] = x.z;
            u[4 * q + 3] = x.w;
        }
    };
    const bool staged = n_win == 1 && a.k > 0;  // one window: staged once for every pass
    if (staged) stage(0);
    uint32_t want = (uint32_t)a.k;
    uint32_t prefix_bits = 0, mask = 0;
    if (want > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            if (t < 256) hist[t] = 0;
            for (int w = 0; w < n_win; ++w) {
                if (!staged) {
                    __syncthreads();  // the previous window's keys are read
                    stage(w);
                }
                __syncthreads();  // keys staged, histogram cleared
                uint32_t u[kPer];
                my_keys(u);
                const int p0 = w * kWin + kPer * t;
#pragma unroll
                for (int j = 0; j < kPer; ++j) {
                    const int p = p0 + j;
                    if (p >= lo && p < hi && (u[j] & mask) == prefix_bits) atomicAdd(&hist[(u[j] >> shift) & 0xffu], 1u);
                }
            }
            __syncthreads();  // the pass's histogram is complete
            // bins from the top: the one where the running count reaches want
            // (unique: want >= 1 and the matching keys number at least want)
            const uint32_t h = t < 256 ? hist[255 - t] : 0u;
            uint32_t tot;
            const uint32_t incl = block_scan(h, scan_lds, &tot);
            if (t < 256 && incl >= want && incl - h < want) {
                sel[0] = 255u - (uint32_t)t;
                sel[1] = incl - h;
            }
            __syncthreads();
            want -= sel[1];
            prefix_bits |= sel[0] << shift;
            mask |= 0xffu << shift;
        }
    }
    // want = number of threshold-equal keys to keep (lowest positions first)
    const uint32_t thr = prefix_bits;
    const uint32_t take_eq = a.k > 0 ? want : 0u;
    uint32_t eq_before = 0, kept_before = 0;
    uint8_t* krow = a.keep + (size_t)row * a.seq;
    int32_t* idx = a.kept_idx + (size_t)row * a.seq;
    for (int w = 0; w < n_win; ++w) {
        const int base = w * kWin;
        if (a.k > 0 && !staged) {
            __syncthreads();
            stage(w);
        }
        __syncthreads();
        uint32_t u[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) u[j] = 0u;
        if (a.k > 0) my_keys(u);
        const int p0 = base + kPer * t;
        uint32_t eqm = 0, gtm = 0;  // this thread's threshold-equal / greater candidates
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int p = p0 + j;
            const bool cand = a.k > 0 && p >= lo && p < hi;
            if (cand && u[j] == thr) eqm |= 1u << j;
            if (cand && u[j] > thr) gtm |= 1u << j;
        }
        const uint32_t n_eq = (uint32_t)__builtin_popcount(eqm);
        uint32_t eq_tot;
        uint32_t rank = eq_before + block_scan(n_eq, scan_lds, &eq_tot) - n_eq;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int p = p0 + j;
            bool keep = p == 0 || (a.window > 0 && p >= a.seq - a.window) || ((gtm >> j) & 1u);
            if ((eqm >> j) & 1u) {
                keep = keep || rank < take_eq;
                ++rank;
            }
            s_keep[kPer * t + j] = (p < a.seq && keep) ? 1 : 0;
        }
        eq_before += eq_tot;
        __syncthreads();
        // protected positions never reduce the set
        for (int j = t; j < a.n_protected; j += kSelThreads) {
            const int p = a.protected_pos[j];
            if (p >= base && p < base + kWin && p < a.seq) s_keep[p - base] = 1;
        }
        __syncthreads();
        uint32_t km = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) km |= (uint32_t)(s_keep[kPer * t + j] != 0) << j;
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (p0 + j < a.seq) krow[p0 + j] = (uint8_t)((km >> j) & 1u);
        const uint32_t n_k = (uint32_t)__builtin_popcount(km);
        uint32_t k_tot;
        uint32_t out = kept_before + block_scan(n_k, scan_lds, &k_tot) - n_k;
        // kept positions ascending from the front; an evicted position p has
        // p - out evicted positions before it and goes to seq - 1 - (p - out),
        // so the evicted ones fill the tail descending
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int p = p0 + j;
            if ((km >> j) & 1u) idx[out++] = p;
            else if (p < a.seq) idx[a.seq - 1 - (p - (int)out)] = p;
        }
        kept_before += k_tot;
    }
    if (t == 0) a.n_kept[row] = (int32_t)kept_before;
}

}  // namespace nq

extern "C" int nq_keep_mask(const float* importance, int32_t batch, int32_t seq, int32_t sliding_window,
                            int32_t prefix, int32_t k, const int32_t* protected_pos, int32_t n_protected,
                            uint8_t* keep, int32_t* kept_idx, int32_t* n_kept, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(importance && keep && kept_idx && n_kept, "nq_keep_mask: NULL pointer");
    NQ_CHECK_ARG(batch > 0 && batch <= 65535 && seq >= 0, "nq_keep_mask: bad shape");
    NQ_CHECK_ARG(prefix >= 0 && prefix <= seq, "nq_keep_mask: prefix %d outside [0, %d]", prefix, seq);
    NQ_CHECK_ARG(k >= 0 && k <= (prefix > 1 ? prefix - 1 : 0), "nq_keep_mask: k %d exceeds the prefix", k);
    NQ_CHECK_ARG(sliding_window >= 0, "nq_keep_mask: negative window");
    NQ_CHECK_ARG(n_protected == 0 || protected_pos, "nq_keep_mask: protected list is NULL");
    if (seq == 0) return NQ_OK;
    SelectArgs a;
    a.importance = importance;
    a.keep = keep;
    a.kept_idx = kept_idx;
    a.n_kept = n_kept;
    a.protected_pos = protected_pos;
    a.n_protected = n_protected;
    a.seq = seq;
    a.prefix = prefix;
    a.k = k;
    a.window = sliding_window;
    hipLaunchKernelGGL(keep_mask_kernel, dim3(batch), dim3(kSelThreads), 0, (hipStream_t)stream, a);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
