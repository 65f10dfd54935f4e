// Keep-mask construction on gfx950: BOS + recent window + top-k of the
// evictable prefix + protected positions, and the ascending kept-index list.
//
// One 1024-thread block per batch row.  The k-th largest importance of the
// prefix is found by an MSB-first radix select over order-preserving 32-bit
// keys (4 passes of 8 bits, 256-bin LDS histograms, the row read from global
// memory each pass), then one stable pass marks keys above the threshold and
// the first (lowest-index) keys equal to it, and compacts the kept indices
// with a block prefix sum.  Ties at the threshold therefore keep the lowest
// positions; torch.topk leaves their order unspecified.
#include "nq_common.h"

namespace nq {

constexpr int kSelThreads = 1024;

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
    int32_t* kept_idx;        // [batch, seq] ascending kept positions (rest untouched)
    int32_t* n_kept;          // [batch]
    const int32_t* protected_pos;
    int32_t n_protected;
    int32_t seq, prefix, k, window;
};

__global__ __launch_bounds__(kSelThreads) void keep_mask_kernel(SelectArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scan_lds[64];
    __shared__ uint32_t sel[4];
    const int row = blockIdx.x;
    const int t = threadIdx.x;
    const float* imp = a.importance + (size_t)row * a.seq;
    // candidates: positions 1 .. prefix-1
    const int lo = 1, hi = a.prefix;
    uint32_t want = (uint32_t)a.k;
    uint32_t prefix_bits = 0, mask = 0;
    if (want > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = t; i < 256; i += kSelThreads) hist[i] = 0;
            __syncthreads();
            for (int i = lo + t; i < hi; i += kSelThreads) {
                uint32_t u = order_key(imp[i]);
                if ((u & mask) == prefix_bits) atomicAdd(&hist[(u >> shift) & 0xffu], 1u);
            }
            __syncthreads();
            if (t == 0) {
                uint32_t acc = 0;
                int b = 255;
                for (; b > 0; --b) {
                    if (acc + hist[b] >= want) break;
                    acc += hist[b];
                }
                sel[0] = (uint32_t)b;
                sel[1] = acc;
            }
            __syncthreads();
            want -= sel[1];
            prefix_bits |= sel[0] << shift;
            mask |= 0xffu << shift;
            __syncthreads();
        }
    }
    // want = number of threshold-equal keys to keep (lowest positions first)
    const uint32_t thr = prefix_bits;
    const uint32_t take_eq = (a.k > 0) ? want : 0u;
    uint32_t eq_before = 0, kept_before = 0;
    for (int base = 0; base < a.seq; base += kSelThreads) {
        const int i = base + t;
        bool valid = i < a.seq;
        bool cand = valid && i >= lo && i < hi && a.k > 0;
        uint32_t u = cand ? order_key(imp[i]) : 0u;
        uint32_t is_eq = (cand && u == thr) ? 1u : 0u;
        uint32_t eq_total;
        uint32_t eq_incl = block_scan(is_eq, scan_lds, &eq_total);
        bool keep = false;
        if (valid) {
            keep = (i == 0) || (a.window > 0 && i >= a.seq - a.window);
            if (cand && u > thr) keep = true;
            if (is_eq && (eq_before + eq_incl - 1u) < take_eq) keep = true;
        }
        eq_before += eq_total;
        if (valid) a.keep[(size_t)row * a.seq + i] = keep ? 1 : 0;
        __syncthreads();
    }
    // Protected positions (after the stable pass; they never reduce the set).
    // The keep bytes are re-read below by other waves of the block: the device
    // scope fences make the stores complete and visible before the barrier.
    __threadfence();
    __syncthreads();
    for (int j = t; j < a.n_protected; j += kSelThreads) {
        int p = a.protected_pos[j];
        if (p >= 0 && p < a.seq) a.keep[(size_t)row * a.seq + p] = 1;
    }
    __threadfence();
    __syncthreads();
    for (int base = 0; base < a.seq; base += kSelThreads) {
        const int i = base + t;
        uint32_t kv = (i < a.seq && a.keep[(size_t)row * a.seq + i]) ? 1u : 0u;
        uint32_t tot;
        uint32_t incl = block_scan(kv, scan_lds, &tot);
        if (kv) a.kept_idx[(size_t)row * a.seq + kept_before + incl - 1u] = i;
        kept_before += tot;
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
