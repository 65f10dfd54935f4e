// Merge eviction on gfx950: before hard eviction, every evicted token's
// value is added into its most similar surviving token, weighted by
// importance.  Steps, per batch row:
//  1. centroids c[t] = (sum over layers of mean over heads of v[l, h, t, :]) /
//     n_layers in fp32, in the reference's reduction order: heads summed in
//     runs of 16 from zero, runs added in order, divided by the head count;
//     layers added in order, divided by the layer count;
//  2. unit vectors c / max(|c|, 1e-12);
//  3. for each evicted token the kept token of largest cosine (first on ties),
//     tiled 64 x 64 in LDS over (evicted, kept) with the kept range split
//     across blocks, then reduced over the splits in order;
//  4. weights w = fp32(imp_e / (imp_s + imp_e + 1e-8)) in double, and per
//     survivor the list of its evicted tokens in ascending order (a stable
//     bucket fill run by one block per row);
//  5. per layer, head and survivor: v_s = fl(v_s + fl(w_e * v_e)) over its list
//     in order, rounded once to the cache type; every other row is copied.
#include "nq_rowmath.h"

namespace nq {

constexpr int kMT = 64;     // tile rows (evicted) and columns (kept)
constexpr int kMPad = 4;    // LDS row padding (floats)

typedef float f32x16v __attribute__((ext_vector_type(16)));

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, size_t i) {
    if constexpr (DT == NQ_F32) return static_cast<const float*>(p)[i];
    else if constexpr (DT == NQ_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    else return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, size_t i, float v) {
    if constexpr (DT == NQ_F32) {
        static_cast<float*>(p)[i] = v;
    } else if constexpr (DT == NQ_BF16) {
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        uint32_t r;
        if ((u & 0x7f800000u) == 0x7f800000u) r = (u >> 16) | ((u & 0xffffu) ? 0x40u : 0u);  // inf / nan
        else r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
        static_cast<uint16_t*>(p)[i] = (uint16_t)r;
    } else {
        static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_f16_bits(v);
    }
}

// 8 consecutive elements <-> fp32 (16-byte loads for fp16 / bf16, 2 x 16 for fp32)
template <int DT>
__device__ __forceinline__ void load8_elem(const void* p, size_t i, float (&x)[8]) {
    if constexpr (DT == NQ_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (DT == NQ_BF16) {
                x[2 * k] = bf16_bits_to_f32(ws[k] & 0xffffu);
                x[2 * k + 1] = bf16_bits_to_f32(ws[k] >> 16);
            } else {
                x[2 * k] = f16_bits_to_f32(ws[k] & 0xffffu);
                x[2 * k + 1] = f16_bits_to_f32(ws[k] >> 16);
            }
        }
    }
}

__global__ __launch_bounds__(256) void nq_fill_i32(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

// workspace layout shared by nq_merge_workspace and nq_merge_values
struct MergeLayout {
    int n_split;
    int64_t cent, unit, ev_idx, n_ev, best_val, best_idx, surv, weight, count, offset, list, kept_local, total;
    MergeLayout(int b, int s, int d, bool own_centroids) {
        n_split = (int)(((int64_t)s + 63) / 64 / 16);
        n_split = n_split < 1 ? 1 : (n_split > 64 ? 64 : n_split);
        const int64_t bs = (int64_t)b * s;
        int64_t at = 0;
        auto take = [&](int64_t bytes) {
            const int64_t p = at;
            at += (bytes + 255) / 256 * 256;
            return p;
        };
        cent = own_centroids ? -1 : take(bs * d * 4);
        unit = take(bs * d * 4);
        ev_idx = take(bs * 4);
        n_ev = take((int64_t)b * 4);
        best_val = take(bs * n_split * 4);
        best_idx = take(bs * n_split * 4);
        surv = take(bs * 4);
        weight = take(bs * 4);
        count = take(bs * 4);
        offset = take(bs * 4);
        list = take(bs * 4);
        kept_local = take(bs * 4);
        total = at;
    }
};

// 1. centroids [b, s, d]; a thread owns 8 consecutive coordinates
template <int DT>
__global__ __launch_bounds__(256) void merge_centroid_kernel(const uint64_t* src, int n_layers, int b, int h,
                                                             int s, int d, float* cent) {
    const size_t i8 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    const size_t total = (size_t)b * s * d;
    if (i8 >= total) return;
    const int j = (int)(i8 % d);
    const size_t bt = i8 / d;
    const int t = (int)(bt % s);
    const int bi = (int)(bt / s);
    float acc[8];
    for (int l = 0; l < n_layers; ++l) {
        const void* v = reinterpret_cast<const void*>(src[l]);
        float sum[8];
        for (int h0 = 0; h0 < h; h0 += 16) {
            float run[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const int h1 = h0 + 16 < h ? h0 + 16 : h;
            for (int hh = h0; hh < h1; ++hh) {
                float x[8];
                load8_elem<DT>(v, (((size_t)bi * h + hh) * s + t) * d + j, x);
#pragma unroll
                for (int k = 0; k < 8; ++k) run[k] += x[k];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) sum[k] = h0 == 0 ? run[k] : sum[k] + run[k];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float mean = sum[k] / (float)h;
            acc[k] = l == 0 ? mean : acc[k] + mean;
        }
    }
    float4* o = reinterpret_cast<float4*>(cent + i8);
    o[0] = make_float4(acc[0] / (float)n_layers, acc[1] / (float)n_layers, acc[2] / (float)n_layers,
                       acc[3] / (float)n_layers);
    o[1] = make_float4(acc[4] / (float)n_layers, acc[5] / (float)n_layers, acc[6] / (float)n_layers,
                       acc[7] / (float)n_layers);
}

// 2. unit vectors, one wave per row
__global__ __launch_bounds__(256) void merge_normalize_kernel(const float* cent, int rows, int d, float* unit) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* c = cent + (size_t)r * d;
    float ss = 0.0f;
    for (int j = lane; j < d; j += 64) ss = __builtin_fmaf(c[j], c[j], ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float nrm = __builtin_fmaxf(__builtin_sqrtf(ss), 1e-12f);
    for (int j = lane; j < d; j += 64) unit[(size_t)r * d + j] = c[j] / nrm;
}

// evicted positions per row, ascending (block scan compaction), one block per row
__global__ __launch_bounds__(1024) void merge_evicted_kernel(const uint8_t* keep, int s, int32_t* ev_idx,
                                                             int32_t* n_ev) {
    __shared__ int32_t s_sum[1024];
    const int bi = blockIdx.x;
    int base = 0;
    for (int t0 = 0; t0 < s; t0 += 1024) {
        const int t = t0 + threadIdx.x;
        const int f = (t < s && keep[(size_t)bi * s + t] == 0) ? 1 : 0;
        s_sum[threadIdx.x] = f;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int add = threadIdx.x >= o ? s_sum[threadIdx.x - o] : 0;
            __syncthreads();
            s_sum[threadIdx.x] += add;
            __syncthreads();
        }
        if (f) ev_idx[(size_t)bi * s + base + s_sum[threadIdx.x] - 1] = t;
        base += s_sum[1023];
        __syncthreads();
    }
    if (threadIdx.x == 0) n_ev[bi] = base;
}

// 3. best kept token per evicted token over one split of the kept range:
//    block (row, evicted tile, split), 64 x 64 tiles staged in LDS; wave w takes
//    the 32 x 32 quarter (w / 2, w % 2) on the fp32 32x32x2 MFMA.
struct AssignArgs {
    const float* unit;      // [b, s, d]
    const int32_t* ev_idx;  // [b, s]
    const int32_t* n_ev;    // [b]
    const int32_t* kept_idx;
    const int32_t* n_kept;
    float* best_val;        // [b, s, n_split]
    int32_t* best_idx;      // kept-list index
    int b, s, d, n_split, split_len, e_tiles;
};

template <int D>
__global__ __launch_bounds__(256) void merge_assign_kernel(AssignArgs a) {
    constexpr int DC = D < 64 ? D : (D == 96 ? 96 : 64);  // coordinates staged per pass (LDS <= 52 KB)
    __shared__ __attribute__((aligned(16))) float s_e[kMT][DC + kMPad];
    __shared__ __attribute__((aligned(16))) float s_k[kMT][DC + kMPad];
    const int split = blockIdx.x % a.n_split;
    const int et = (blockIdx.x / a.n_split) % a.e_tiles;
    const int bi = blockIdx.x / a.n_split / a.e_tiles;
    const int ne = a.n_ev[bi], nk = a.n_kept[bi];
    const int e0 = et * kMT;
    const int k_begin = split * a.split_len;
    const int k_end = k_begin + a.split_len < nk ? k_begin + a.split_len : nk;
    if (e0 >= ne || k_begin >= k_end) return;  // whole block
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int we = wave >> 1, wk = wave & 1;  // this wave: evicted rows 32 we .., kept columns 32 wk .. of a tile
    const int c = lane & 31, g = lane >> 5;
    const float* U = a.unit + (size_t)bi * a.s * D;
    // running first maximum per row over this wave's columns: lane (c, g), value v
    // holds row 8 (v / 4) + 4 g + v % 4 of the wave's 32 (all 32 lanes of a g agree)
    float bv[16];
    int bidx[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        bv[v] = -__builtin_inff();
        bidx[v] = k_begin;
    }
    for (int k0 = k_begin; k0 < k_end; k0 += kMT) {
        f32x16v acc = {};
        for (int dc = 0; dc < D; dc += DC) {
            __syncthreads();
            // rows past ne / k_end repeat the last valid row; their results are dropped
            for (int i = tid; i < kMT * (DC / 4); i += 256) {
                const int r = i / (DC / 4), c4 = i % (DC / 4);
                const int e = e0 + r < ne ? e0 + r : ne - 1;
                const int k = k0 + r < k_end ? k0 + r : k_end - 1;
                const int pe = a.ev_idx[(size_t)bi * a.s + e];
                const int pk = a.kept_idx[(size_t)bi * a.s + k];
                *reinterpret_cast<float4*>(&s_e[r][4 * c4]) =
                    *reinterpret_cast<const float4*>(U + (size_t)pe * D + dc + 4 * c4);
                *reinterpret_cast<float4*>(&s_k[r][4 * c4]) =
                    *reinterpret_cast<const float4*>(U + (size_t)pk * D + dc + 4 * c4);
            }
            __syncthreads();
            // fp32 MFMA 32x32x2: A[i][k] = evicted row 32 we + i, B[k][j] = kept row 32 wk + j
            const float* ea = &s_e[32 * we + c][g];
            const float* kb = &s_k[32 * wk + c][g];
#pragma unroll 8
            for (int kk = 0; kk < DC; kk += 2)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ea[kk], kb[kk], acc, 0, 0, 0);
        }
        // best of this tile per row over the wave's 32 columns (first index on ties)
        const int col = k0 + 32 * wk + c;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float x = col < k_end ? acc[v] : -__builtin_inff();
            int idx = col < k_end ? col : 0x7fffffff;
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) {
                const float ox = __shfl_xor(x, o, 64);
                const int oi = __shfl_xor(idx, o, 64);
                if (ox > x || (ox == x && oi < idx)) {
                    x = ox;
                    idx = oi;
                }
            }
            if (x > bv[v]) {  // strict: an earlier tile keeps ties
                bv[v] = x;
                bidx[v] = idx;
            }
        }
    }
    // the two column halves of each row: larger value, then the lower index
    __shared__ float s_bv[2][kMT];
    __shared__ int s_bi[2][kMT];
    if (c == 0) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = 32 * we + 8 * (v >> 2) + 4 * g + (v & 3);
            s_bv[wk][r] = bv[v];
            s_bi[wk][r] = bidx[v];
        }
    }
    __syncthreads();
    if (tid < kMT) {
        const int e = e0 + tid;
        if (e < ne) {
            float x = s_bv[0][tid];
            int idx = s_bi[0][tid];
            const float x1 = s_bv[1][tid];
            const int i1 = s_bi[1][tid];
            if (x1 > x || (x1 == x && i1 < idx)) {
                x = x1;
                idx = i1;
            }
            const size_t o = ((size_t)bi * a.s + e) * a.n_split + split;
            a.best_val[o] = x;
            a.best_idx[o] = idx;
        }
    }
}

// 3b + 4. reduce the splits (in order, first max), survivor weights, and the
// per-survivor ascending lists; one block per row.
struct ListArgs {
    const float* best_val;
    const int32_t* best_idx;
    const int32_t* ev_idx;
    const int32_t* n_ev;
    const int32_t* kept_idx;
    const int32_t* n_kept;
    const float* importance;
    int32_t* surv;          // [b, s]: kept-list index of each evicted entry
    float* weight;          // [b, s]: per evicted entry
    int32_t* count;         // [b, s]: per kept-list index
    int32_t* offset;        // [b, s]
    int32_t* list;          // [b, s]: evicted entries grouped by survivor, ascending
    int32_t* kept_local;    // [b, s]: position -> kept-list index or -1
    int32_t* survivor_out;  // optional [b, s]: survivor position of evicted positions, -1 for kept
    int b, s, n_split;
};

__global__ __launch_bounds__(1024) void merge_list_kernel(ListArgs a) {
    __shared__ int32_t s_scan[1024];
    __shared__ int32_t s_key[1024];
    const int bi = blockIdx.x;
    const int tid = threadIdx.x;
    const int ne = a.n_ev[bi], nk = a.n_kept[bi];
    const size_t rb = (size_t)bi * a.s;
    for (int t = tid; t < a.s; t += 1024) {
        a.kept_local[rb + t] = -1;
        a.count[rb + t] = 0;
    }
    __syncthreads();
    for (int k = tid; k < nk; k += 1024) a.kept_local[rb + a.kept_idx[rb + k]] = k;
    if (nk == 0) {  // nothing survives: no merge, every row is copied
        if (a.survivor_out)
            for (int t = tid; t < a.s; t += 1024) a.survivor_out[rb + t] = -1;
        return;
    }
    // survivors and weights
    for (int e = tid; e < ne; e += 1024) {
        float v = -__builtin_inff();
        int idx = 0;
        for (int sp = 0; sp < a.n_split; ++sp) {
            const size_t o = (rb + e) * a.n_split + sp;
            if (a.best_idx[o] >= 0 && a.best_val[o] > v) {  // splits in order: first max
                v = a.best_val[o];
                idx = a.best_idx[o];
            }
        }
        a.surv[rb + e] = idx;
        const int pe = a.ev_idx[rb + e];
        const int ps = a.kept_idx[rb + idx];
        const double ie = (double)a.importance[rb + pe];
        const double is = (double)a.importance[rb + ps];
        a.weight[rb + e] = (float)(ie / (is + ie + 1e-8));
        atomicAdd(&a.count[rb + idx], 1);
    }
    __syncthreads();
    if (a.survivor_out) {
        for (int t = tid; t < a.s; t += 1024)
            if (a.kept_local[rb + t] >= 0) a.survivor_out[rb + t] = -1;
        for (int e = tid; e < ne; e += 1024) a.survivor_out[rb + a.ev_idx[rb + e]] = a.kept_idx[rb + a.surv[rb + e]];
    }
    // exclusive scan of the counts over the kept list
    int carry = 0;
    for (int k0 = 0; k0 < nk; k0 += 1024) {
        const int k = k0 + tid;
        const int c = k < nk ? a.count[rb + k] : 0;
        s_scan[tid] = c;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int add = tid >= o ? s_scan[tid - o] : 0;
            __syncthreads();
            s_scan[tid] += add;
            __syncthreads();
        }
        if (k < nk) a.offset[rb + k] = carry + s_scan[tid] - c;
        carry += s_scan[1023];
        __syncthreads();
    }
    // stable fill: chunks of 1024 evicted entries in order; an entry's slot is
    // its survivor's next free slot plus the number of earlier entries of the
    // chunk with the same survivor.  count[] becomes the running fill.
    for (int k = tid; k < nk; k += 1024) a.count[rb + k] = a.offset[rb + k];
    __syncthreads();
    for (int e0 = 0; e0 < ne; e0 += 1024) {
        const int e = e0 + tid;
        const int key = e < ne ? a.surv[rb + e] : -1;
        s_key[tid] = key;
        __syncthreads();
        int rank = 0;
        bool last = true;
        const int m = ne - e0 < 1024 ? ne - e0 : 1024;
        if (e < ne) {
            for (int j = 0; j < m; ++j) {
                if (s_key[j] == key) {
                    if (j < tid) ++rank;
                    else if (j > tid) last = false;
                }
            }
            a.list[rb + a.count[rb + key] + rank] = e;
        }
        __syncthreads();
        if (e < ne && last) a.count[rb + key] += rank + 1;
        __syncthreads();
    }
}

// 5. merged rows: D/8 lanes per (layer, row, head, token), 8 coordinates per
//    lane.  Every row is written (copied unless it is a survivor with merges).
struct ApplyArgs {
    const uint64_t* src;
    const uint64_t* dst;
    const int32_t* kept_local;
    const int32_t* offset;
    const int32_t* count;    // after the fill: offset + number of merged entries
    const int32_t* list;
    const int32_t* ev_idx;
    const float* weight;
    int n_layers, b, h, s, d;
};

// Grid: x over (token, 8-element piece) of one head's rows, y over batch x head
// (strided when there are more than the grid allows), z over the layers; all
// index arithmetic is 32-bit, the row split a shift for power-of-two head dims.
template <int DT>
__global__ __launch_bounds__(256) void merge_apply_kernel(ApplyArgs a) {
    const uint32_t lanes_per_row = (uint32_t)a.d / 8u;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    const uint32_t t = (lanes_per_row & (lanes_per_row - 1u)) == 0u ? idx >> __builtin_ctz(lanes_per_row)
                                                                     : idx / lanes_per_row;
    if (t >= (uint32_t)a.s) return;
    const int j = (int)(idx - t * lanes_per_row) * 8;
    const int layer = blockIdx.z;
    const void* src = reinterpret_cast<const void*>(a.src[layer]);
    void* dst = reinterpret_cast<void*>(a.dst[layer]);
    const uint32_t bh_count = (uint32_t)a.b * (uint32_t)a.h;
    for (uint32_t bh = blockIdx.y; bh < bh_count; bh += gridDim.y) {
        const uint32_t bi = bh / (uint32_t)a.h;
        const size_t row_off = ((size_t)bh * a.s + t) * (size_t)a.d + j;
        const size_t rb = (size_t)bi * a.s;
        // the row's own 8 elements load alongside its list entry (both are needed
        // on either path), so the two memory latencies overlap
        constexpr int NW = DT == NQ_F32 ? 2 : 1;
        const uint4* sp = reinterpret_cast<const uint4*>(static_cast<const char*>(src) + row_off * (DT == NQ_F32 ? 4 : 2));
        uint4 raw[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k) raw[k] = sp[k];
        const int kl = a.kept_local[rb + t];
        const int beg = kl >= 0 ? a.offset[rb + kl] : 0;
        const int end = kl >= 0 ? a.count[rb + kl] : 0;
        uint4* dp = reinterpret_cast<uint4*>(static_cast<char*>(dst) + row_off * (DT == NQ_F32 ? 4 : 2));
        if (end <= beg) {  // no merges: the bits unchanged
#pragma unroll
            for (int k = 0; k < NW; ++k) dp[k] = raw[k];
            continue;
        }
        const size_t head_base = (size_t)bh * a.s * (size_t)a.d + j;
        float v[8];
        load8_elem<DT>(src, row_off, v);
        for (int i = beg; i < end; ++i) {
            const int e = a.list[rb + i];
            const int pe = a.ev_idx[rb + e];
            const float w = a.weight[rb + e];
            float x[8];
            load8_elem<DT>(src, head_base + (size_t)pe * a.d, x);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = v[k] + w * x[k];  // two roundings, as the reference's separate ops
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) store_elem<DT>(dst, row_off + k, v[k]);
    }
}

}  // namespace nq

extern "C" int64_t nq_merge_workspace(int32_t batch, int32_t seq, int32_t head_dim) {
    if (batch <= 0 || seq <= 0 || head_dim <= 0) return 0;
    return nq::MergeLayout(batch, seq, head_dim, false).total;
}

extern "C" int nq_merge_values(const nq_merge_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_merge_values: desc is NULL");
    NQ_CHECK_ARG(d->n_tensors >= 1 && d->n_tensors <= 65535, "nq_merge_values: n_tensors %d out of range",
                 d->n_tensors);
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 96 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_merge_values: head_dim %d unsupported (64, 96, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->dtype == NQ_F16 || d->dtype == NQ_BF16 || d->dtype == NQ_F32, "nq_merge_values: unknown dtype %d",
                 d->dtype);
    NQ_CHECK_ARG(d->batch > 0 && d->heads > 0 && d->heads <= 256 && d->seq > 0,
                 "nq_merge_values: bad geometry (heads must be 1..256)");
    NQ_CHECK_ARG(d->src && d->dst && d->keep && d->kept_idx && d->n_kept && d->importance,
                 "nq_merge_values: src, dst, keep, kept_idx, n_kept and importance are required");
    const int64_t need = nq_merge_workspace(d->batch, d->seq, d->head_dim);
    NQ_CHECK_ARG(d->workspace != nullptr && d->workspace_bytes >= need, "nq_merge_values: workspace of %lld bytes needed",
                 (long long)need);
    const int b = d->batch, h = d->heads, s = d->seq, D = d->head_dim;
    const int64_t bs = (int64_t)b * s;
    NQ_CHECK_ARG(bs * D < (1ll << 40) && bs < (1ll << 31), "nq_merge_values: too large");
    const MergeLayout L(b, s, D, d->centroids != nullptr);
    const int n_split = L.n_split;
    const int k_tiles = (s + kMT - 1) / kMT;
    const int split_len = (k_tiles + n_split - 1) / n_split * kMT;
    char* w = static_cast<char*>(d->workspace);
    float* cent = d->centroids ? d->centroids : reinterpret_cast<float*>(w + L.cent);
    float* unit = reinterpret_cast<float*>(w + L.unit);
    int32_t* ev_idx = reinterpret_cast<int32_t*>(w + L.ev_idx);
    int32_t* n_ev = reinterpret_cast<int32_t*>(w + L.n_ev);
    float* best_val = reinterpret_cast<float*>(w + L.best_val);
    int32_t* best_idx = reinterpret_cast<int32_t*>(w + L.best_idx);
    int32_t* surv = reinterpret_cast<int32_t*>(w + L.surv);
    float* weight = reinterpret_cast<float*>(w + L.weight);
    int32_t* count = reinterpret_cast<int32_t*>(w + L.count);
    int32_t* offset = reinterpret_cast<int32_t*>(w + L.offset);
    int32_t* list = reinterpret_cast<int32_t*>(w + L.list);
    int32_t* kept_local = reinterpret_cast<int32_t*>(w + L.kept_local);
    hipStream_t st = (hipStream_t)stream;

    const int64_t n_el = bs * D / 8;  // 8 coordinates per thread
#define NQ_CENT(DT)                                                                                           \
    hipLaunchKernelGGL(merge_centroid_kernel<DT>, dim3((uint32_t)((n_el + 255) / 256)), dim3(256), 0, st, d->src, \
                       d->n_tensors, b, h, s, D, cent)
    if (d->dtype == NQ_F16) NQ_CENT(NQ_F16);
    else if (d->dtype == NQ_BF16) NQ_CENT(NQ_BF16);
    else NQ_CENT(NQ_F32);
#undef NQ_CENT
    NQ_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(merge_normalize_kernel, dim3((uint32_t)((bs + 3) / 4)), dim3(256), 0, st, cent, (int)bs, D, unit);
    NQ_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(merge_evicted_kernel, dim3(b), dim3(1024), 0, st, d->keep, s, ev_idx, n_ev);
    NQ_CHECK_HIP(hipGetLastError());

    AssignArgs aa;
    aa.unit = unit;
    aa.ev_idx = ev_idx;
    aa.n_ev = n_ev;
    aa.kept_idx = d->kept_idx;
    aa.n_kept = d->n_kept;
    aa.best_val = best_val;
    aa.best_idx = best_idx;
    aa.b = b;
    aa.s = s;
    aa.d = D;
    aa.n_split = n_split;
    aa.split_len = split_len;
    aa.e_tiles = (s + kMT - 1) / kMT;
    const uint64_t grid = (uint64_t)b * aa.e_tiles * n_split;
    NQ_CHECK_ARG(grid <= max_blocks(256), "nq_merge_values: assignment grid too large");
    // partials of splits a row never reaches stay unwritten: mark them empty
    hipLaunchKernelGGL(nq_fill_i32, dim3((uint32_t)((bs * n_split + 255) / 256)), dim3(256), 0, st, best_idx,
                       bs * n_split, -1);
    NQ_CHECK_HIP(hipGetLastError());
    switch (D) {
        case 64: hipLaunchKernelGGL(merge_assign_kernel<64>, dim3((uint32_t)grid), dim3(256), 0, st, aa); break;
        case 96: hipLaunchKernelGGL(merge_assign_kernel<96>, dim3((uint32_t)grid), dim3(256), 0, st, aa); break;
        case 128: hipLaunchKernelGGL(merge_assign_kernel<128>, dim3((uint32_t)grid), dim3(256), 0, st, aa); break;
        default: hipLaunchKernelGGL(merge_assign_kernel<256>, dim3((uint32_t)grid), dim3(256), 0, st, aa); break;
    }
    NQ_CHECK_HIP(hipGetLastError());

    ListArgs la;
    la.best_val = best_val;
    la.best_idx = best_idx;
    la.ev_idx = ev_idx;
    la.n_ev = n_ev;
    la.kept_idx = d->kept_idx;
    la.n_kept = d->n_kept;
    la.importance = d->importance;
    la.surv = surv;
    la.weight = weight;
    la.count = count;
    la.offset = offset;
    la.list = list;
    la.kept_local = kept_local;
    la.survivor_out = d->survivor;
    la.b = b;
    la.s = s;
    la.n_split = n_split;
    hipLaunchKernelGGL(merge_list_kernel, dim3(b), dim3(1024), 0, st, la);
    NQ_CHECK_HIP(hipGetLastError());

    ApplyArgs ap;
    ap.src = d->src;
    ap.dst = d->dst;
    ap.kept_local = kept_local;
    ap.offset = offset;
    ap.count = count;
    ap.list = list;
    ap.ev_idx = ev_idx;
    ap.weight = weight;
    ap.n_layers = d->n_tensors;
    ap.b = b;
    ap.h = h;
    ap.s = s;
    ap.d = D;
    const uint64_t threads = (uint64_t)s * (uint64_t)(D / 8);  // per (layer, batch, head)
    NQ_CHECK_ARG(threads < (1ull << 31), "nq_merge_values: sequence too long");
    const uint32_t bh = (uint32_t)b * (uint32_t)h;
    const dim3 g((uint32_t)((threads + 255) / 256), bh < 65535u ? bh : 65535u, (uint32_t)d->n_tensors);
    if (d->dtype == NQ_F16) hipLaunchKernelGGL(merge_apply_kernel<NQ_F16>, g, dim3(256), 0, st, ap);
    else if (d->dtype == NQ_BF16) hipLaunchKernelGGL(merge_apply_kernel<NQ_BF16>, g, dim3(256), 0, st, ap);
    else hipLaunchKernelGGL(merge_apply_kernel<NQ_F32>, g, dim3(256), 0, st, ap);
    NQ_CHECK_HIP(hipGetLastError());
    return NQ_OK;
}
