// Key-key importance scorer on gfx950 MFMA (reference: NexusQuantEvict.
// _score_importance, pipeline.py:756-782).
//
// Per (batch, head): queries = the last obs keys, logits x = (q . k) * scale in
// fp32 over all s keys, softmax over the keys of each query, importance[b, j] =
// mean over heads of the sum over queries of p[q, j].
//
// Two launches; the keys are read twice, each time by a grid that fills the
// chip:
//   kk_stats   per (batch, head), 32-query block and 512-key split: the
//              split's row maximum m and sum z = sum exp(x - m) for each query
//              (online over 32-key tiles).  Keys are the MFMA A operand
//              (rows), so a lane holds one query's logits against 16 keys and
//              keeps (m, z) alone.
//   kk_colsum  per 32-key tile of one batch row, one wave per head: combines
//              the splits' (m, z) into the row maximum M and sum Z,
//              recomputes the logits with the keys as the B operand (columns),
//              sums p = exp(x - M) * (1 / Z) over the queries of each key
//              column, and the workgroup adds its heads in order and divides
//              by the head count.
// The second read of the keys directly follows the first, so at the benchmark
// shapes (64 MiB of keys per layer) it is served from the last-level cache.
//
// kk_stats stages its queries in LDS (rows padded by 16 bytes, so the 16-byte
// operand reads of 8 consecutive lanes hit distinct banks) and takes the keys
// straight from global memory into the lanes' operand registers, one tile
// ahead; kk_colsum holds both operands in registers.  Operand unit u of lane
// group g = lane / 32 is the 16 bytes at 32 u + 16 g of the lane's row, so
// lanes c and c + 32 read one 32-byte run; a unit is one MFMA step for f16 /
// bf16 (the hardware's own k order) and four steps for f32.  Both operands use
// the same order, so the products cover every coordinate once.
#include <mutex>

#include "nq_common.h"

namespace nq {
namespace kk {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQueryBlock = 32;
constexpr int kMaxWaves = 8;      // kk_colsum: waves (heads in flight) per workgroup

template <int DT>
struct EB { static constexpr int v = (DT == NQ_F32) ? 4 : 2; };

template <int DT, int D>
struct Geom {
    static constexpr int ROW = D * EB<DT>::v;          // bytes of one key row
    static constexpr int UNITS = ROW / 32;             // 16-byte operand units per lane
    static constexpr int CH = UNITS < 16 ? UNITS : 16; // units held in registers at once
    static constexpr int NCH = UNITS / CH;             // register chunks per tile
    static constexpr int QROWB = ROW + 16;             // padded LDS query row
    static constexpr int ROW_UNITS = ROW / 16;
    static_assert(ROW % 32 == 0 && UNITS % CH == 0, "rows are whole 32-byte units");
};

struct Args {
    const char* keys;   // [bh, seq, d]
    float2* part;       // [bh, nsplit, nq] (m, z) per split and query
    float* importance;  // [batch, seq]
    int32_t seq, obs, nq, nsplit, split_keys, heads, batch;
    float scale;
};

__device__ __forceinline__ int acc_row(int j, int g) { return 8 * (j >> 2) + 4 * g + (j & 3); }

// one MFMA step over 16 operand bytes per lane; KROWS: keys are the A operand
template <int DT, bool KROWS>
__device__ __forceinline__ f32x16 mfma_unit(uint4 k, uint4 q, f32x16 acc) {
    if constexpr (DT == NQ_F16) {
        const f16x8 a = __builtin_bit_cast(f16x8, KROWS ? k : q), b = __builtin_bit_cast(f16x8, KROWS ? q : k);
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
    } else if constexpr (DT == NQ_BF16) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, KROWS ? k : q), b = __builtin_bit_cast(bf16x8, KROWS ? q : k);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    } else {
        const float kf[4] = {__builtin_bit_cast(float, k.x), __builtin_bit_cast(float, k.y),
                             __builtin_bit_cast(float, k.z), __builtin_bit_cast(float, k.w)};
        const float qf[4] = {__builtin_bit_cast(float, q.x), __builtin_bit_cast(float, q.y),
                             __builtin_bit_cast(float, q.z), __builtin_bit_cast(float, q.w)};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(KROWS ? kf[e] : qf[e], KROWS ? qf[e] : kf[e], acc, 0, 0, 0);
        return acc;
    }
}

// this lane's operand units of chunk `ch` of key row `row` (clamped by the caller)
template <int DT, int D>
__device__ __forceinline__ void load_key(const char* kbase, int row, int g, int ch,
                                         uint4 (&r)[Geom<DT, D>::CH]) {
    using G = Geom<DT, D>;
    const char* p = kbase + (size_t)row * G::ROW + 16 * g + 32 * ch * G::CH;
#pragma unroll
    for (int u = 0; u < G::CH; ++u) r[u] = *reinterpret_cast<const uint4*>(p + 32 * u);
}

// 32 x 32 logits of one key tile: the first chunk of key operands is given
// (prefetched), later chunks are loaded here.  q_lds: this lane's query row in
// LDS, offset by 16 g.
template <int DT, int D, bool KROWS>
__device__ __forceinline__ f32x16 tile_logits(const uint4 (&k0)[Geom<DT, D>::CH], const char* kbase, int row, int g,
                                              const char* q_lds) {
    using G = Geom<DT, D>;
    f32x16 acc = {};
#pragma unroll
    for (int u = 0; u < G::CH; ++u)
        acc = mfma_unit<DT, KROWS>(k0[u], *reinterpret_cast<const uint4*>(q_lds + 32 * u), acc);
#pragma unroll
    for (int ch = 1; ch < G::NCH; ++ch) {
        uint4 kc[G::CH];
        load_key<DT, D>(kbase, row, g, ch, kc);
#pragma unroll
        for (int u = 0; u < G::CH; ++u)
            acc = mfma_unit<DT, KROWS>(kc[u], *reinterpret_cast<const uint4*>(q_lds + 32 * (ch * G::CH + u)), acc);
    }
    return acc;
}

// 32 x 32 logits with both operands in registers (first chunk given; later
// chunks of both rows are loaded here).  q_row / k_row: this lane's rows.
template <int DT, int D, bool KROWS>
__device__ __forceinline__ f32x16 tile_logits_rr(const uint4 (&k0)[Geom<DT, D>::CH], const uint4 (&q0)[Geom<DT, D>::CH],
                                                 const char* kbase, int k_row, int q_row, int g) {
    using G = Geom<DT, D>;
    f32x16 acc = {};
#pragma unroll
    for (int u = 0; u < G::CH; ++u) acc = mfma_unit<DT, KROWS>(k0[u], q0[u], acc);
#pragma unroll
    for (int ch = 1; ch < G::NCH; ++ch) {
        uint4 kc[G::CH], qc[G::CH];
        load_key<DT, D>(kbase, k_row, g, ch, kc);
        load_key<DT, D>(kbase, q_row, g, ch, qc);
#pragma unroll
        for (int u = 0; u < G::CH; ++u) acc = mfma_unit<DT, KROWS>(kc[u], qc[u], acc);
    }
    return acc;
}

// Stage query block qb (rows seq - obs + 32 qb + r, clamped to the last key)
// into LDS, padded rows.  Ends with a barrier.
template <int DT, int D>
__device__ __forceinline__ void stage_queries(const char* kbase, const Args& a, int qb, char* qs) {
    using G = Geom<DT, D>;
    for (int u = threadIdx.x; u < kQueryBlock * G::ROW_UNITS; u += blockDim.x) {
        const int r = u / G::ROW_UNITS, c = u - r * G::ROW_UNITS;
        const int qi = min(qb * kQueryBlock + r, a.obs - 1);
        const int row = a.seq - a.obs + qi;
        *reinterpret_cast<uint4*>(qs + r * G::QROWB + 16 * c) =
            *reinterpret_cast<const uint4*>(kbase + (size_t)row * G::ROW + 16 * c);
    }
    __syncthreads();
}

// (m1, z1) + (m2, z2) of two partial softmax sums over disjoint key sets
__device__ __forceinline__ float2 combine(float2 p, float2 q) {
    const float m = fmaxf(p.x, q.x);
    if (m == -__builtin_inff()) return make_float2(m, 0.0f);
    const float zp = p.x == m ? p.y : p.y * __builtin_amdgcn_exp2f((p.x - m) * kLog2e);
    const float zq = q.x == m ? q.y : q.y * __builtin_amdgcn_exp2f((q.x - m) * kLog2e);
    return make_float2(m, zp + zq);
}

// grid: bh * nsplit workgroups of 4 waves; wave w takes TPW 32-key tiles of
// the split, from key split * split_keys + w * 32 * TPW.
template <int DT, int D, int TPW>
__global__ __launch_bounds__(256) void kk_stats(Args a) {
    using G = Geom<DT, D>;
    __shared__ __align__(16) char qs[kQueryBlock * G::QROWB];
    __shared__ float2 red[4][kQueryBlock];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, c = lane & 31;
    const int split = blockIdx.x % a.nsplit;
    const int bh = blockIdx.x / a.nsplit;
    const char* kbase = a.keys + (size_t)bh * a.seq * G::ROW;
    const int w0 = split * a.split_keys + wave * 32 * TPW;  // this wave's first key
    const int n_tiles = max(0, min(TPW, (a.seq - w0 + 31) / 32));
    const int n_qb = (a.obs + kQueryBlock - 1) / kQueryBlock;
    uint4 cur[G::CH];
    if (n_tiles > 0) load_key<DT, D>(kbase, min(w0 + c, a.seq - 1), g, 0, cur);  // in flight while staging
    for (int qb = 0; qb < n_qb; ++qb) {
        if (qb) {
            __syncthreads();  // the previous query block's LDS reads are done
            if (n_tiles > 0) load_key<DT, D>(kbase, min(w0 + c, a.seq - 1), g, 0, cur);
        }
        stage_queries<DT, D>(kbase, a, qb, qs);
        const char* q_lds = qs + c * G::QROWB + 16 * g;
        float m = -__builtin_inff(), z = 0.0f;
        for (int t = 0; t < n_tiles; ++t) {
            const int key0 = w0 + 32 * t;
            const int row = min(key0 + c, a.seq - 1);
            uint4 nxt[G::CH];  // the next tile's keys in flight during this one
            if (t + 1 < n_tiles) load_key<DT, D>(kbase, min(key0 + 32 + c, a.seq - 1), g, 0, nxt);
            const f32x16 acc = tile_logits<DT, D, true>(cur, kbase, row, g, q_lds);
            // acc[j]: key key0 + acc_row(j, g), query c of the block.  The
            // maximum is taken on the raw dot products: fl(max(acc) * scale) =
            // max(fl(acc * scale)) because rounding is monotone and scale > 0.
            const bool full = key0 + 32 <= a.seq;  // wave-uniform
            float tmax = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 16; ++j)
                tmax = fmaxf(tmax, full || key0 + acc_row(j, g) < a.seq ? acc[j] : -__builtin_inff());
            const float mn = fmaxf(m, tmax * a.scale);
            if (mn != -__builtin_inff()) {
                if (mn != m) z *= __builtin_amdgcn_exp2f((m - mn) * kLog2e);
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float e = __builtin_amdgcn_exp2f((acc[j] * a.scale - mn) * kLog2e);
                    z += full || key0 + acc_row(j, g) < a.seq ? e : 0.0f;
                }
                m = mn;
            }
            if (t + 1 < n_tiles) {
#pragma unroll
                for (int u = 0; u < G::CH; ++u) cur[u] = nxt[u];
            }
        }
        // lanes c and c + 32 hold the same query over disjoint keys
        float2 s = make_float2(m, z);
        s = combine(s, make_float2(__shfl_xor(s.x, 32, 64), __shfl_xor(s.y, 32, 64)));
        if (g == 0) red[wave][c] = s;
        __syncthreads();
        if (threadIdx.x < kQueryBlock) {
            float2 t = red[0][c];
#pragma unroll
            for (int w = 1; w < 4; ++w) t = combine(t, red[w][c]);
            a.part[((size_t)bh * a.nsplit + split) * a.nq + qb * kQueryBlock + c] = t;
        }
    }
}

// grid: batch * ceil(seq / (32 KT)) workgroups of W = min(heads, 8) waves;
// wave w takes heads w, w + W, ... of KT 32-key tiles of one batch row.
template <int DT, int D, int KT>
__global__ __launch_bounds__(64 * kMaxWaves) void kk_colsum(Args a) {
    using G = Geom<DT, D>;
    constexpr bool PREFETCH = G::CH <= 8;  // the next tile's keys in flight (registers allowing)
    __shared__ __align__(16) float2 st[kMaxWaves][kQueryBlock];  // per wave: (M, 1/Z) per query
    __shared__ float head_sum[kMaxWaves][32 * KT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5, c = lane & 31;
    const int W = blockDim.x >> 6;
    const int n_kr = (a.seq + 32 * KT - 1) / (32 * KT);
    const int kr0 = blockIdx.x % n_kr;
    const int b = blockIdx.x / n_kr;
    const int key_base = kr0 * 32 * KT;
    const int n_t = min(KT, (a.seq - key_base + 31) / 32);  // wave-uniform, >= 1
    const int n_qb = (a.obs + kQueryBlock - 1) / kQueryBlock;
    float hsum[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) hsum[t] = 0.0f;
    for (int h = wave; h < a.heads; h += W) {
        const int bh = b * a.heads + h;
        const char* kbase = a.keys + (size_t)bh * a.seq * G::ROW;
        const float2* part = a.part + (size_t)bh * a.nsplit * a.nq;
        for (int qb = 0; qb < n_qb; ++qb) {
            // the queries (the last obs keys) as the A operand, held for KT tiles
            const int q_row = a.seq - a.obs + min(qb * kQueryBlock + c, a.obs - 1);
            uint4 qr[G::CH], cur[G::CH];
            load_key<DT, D>(kbase, q_row, g, 0, qr);
            load_key<DT, D>(kbase, min(key_base + c, a.seq - 1), g, 0, cur);
            // row maximum and sum of query 32 qb + c: the splits' partials,
            // alternate splits in lanes c and c + 32 (fixed order: deterministic)
            float2 s = make_float2(-__builtin_inff(), 0.0f);
            for (int sp = g; sp < a.nsplit; sp += 2) s = combine(s, part[(size_t)sp * a.nq + qb * kQueryBlock + c]);
            s = combine(s, make_float2(__shfl_xor(s.x, 32, 64), __shfl_xor(s.y, 32, 64)));
            // LDS ops of one wave execute in order; the fences keep the compiler
            // from moving the reads below above the write.  Rows past obs get
            // M = +inf and 1/Z = 0, so their terms are exp2(-inf) * 0 = 0.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            if (g == 0)
                st[wave][c] = qb * kQueryBlock + c < a.obs ? make_float2(s.x, 1.0f / s.y)
                                                           : make_float2(__builtin_inff(), 0.0f);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (t < n_t) {
                    const int k_row = min(key_base + 32 * t + c, a.seq - 1);
                    uint4 nxt[G::CH];
                    if (PREFETCH && t + 1 < n_t)
                        load_key<DT, D>(kbase, min(key_base + 32 * (t + 1) + c, a.seq - 1), g, 0, nxt);
                    if (!PREFETCH && t > 0) load_key<DT, D>(kbase, k_row, g, 0, cur);
                    const f32x16 acc = tile_logits_rr<DT, D, false>(cur, qr, kbase, k_row, q_row, g);
                    // acc[j]: query 32 qb + acc_row(j, g), key key_base + 32 t + c
                    float col = 0.0f;
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int r0 = 8 * jq + 4 * g;
                        const float4 s01 = *reinterpret_cast<const float4*>(&st[wave][r0]);
                        const float4 s23 = *reinterpret_cast<const float4*>(&st[wave][r0 + 2]);
                        const float mm[4] = {s01.x, s01.z, s23.x, s23.z};
                        const float rz[4] = {s01.y, s01.w, s23.y, s23.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            col += __builtin_amdgcn_exp2f((acc[4 * jq + u] * a.scale - mm[u]) * kLog2e) * rz[u];
                    }
                    hsum[t] += col + __shfl_xor(col, 32, 64);
                    if (PREFETCH && t + 1 < n_t) {
#pragma unroll
                        for (int u = 0; u < G::CH; ++u) cur[u] = nxt[u];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();  // reads of st done before the next block's write
        }
    }
    if (g == 0) {
#pragma unroll
        for (int t = 0; t < KT; ++t) head_sum[wave][32 * t + c] = hsum[t];
    }
    __syncthreads();
    const int n_keys = min(32 * n_t, a.seq - key_base);  // keys of this workgroup inside the row
    for (int i = threadIdx.x; i < n_keys; i += blockDim.x) {
        float t = 0.0f;
        for (int w = 0; w < W; ++w) t += head_sum[w][i];
        a.importance[(size_t)b * a.seq + key_base + i] = t / (float)a.heads;
    }
}

constexpr int kTilesPerWave = 4;  // kk_stats: 32-key tiles per wave
constexpr int kColsumTiles = 4;   // kk_colsum: 32-key tiles per wave
constexpr int kSplitKeys = 4 * 32 * kTilesPerWave;

int64_t workspace_bytes(int64_t bh, int64_t seq, int64_t nq) {
    const int64_t nsplit = (seq + kSplitKeys - 1) / kSplitKeys;
    return bh * nsplit * nq * 8;
}

template <int DT, int D>
hipError_t launch(const Args& a, hipStream_t st) {
    const int bh = a.batch * a.heads;
    hipLaunchKernelGGL((kk_stats<DT, D, kTilesPerWave>), dim3(bh * a.nsplit), dim3(256), 0, st, a);
    const int n_kr = (a.seq + 32 * kColsumTiles - 1) / (32 * kColsumTiles);
    const int waves = a.heads < kMaxWaves ? a.heads : kMaxWaves;
    hipLaunchKernelGGL((kk_colsum<DT, D, kColsumTiles>), dim3(a.batch * n_kr), dim3(64 * waves), 0, st, a);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch_d(int d, const Args& a, hipStream_t st) {
    switch (d) {
        case 64: return launch<DT, 64>(a, st);
        case 96: return launch<DT, 96>(a, st);
        case 128: return launch<DT, 128>(a, st);
        default: return launch<DT, 256>(a, st);
    }
}

}  // namespace kk

// Shared by nq_score_keykey (caller's workspace) and the no-allocation entry point.
int score_keykey_ws(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq, int32_t head_dim,
                    int32_t obs_window, float scale, float* importance, void* workspace, int64_t workspace_bytes,
                    void* stream, const char* who) {
    using namespace kk;
    NQ_CHECK_ARG(keys && importance && workspace, "%s: NULL pointer", who);
    NQ_CHECK_ARG(batch > 0 && heads > 0 && seq >= 0, "%s: bad shape", who);
    NQ_CHECK_ARG((int64_t)batch * heads * ((int64_t)seq + kSplitKeys - 1) / kSplitKeys < (1LL << 31) &&
                     (int64_t)batch * (((int64_t)seq + 31) / 32) < (1LL << 31),
                 "%s: too many keys for one launch", who);
    NQ_CHECK_ARG(head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256,
                 "%s: head_dim %d unsupported (64, 96, 128, 256)", who, head_dim);
    NQ_CHECK_ARG(dtype == NQ_F16 || dtype == NQ_BF16 || dtype == NQ_F32, "%s: bad dtype", who);
    NQ_CHECK_ARG(obs_window > 0, "%s: obs_window must be positive", who);
    if (seq == 0) return NQ_OK;
    Args a;
    a.obs = obs_window < seq ? obs_window : seq;
    a.nq = (a.obs + kQueryBlock - 1) / kQueryBlock * kQueryBlock;
    const int64_t bh = (int64_t)batch * heads;
    const int64_t need = kk::workspace_bytes(bh, seq, a.nq);
    NQ_CHECK_ARG(workspace_bytes >= need, "%s: workspace %lld bytes < %lld", who, (long long)workspace_bytes,
                 (long long)need);
    a.keys = static_cast<const char*>(keys);
    a.seq = seq;
    a.split_keys = kSplitKeys;
    a.nsplit = (seq + kSplitKeys - 1) / kSplitKeys;
    a.heads = heads;
    a.batch = batch;
    a.scale = scale;
    a.part = static_cast<float2*>(workspace);
    a.importance = importance;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (dtype) {
        case NQ_F16: e = dispatch_d<NQ_F16>(head_dim, a, st); break;
        case NQ_BF16: e = dispatch_d<NQ_BF16>(head_dim, a, st); break;
        default: e = dispatch_d<NQ_F32>(head_dim, a, st); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

}  // namespace nq

// ---------------------------------------------------------------------------
// No-allocation variant: the workspace is this file-scope device array, one
// copy per GPU for the life of the process.  Host code never passes `scratch`
// itself to a kernel (in host code the name is a stand-in, not a device
// address): each device's address comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that pointer is used.
// Nothing in it needs to start at zero: kk_stats writes every partial that
// kk_colsum then reads, in the same call.  Calls that overlap on one GPU
// share the array and race.
// ---------------------------------------------------------------------------
namespace nq {

static __device__ __align__(256) char scratch[NQ_KEYKEY_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// the device address of `scratch` on the current device (looked up once per device)
static int current_scratch(void** out, const char* who) {
    int dev = -1;
    NQ_CHECK_HIP(hipGetDevice(&dev));
    NQ_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d this library tracks", who, dev,
                 kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev, hipGetErrorString(e));
            return NQ_EHIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NQ_OK;
}

}  // namespace nq

extern "C" int nq_score_keykey_noalloc(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq,
                                       int32_t head_dim, int32_t obs_window, float scale, float* importance,
                                       void* stream) {
    using namespace nq;
    static const char* who = "nq_score_keykey_noalloc";
    NQ_CHECK_ARG(batch > 0 && heads > 0 && seq >= 0 && obs_window > 0, "%s: bad shape", who);
    if (seq == 0) return NQ_OK;
    const int64_t need = nq_score_keykey_workspace(batch, heads, seq, obs_window);
    NQ_CHECK_ARG(need <= NQ_KEYKEY_SCRATCH_BYTES,
                 "%s: batch %d x heads %d x seq %d (obs %d) needs %lld bytes of scratch, above the static "
                 "%d; use nq_score_keykey with a workspace",
                 who, batch, heads, seq, obs_window, (long long)need, NQ_KEYKEY_SCRATCH_BYTES);
    int cur = -1;
    NQ_CHECK_HIP(hipGetDevice(&cur));
    if (stream) {
        hipDevice_t sdev = -1;
        NQ_CHECK_HIP(hipStreamGetDevice((hipStream_t)stream, &sdev));
        NQ_CHECK_ARG((int)sdev == cur, "%s: the stream belongs to device %d, the current device is %d", who,
                     (int)sdev, cur);
    }
    void* ws = nullptr;
    const int st = current_scratch(&ws, who);
    if (st != NQ_OK) return st;
    return score_keykey_ws(keys, dtype, batch, heads, seq, head_dim, obs_window, scale, importance, ws,
                           NQ_KEYKEY_SCRATCH_BYTES, stream, who);
}

extern "C" int64_t nq_score_keykey_workspace(int32_t batch, int32_t heads, int32_t seq, int32_t obs_window) {
    if (batch <= 0 || heads <= 0 || seq <= 0 || obs_window <= 0) return 0;
    const int64_t obs = obs_window < seq ? obs_window : seq;
    const int64_t nq = (obs + nq::kk::kQueryBlock - 1) / nq::kk::kQueryBlock * nq::kk::kQueryBlock;
    return nq::kk::workspace_bytes((int64_t)batch * heads, seq, nq);
}

extern "C" int nq_score_keykey(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq,
                               int32_t head_dim, int32_t obs_window, float scale, float* importance,
                               void* workspace, int64_t workspace_bytes, void* stream) {
    return nq::score_keykey_ws(keys, dtype, batch, heads, seq, head_dim, obs_window, scale, importance, workspace,
                               workspace_bytes, stream, "nq_score_keykey");
}
