// Key-key importance scorer on gfx950 MFMA (reference: NexusQuantEvict.
// _score_importance, pipeline.py:756-782).
//
// Per (batch, head): queries = the last obs <= 32 keys, logits = q . k * d^-0.5
// over all s keys, softmax over keys, importance = sum over queries, then mean
// over heads.  One wave owns a 32-query x 32-key logit tile at a time, computed
// with v_mfma_f32_32x32x8 (f16/bf16 inputs: products exact in fp32) or
// v_mfma_f32_32x32x2 (f32 inputs).  The K dimension is split so that lane group
// g = lane/32 supplies coordinates [g*d/2, (g+1)*d/2): each lane loads d bytes
// (f16) of one key row contiguously.  Accumulator register j of lane l holds
// the logit of query 8*(j/4) + 4*(l/32) + j%4 against key l%32 of the tile.
//
// Three sweeps over the keys recompute the logits instead of storing them:
// row maxima, row sums of exp(logit - max), then column sums of the
// probabilities; each sweep is split over key ranges so that every CU works.
#include "nq_common.h"

namespace nq {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kKeysPerWave = 256;  // 8 tiles of 32 keys per wave per sweep

struct KKArgs {
    const void* keys;        // [bh, seq, d]
    float* max_part;         // [bh, nsplit, 32]
    float* sum_part;         // [bh, nsplit, 32]
    float* row_max;          // [bh, 32] reduced over splits
    float* row_sum;          // [bh, 32]
    float* colsum;           // [bh, seq]
    float* importance;       // [batch, seq]
    int32_t seq, d, obs, nsplit, heads, batch;
    float scale;
};

template <int DT>
struct Elem;
template <>
struct Elem<NQ_F16> { static constexpr int bytes = 2; };
template <>
struct Elem<NQ_BF16> { static constexpr int bytes = 2; };
template <>
struct Elem<NQ_F32> { static constexpr int bytes = 4; };

// 32x32 logit tile: queries (rows) x keys (columns), K dimension = d.
// q_row / k_row: base of this lane's query / key row (elements), lane group g.
template <int DT, int D>
__device__ __forceinline__ f32x16 logit_tile(const char* q_row, const char* k_row, int g) {
    f32x16 acc = {};
    if constexpr (DT == NQ_F32) {
        const float* qa = reinterpret_cast<const float*>(q_row) + g * (D / 2);
        const float* kb = reinterpret_cast<const float*>(k_row) + g * (D / 2);
#pragma unroll
        for (int s = 0; s < D / 2; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[s], kb[s], acc, 0, 0, 0);
    } else {
        const uint2* qa = reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(q_row) + g * (D / 2));
        const uint2* kb = reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(k_row) + g * (D / 2));
#pragma unroll
        for (int s = 0; s < D / 8; ++s) {
            uint2 a = qa[s], b = kb[s];
            if constexpr (DT == NQ_F16) {
                acc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b),
                                                           acc, 0, 0, 0);
            } else {
                acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                               __builtin_bit_cast(bf16x4, b), acc, 0, 0, 0);
            }
        }
    }
    return acc;
}

__device__ __forceinline__ int acc_row(int j, int lane) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

// Reduce a per-lane value over the 32 lanes that share lane/32 (the key columns).
__device__ __forceinline__ float reduce32_max(float v) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float reduce32_sum(float v) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// SWEEP 0: row maxima; 1: row sums of exp; 2: column sums of probabilities.
template <int DT, int D, int SWEEP>
__global__ __launch_bounds__(64) void keykey_sweep(KKArgs a) {
    const int lane = threadIdx.x;
    const int g = lane >> 5;
    const int split = blockIdx.x;
    const int bh = blockIdx.y;
    const size_t row_bytes = (size_t)D * Elem<DT>::bytes;
    const char* base = static_cast<const char*>(a.keys) + (size_t)bh * a.seq * row_bytes;
    const int qi = lane & 31;
    const bool q_valid = qi < a.obs;
    const int q_pos = a.seq - a.obs + (q_valid ? qi : 0);
    const char* q_row = base + (size_t)q_pos * row_bytes;

    float m[16], z[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        m[j] = -__builtin_inff();
        z[j] = 0.0f;
    }
    if constexpr (SWEEP >= 1) {
        // global row statistics for this lane's 16 query rows
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = acc_row(j, lane);
            m[j] = a.row_max[(size_t)bh * 32 + r];
            if constexpr (SWEEP == 2) z[j] = a.row_sum[(size_t)bh * 32 + r];
        }
    }
    const int k0 = split * kKeysPerWave;
    const int k1 = min(a.seq, k0 + kKeysPerWave);
    for (int t0 = k0; t0 < k1; t0 += 32) {
        const int key = t0 + qi;
        const bool k_valid = key < k1;
        const char* k_row = base + (size_t)(k_valid ? key : k1 - 1) * row_bytes;
        f32x16 acc = logit_tile<DT, D>(q_row, k_row, g);
        float col = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = acc_row(j, lane);
            const bool ok = k_valid && r < a.obs;
            const float x = acc[j] * a.scale;
            if constexpr (SWEEP == 0) {
                if (ok) m[j] = __builtin_fmaxf(m[j], x);
            } else if constexpr (SWEEP == 1) {
                if (ok) z[j] += expf(x - m[j]);
            } else {
                if (ok) col += expf(x - m[j]) / z[j];
            }
        }
        if constexpr (SWEEP == 2) {
            col += __shfl_xor(col, 32, 64);
            if (g == 0 && k_valid) a.colsum[(size_t)bh * a.seq + key] = col;
        }
    }
    if constexpr (SWEEP <= 1) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float v = SWEEP == 0 ? reduce32_max(m[j]) : reduce32_sum(z[j]);
            if (qi == 0) {
                const int r = acc_row(j, lane);
                float* dst = SWEEP == 0 ? a.max_part : a.sum_part;
                dst[((size_t)bh * a.nsplit + split) * 32 + r] = v;
            }
        }
    }
}

// Reduce the per-split row statistics: MAX = 1 -> maxima, else sums (in split order).
template <bool MAX>
__global__ __launch_bounds__(32) void rowstat_reduce(const float* part, float* out, int nsplit) {
    const int bh = blockIdx.x, r = threadIdx.x;
    float v = MAX ? -__builtin_inff() : 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) {
        const float x = part[((size_t)bh * nsplit + sp) * 32 + r];
        v = MAX ? __builtin_fmaxf(v, x) : v + x;
    }
    out[(size_t)bh * 32 + r] = v;
}

__global__ __launch_bounds__(256) void head_mean_kernel(const float* colsum, float* importance, int batch, int heads,
                                                        int seq) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= seq) return;
    float s = 0.0f;
    for (int h = 0; h < heads; ++h) s += colsum[((size_t)b * heads + h) * seq + i];
    importance[(size_t)b * seq + i] = s / (float)heads;
}

template <int DT, int D>
static hipError_t launch_keykey(const KKArgs& a, hipStream_t st) {
    dim3 grid(a.nsplit, a.batch * a.heads);
    const int bh = a.batch * a.heads;
    hipLaunchKernelGGL((keykey_sweep<DT, D, 0>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL((rowstat_reduce<true>), dim3(bh), dim3(32), 0, st, a.max_part, a.row_max, a.nsplit);
    hipLaunchKernelGGL((keykey_sweep<DT, D, 1>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL((rowstat_reduce<false>), dim3(bh), dim3(32), 0, st, a.sum_part, a.row_sum, a.nsplit);
    hipLaunchKernelGGL((keykey_sweep<DT, D, 2>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL(head_mean_kernel, dim3((a.seq + 255) / 256, a.batch), dim3(256), 0, st, a.colsum,
                       a.importance, a.batch, a.heads, a.seq);
    return hipGetLastError();
}

template <int DT>
static hipError_t dispatch_keykey_d(const KKArgs& a, hipStream_t st) {
    switch (a.d) {
        case 64: return launch_keykey<DT, 64>(a, st);
        case 96: return launch_keykey<DT, 96>(a, st);
        case 128: return launch_keykey<DT, 128>(a, st);
        default: return launch_keykey<DT, 256>(a, st);
    }
}

// ---------------------------------------------------------------------------
// Real-attention scorer (reference: NexusQuantEvict._score_importance_real,
// pipeline.py:784-836, on transformers' eager attention, modeling_llama.py:
// 179-213 in transformers 5.15.0).  Per layer:
//   w = round_T(round_T(Q K^T) * scaling), causal, p = round_T(softmax_fp32(w)),
//   importance[b, j] += mean over query heads of sum_{i >= j} p[i, j]
// where round_T rounds to the model dtype (fp16 / bf16; identity for fp32) as
// the eager path does (matmul output, scaling multiply, softmax(...).to(dtype)).
// Query head h reads key head h / (hq / hkv) (repeat_kv).  Sweeps: row maxima
// and row sums per query tile (keys <= query), then column sums per key tile
// over the query tiles at or after it.
// ---------------------------------------------------------------------------

struct RealArgs {
    const void* q;     // [batch, hq, seq, d]
    const void* k;     // [batch, hkv, seq, d]
    float* row_max;    // [batch * hq, seq]
    float* row_sum;    // [batch * hq, seq]
    float* colsum;     // [batch * hq, seq]
    float* importance; // [batch, seq] accumulated
    int32_t seq, hq, hkv, batch;
    float scaling;
};

__device__ __forceinline__ float round_bf16(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;  // finite inputs: round to nearest even
    return __builtin_bit_cast(float, u);
}

template <int DT>
__device__ __forceinline__ float round_model(float x) {
    if constexpr (DT == NQ_F16) return __half2float(__float2half_rn(x));
    else if constexpr (DT == NQ_BF16) return round_bf16(x);
    else return x;
}

template <int DT, int D, int SWEEP>
__global__ __launch_bounds__(64) void real_sweep(RealArgs a) {
    const int lane = threadIdx.x;
    const int g = lane >> 5;
    const int col_lane = lane & 31;
    const int tile = blockIdx.x;  // query tile (sweeps 0, 1) or key tile (sweep 2)
    const int bhq = blockIdx.y;
    const int b = bhq / a.hq, hq = bhq - b * a.hq;
    const int hk = hq / (a.hq / a.hkv);
    const size_t row_bytes = (size_t)D * Elem<DT>::bytes;
    const char* qbase = static_cast<const char*>(a.q) + (size_t)bhq * a.seq * row_bytes;
    const char* kbase = static_cast<const char*>(a.k) + ((size_t)b * a.hkv + hk) * a.seq * row_bytes;
    const int n_tiles = (a.seq + 31) / 32;
    const size_t stat = (size_t)bhq * a.seq;

    if constexpr (SWEEP <= 1) {
        const int qt = tile;
        const int qi = qt * 32 + col_lane;  // query row this lane supplies to A
        const char* q_row = qbase + (size_t)(qi < a.seq ? qi : a.seq - 1) * row_bytes;
        float m[16], z[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = qt * 32 + acc_row(j, lane);
            m[j] = -__builtin_inff();
            z[j] = 0.0f;
            if constexpr (SWEEP == 1) m[j] = (i < a.seq) ? a.row_max[stat + i] : 0.0f;
        }
        for (int kt = 0; kt <= qt; ++kt) {
            const int key = kt * 32 + col_lane;
            const char* k_row = kbase + (size_t)(key < a.seq ? key : a.seq - 1) * row_bytes;
            f32x16 acc = logit_tile<DT, D>(q_row, k_row, g);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int i = qt * 32 + acc_row(j, lane);
                if (key <= i && i < a.seq) {
                    const float x = round_model<DT>(round_model<DT>(acc[j]) * a.scaling);
                    if constexpr (SWEEP == 0) m[j] = __builtin_fmaxf(m[j], x);
                    else z[j] += expf(x - m[j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float v = SWEEP == 0 ? reduce32_max(m[j]) : reduce32_sum(z[j]);
            const int i = qt * 32 + acc_row(j, lane);
            if (col_lane == 0 && i < a.seq) (SWEEP == 0 ? a.row_max : a.row_sum)[stat + i] = v;
        }
    } else {
        const int kt = tile;
        const int key = kt * 32 + col_lane;
        const char* k_row = kbase + (size_t)(key < a.seq ? key : a.seq - 1) * row_bytes;
        float col = 0.0f;
        for (int qt = kt; qt < n_tiles; ++qt) {
            const int qi = qt * 32 + col_lane;
            const char* q_row = qbase + (size_t)(qi < a.seq ? qi : a.seq - 1) * row_bytes;
            f32x16 acc = logit_tile<DT, D>(q_row, k_row, g);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int i = qt * 32 + acc_row(j, lane);
                if (key <= i && i < a.seq) {
                    const float x = round_model<DT>(round_model<DT>(acc[j]) * a.scaling);
                    const float p = expf(x - a.row_max[stat + i]) / a.row_sum[stat + i];
                    col += round_model<DT>(p);
                }
            }
        }
        col += __shfl_xor(col, 32, 64);
        if (g == 0 && key < a.seq) a.colsum[stat + key] = col;
    }
}

__global__ __launch_bounds__(256) void head_mean_accumulate(const float* colsum, float* importance, int hq,
                                                            int seq) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= seq) return;
    float s = 0.0f;
    for (int h = 0; h < hq; ++h) s += colsum[((size_t)b * hq + h) * seq + i];
    importance[(size_t)b * seq + i] += s / (float)hq;
}

template <int DT, int D>
static hipError_t launch_real(const RealArgs& a, hipStream_t st) {
    const int n_tiles = (a.seq + 31) / 32;
    dim3 grid(n_tiles, a.batch * a.hq);
    hipLaunchKernelGGL((real_sweep<DT, D, 0>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL((real_sweep<DT, D, 1>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL((real_sweep<DT, D, 2>), grid, dim3(64), 0, st, a);
    hipLaunchKernelGGL(head_mean_accumulate, dim3((a.seq + 255) / 256, a.batch), dim3(256), 0, st, a.colsum,
                       a.importance, a.hq, a.seq);
    return hipGetLastError();
}

template <int DT>
static hipError_t dispatch_real_d(int d, const RealArgs& a, hipStream_t st) {
    switch (d) {
        case 64: return launch_real<DT, 64>(a, st);
        case 96: return launch_real<DT, 96>(a, st);
        case 128: return launch_real<DT, 128>(a, st);
        default: return launch_real<DT, 256>(a, st);
    }
}

static int64_t keykey_ws_bytes(int64_t bh, int64_t seq) {
    const int64_t nsplit = (seq + kKeysPerWave - 1) / kKeysPerWave;
    return bh * nsplit * 32 * 4 * 2 + bh * 32 * 4 * 2 + bh * seq * 4;
}

}  // namespace nq

extern "C" int64_t nq_score_keykey_workspace(int32_t batch, int32_t heads, int32_t seq) {
    return nq::keykey_ws_bytes((int64_t)batch * heads, seq);
}

extern "C" int nq_score_keykey(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq,
                               int32_t head_dim, int32_t obs_window, float scale, float* importance,
                               void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(keys && importance && workspace, "nq_score_keykey: NULL pointer");
    NQ_CHECK_ARG(batch > 0 && heads > 0 && batch * heads <= 65535 && seq >= 0, "nq_score_keykey: bad shape");
    NQ_CHECK_ARG(head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256,
                 "nq_score_keykey: head_dim %d unsupported (64, 96, 128, 256)", head_dim);
    NQ_CHECK_ARG(dtype == NQ_F16 || dtype == NQ_BF16 || dtype == NQ_F32, "nq_score_keykey: bad dtype");
    NQ_CHECK_ARG(obs_window > 0, "nq_score_keykey: obs_window must be positive");
    if (seq == 0) return NQ_OK;
    const int64_t need = keykey_ws_bytes((int64_t)batch * heads, seq);
    NQ_CHECK_ARG(workspace_bytes >= need, "nq_score_keykey: workspace %lld bytes < %lld",
                 (long long)workspace_bytes, (long long)need);
    KKArgs a;
    a.keys = keys;
    a.seq = seq;
    a.d = head_dim;
    a.obs = obs_window < seq ? obs_window : seq;
    if (a.obs > 32) {
        set_error("nq_score_keykey: %d observation queries; this kernel takes at most 32", a.obs);
        return NQ_EUNSUPPORTED;
    }
    a.nsplit = (seq + kKeysPerWave - 1) / kKeysPerWave;
    a.heads = heads;
    a.batch = batch;
    a.scale = scale;
    char* ws = static_cast<char*>(workspace);
    const int64_t bh = (int64_t)batch * heads;
    a.max_part = reinterpret_cast<float*>(ws);
    a.sum_part = reinterpret_cast<float*>(ws + bh * a.nsplit * 32 * 4);
    a.row_max = reinterpret_cast<float*>(ws + bh * a.nsplit * 32 * 8);
    a.row_sum = reinterpret_cast<float*>(ws + bh * a.nsplit * 32 * 8 + bh * 32 * 4);
    a.colsum = reinterpret_cast<float*>(ws + bh * a.nsplit * 32 * 8 + bh * 32 * 8);
    a.importance = importance;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (dtype) {
        case NQ_F16: e = dispatch_keykey_d<NQ_F16>(a, st); break;
        case NQ_BF16: e = dispatch_keykey_d<NQ_BF16>(a, st); break;
        default: e = dispatch_keykey_d<NQ_F32>(a, st); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

extern "C" int64_t nq_score_real_workspace(int32_t batch, int32_t q_heads, int32_t seq) {
    return (int64_t)batch * q_heads * seq * 4 * 3;
}

extern "C" int nq_score_real(const void* q, const void* k, int32_t dtype, int32_t batch, int32_t q_heads,
                             int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling, float* importance,
                             void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(q && k && importance && workspace, "nq_score_real: NULL pointer");
    NQ_CHECK_ARG(batch > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
                 "nq_score_real: q_heads must be a positive multiple of kv_heads");
    NQ_CHECK_ARG((int64_t)batch * q_heads <= 65535 && seq >= 0, "nq_score_real: bad shape");
    NQ_CHECK_ARG(head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256,
                 "nq_score_real: head_dim %d unsupported (64, 96, 128, 256)", head_dim);
    NQ_CHECK_ARG(dtype == NQ_F16 || dtype == NQ_BF16 || dtype == NQ_F32, "nq_score_real: bad dtype");
    if (seq == 0) return NQ_OK;
    const int64_t need = nq_score_real_workspace(batch, q_heads, seq);
    NQ_CHECK_ARG(workspace_bytes >= need, "nq_score_real: workspace %lld bytes < %lld",
                 (long long)workspace_bytes, (long long)need);
    RealArgs a;
    a.q = q;
    a.k = k;
    const int64_t n = (int64_t)batch * q_heads * seq;
    a.row_max = static_cast<float*>(workspace);
    a.row_sum = a.row_max + n;
    a.colsum = a.row_sum + n;
    a.importance = importance;
    a.seq = seq;
    a.hq = q_heads;
    a.hkv = kv_heads;
    a.batch = batch;
    a.scaling = scaling;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (dtype) {
        case NQ_F16: e = dispatch_real_d<NQ_F16>(head_dim, a, st); break;
        case NQ_BF16: e = dispatch_real_d<NQ_BF16>(head_dim, a, st); break;
        default: e = dispatch_real_d<NQ_F32>(head_dim, a, st); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}
