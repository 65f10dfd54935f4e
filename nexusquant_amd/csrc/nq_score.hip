// Real-attention importance scorer on gfx950 MFMA (reference: NexusQuantEvict.
// _score_importance_real, pipeline.py:784-836, on transformers' eager attention).
// The key-key scorer is in nq_keykey.hip.
#include "nq_common.h"

namespace nq {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int DT>
struct Elem;
template <>
struct Elem<NQ_F16> { static constexpr int bytes = 2; };
template <>
struct Elem<NQ_BF16> { static constexpr int bytes = 2; };
template <>
struct Elem<NQ_F32> { static constexpr int bytes = 4; };

// 32x32 logit tile of the fp32 path: queries (rows) x keys (columns), K dimension = d;
// lane group g = lane/32 supplies coordinates [g*d/2, (g+1)*d/2) of its row.
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
    int32_t n_items, per_xcd;  // 128-row blocks x batch*hq; blocks per XCD range
    // sliding window (transformers' sliding_window_overlay): query i sees keys
    // j with i - window < j <= i; kNoWindow when the mask is plain causal
    int32_t window;
    // MAP instantiations: logit_map[bits of w] = bits of the model's
    // elementwise logit transform of w (soft-capping), 65536 entries in the
    // model dtype; monotone non-decreasing, so a row's maximum maps to the
    // maximum of the mapped logits
    const uint16_t* logit_map;
};

constexpr int32_t kNoWindow = 0x3fffffff;  // wider than any sequence, and 2 * it fits an int

// Block -> work item: consecutive block ids go round-robin to the 8 XCDs, so
// block 8k + x takes item x * per_xcd + k and each XCD walks one contiguous
// range of the item order (which keeps one operand set in its L2).
__device__ __forceinline__ int xcd_item(const RealArgs& a) {
    return (int)(blockIdx.x & 7u) * a.per_xcd + (int)(blockIdx.x >> 3);
}

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
                if (key <= i && i - key < a.window && i < a.seq) {
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
                if (key <= i && i - key < a.window && i < a.seq) {
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

// ---------------------------------------------------------------------------
// Real scorer, fp16 / bf16 models: workgroups of 4 waves on the gfx950
// 32x32x16 MFMA, one operand resident in registers and the other streamed
// through LDS tiles of 32 rows x D (rows padded by 16 bytes, so the 16-byte
// operand reads of 16 consecutive lanes hit 64 distinct banks).
//
// real_rowstats: a workgroup owns 128 query rows (wave w: rows 32w..32w+31 of
// the block) of one query head, held in registers as the MFMA B operand, and
// streams the key tiles 0..(last row)/32 once, keys as the A operand: a lane
// then holds one query's logits against 16 keys of the tile.  Each lane keeps
// the running maximum m of its raw logits (the rounding chain
// round_T(round_T(.) * scaling) is monotone, so it is applied to the maximum
// alone) and the sum z of exp(x - max) relative to it, rescaling z when m
// grows; lanes c and c + 32 (the same query) are combined at the end.  Writes
// -max * log2(e) and 1 / sum per row.
// real_colsum: a workgroup owns 128 keys (wave w: keys 32w..32w+31) as the B
// operand and streams the query tiles from its first key on; it accumulates
// round_T(exp(x - max) / sum) per key column in registers (fixed order, so the
// result does not depend on scheduling) and writes the column sums.
// exp is v_exp_f32 on x * log2(e) - max * log2(e) and the division a multiply
// by the row's reciprocal sum: within a few ulp of the eager fp32 softmax.
// ---------------------------------------------------------------------------

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;

template <int D>
struct RealTile {
    static constexpr int ROWB = 2 * D + 16;          // padded LDS row bytes
    static constexpr int ROWS = 64;                  // rows per LDS stage (two 32-row MFMA blocks)
    static constexpr int UNITS = ROWS * D / 8;       // 16-byte units per stage
    static constexpr int PER_THREAD = (UNITS + 255) / 256;
    static constexpr int KS = D / 16;                // MFMA K steps
    static constexpr int BUF = ROWS * ROWB;
};

template <int DT>
__device__ __forceinline__ f32x16 mfma16(uint4 a, uint4 b, f32x16 acc) {
    if constexpr (DT == NQ_F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                      acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
}

// 16-byte units of rows [row0, row0 + 64) of a [seq, D] matrix (rows clamped to seq - 1).
// Every thread loads PER_THREAD units unconditionally (UNITS is a multiple of
// 256 for every supported D), so the loads issue back to back and only the
// LDS store waits for them.
template <int D>
__device__ __forceinline__ void tile_load(const uint16_t* base, int row0, int seq, uint4 (&r)[RealTile<D>::PER_THREAD]) {
    static_assert(RealTile<D>::UNITS % 256 == 0, "64-row stages of 16-byte units fill 256 threads evenly");
#pragma unroll
    for (int k = 0; k < RealTile<D>::PER_THREAD; ++k) {
        const int u = threadIdx.x + 256 * k;
        int row = row0 + u / (D / 8);
        row = row < seq ? row : seq - 1;
        r[k] = *reinterpret_cast<const uint4*>(base + (size_t)row * D + (u % (D / 8)) * 8);
    }
}

template <int D>
__device__ __forceinline__ void tile_store(char* lds, const uint4 (&r)[RealTile<D>::PER_THREAD]) {
#pragma unroll
    for (int k = 0; k < RealTile<D>::PER_THREAD; ++k) {
        const int u = threadIdx.x + 256 * k;
        *reinterpret_cast<uint4*>(lds + (u / (D / 8)) * RealTile<D>::ROWB + (u % (D / 8)) * 16) = r[k];
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// vmcnt(0) with the other counters left open (gfx9 s_waitcnt encoding)
constexpr int kWaitVm0 = 0x0f70;

// Rows [row0, row0 + 64) of a [seq, D] matrix into one LDS stage by direct-to-LDS
// loads, in the padded layout tile_store writes (row r at r * ROWB).  The stage
// is UPR = ROWB / 16 windows of 64 16-byte slots; window w goes to wave w mod 4,
// and lane l of it fills slot 64 w + l: row (64 w + l) / UPR, unit
// (64 w + l) mod UPR, the pad unit (D / 8) masked off.  Nothing passes through
// registers, so a stage in flight costs no VGPRs; the caller waits (vmcnt) and
// then synchronises the workgroup.
//
// The lane's slots do not depend on the stage, so DmaPlan computes them once:
// the byte offset of each slot within a stage (row * 2D + 16 unit) and its
// row.  A full stage (row0 + 64 <= seq) then issues each load from the
// wave-uniform stage base plus that fixed offset; the last, partial stage
// clamps rows past seq to the last row.
template <int D>
struct DmaPlan {
    static constexpr int UPR = RealTile<D>::ROWB / 16;
    static constexpr int NW = (UPR + 3) / 4;  // windows per wave (the last may be empty)
    uint32_t off[NW];
    int row[NW];   // -1: pad slot or no window
    __device__ __forceinline__ DmaPlan() {
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const int w = 4 * k + wave;
            const int slot = 64 * w + lane;
            const int r = slot / UPR, u = slot - r * UPR;
            const bool ok = w < UPR && u < D / 8;
            row[k] = ok ? r : -1;
            off[k] = ok ? (uint32_t)(r * D * 2 + 16 * u) : 0u;
        }
    }
};

template <int D>
__device__ __forceinline__ void tile_dma(const DmaPlan<D>& plan, const uint16_t* base, int row0, int seq, char* buf) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const char* stage = reinterpret_cast<const char*>(base) + (size_t)row0 * D * 2;  // wave-uniform
    if (row0 + 64 <= seq) {
        // uniform base + 32-bit lane offset: the scalar-base form of the load, no VALU
#pragma unroll
        for (int k = 0; k < DmaPlan<D>::NW; ++k) {
            const int w = 4 * k + wave;
            if (w < DmaPlan<D>::UPR && plan.row[k] >= 0)
                __builtin_amdgcn_global_load_lds((global_void_t*)(stage + plan.off[k]), (lds_void_t*)(buf + 1024 * w),
                                                 16, 0, 0);
        }
    } else {
        const char* last = reinterpret_cast<const char*>(base) + (size_t)(seq - 1) * D * 2;
#pragma unroll
        for (int k = 0; k < DmaPlan<D>::NW; ++k) {
            const int w = 4 * k + wave;
            if (w < DmaPlan<D>::UPR && plan.row[k] >= 0) {
                // rows past seq read the last row (same unit)
                const char* src = row0 + plan.row[k] < seq ? stage + plan.off[k]
                                                           : last + (plan.off[k] - (uint32_t)plan.row[k] * D * 2);
                __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)(buf + 1024 * w), 16, 0, 0);
            }
        }
    }
}

// 32x32 logits: A from registers (this lane's row, K chunks), B from 32 LDS rows.
template <int DT, int D>
__device__ __forceinline__ f32x16 logits_regs_lds(const uint4 (&a)[RealTile<D>::KS], const char* lds, int c, int g) {
    f32x16 acc = {};
    const char* row = lds + c * RealTile<D>::ROWB + 16 * g;
#pragma unroll
    for (int s = 0; s < RealTile<D>::KS; ++s)
        acc = mfma16<DT>(a[s], *reinterpret_cast<const uint4*>(row + 32 * s), acc);
    return acc;
}

// 32x32 logits: A (queries) from 32 LDS rows, B (keys) from registers.
template <int DT, int D>
__device__ __forceinline__ f32x16 logits_lds_regs(const char* lds, const uint4 (&b)[RealTile<D>::KS], int c, int g) {
    f32x16 acc = {};
    const char* row = lds + c * RealTile<D>::ROWB + 16 * g;
#pragma unroll
    for (int s = 0; s < RealTile<D>::KS; ++s)
        acc = mfma16<DT>(*reinterpret_cast<const uint4*>(row + 32 * s), b[s], acc);
    return acc;
}

// this lane's K chunks of one row of a [seq, D] matrix (row clamped)
template <int D>
__device__ __forceinline__ void row_operand(const uint16_t* base, int row, int seq, int g, uint4 (&r)[RealTile<D>::KS]) {
    row = row < seq ? row : seq - 1;
    const uint16_t* p = base + (size_t)row * D + 8 * g;
#pragma unroll
    for (int s = 0; s < RealTile<D>::KS; ++s) r[s] = *reinterpret_cast<const uint4*>(p + 16 * s);
}

// x = round_T(round_T(logit) * scaling), both roundings kept (the empty asm
// stops the fp32 product and the second rounding from fusing into one
// mixed-precision instruction that would round once).
// Bits of a model-dtype value held exactly in an fp32 register, and back.
template <int DT>
__device__ __forceinline__ uint32_t model_bits(float x) {
    if constexpr (DT == NQ_F16) return (uint32_t)__builtin_bit_cast(uint16_t, (__fp16)x);  // exact
    else return __builtin_bit_cast(uint32_t, x) >> 16;                                     // exact
}
template <int DT>
__device__ __forceinline__ float from_model_bits(uint32_t h) {
    if constexpr (DT == NQ_F16) return (float)__builtin_bit_cast(__fp16, (uint16_t)h);
    else return __builtin_bit_cast(float, h << 16);
}

template <int DT, bool MAP = false>
__device__ __forceinline__ float eager_logit(float acc, float scaling, const uint16_t* map = nullptr) {
    float t = round_model<DT>(acc) * scaling;
    asm("" : "+v"(t));
    const float x = round_model<DT>(t);
    if constexpr (MAP) return from_model_bits<DT>(map[model_bits<DT>(x)]);
    return x;
}

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef __fp16 f16x2v __attribute__((ext_vector_type(2)));

// two fp32 -> packed fp16, round to nearest even: one v_cvt_pk_f16_f32,
// emitted by the compiler (not inline asm: the operands are often MFMA results
// held in VGPRs, and only compiler-visible reads get the MFMA-to-VALU wait states)
__device__ __forceinline__ f16x2v cvt_pk_f16(float lo, float hi) {
    typedef float f32x2v __attribute__((ext_vector_type(2)));
    typedef _Float16 h16x2v __attribute__((ext_vector_type(2)));
    const f32x2v v = {lo, hi};
    return __builtin_bit_cast(f16x2v, __builtin_convertvector(v, h16x2v));
}

// exp2 arguments of two logits: round_T(round_T(acc) * scaling) * log2(e) + nm,
// the roundings done on packed pairs.
// MAP: the pair goes through the logit map (two table reads) before the exp2
// arguments are formed.
template <int DT, bool MAP = false>
__device__ __forceinline__ void exp_args2(float a0, float a1, float scaling, float nm0, float nm1, float& o0,
                                          float& o1, const uint16_t* map = nullptr) {
    if constexpr (DT == NQ_F16) {
        const f16x2v h = cvt_pk_f16(a0, a1);
        float t0 = __builtin_fmaf((float)h.x, scaling, 0.0f), t1 = __builtin_fmaf((float)h.y, scaling, 0.0f);
        asm("" : "+v"(t0), "+v"(t1));
        f16x2v x = cvt_pk_f16(t0, t1);
        if constexpr (MAP) {
            const uint32_t bits = __builtin_bit_cast(uint32_t, x);
            x = __builtin_bit_cast(f16x2v, (uint32_t)map[bits & 0xffffu] | ((uint32_t)map[bits >> 16] << 16));
        }
        o0 = __builtin_fmaf((float)x.x, kLog2e, nm0);
        o1 = __builtin_fmaf((float)x.y, kLog2e, nm1);
    } else {
        const bf16x2v h = {(__bf16)a0, (__bf16)a1};
        float t0 = (float)h.x * scaling, t1 = (float)h.y * scaling;
        asm("" : "+v"(t0), "+v"(t1));
        bf16x2v x = {(__bf16)t0, (__bf16)t1};
        if constexpr (MAP) {
            const uint32_t bits = __builtin_bit_cast(uint32_t, x);
            x = __builtin_bit_cast(bf16x2v, (uint32_t)map[bits & 0xffffu] | ((uint32_t)map[bits >> 16] << 16));
        }
        o0 = __builtin_fmaf((float)x.x, kLog2e, nm0);
        o1 = __builtin_fmaf((float)x.y, kLog2e, nm1);
    }
}

// round_T of two fp32 values, packed (low = first)
template <int DT>
__device__ __forceinline__ uint32_t round_pair(float p0, float p1) {
    if constexpr (DT == NQ_F16) {
        return __builtin_bit_cast(uint32_t, cvt_pk_f16(p0, p1));
    } else {
        const bf16x2v h = {(__bf16)p0, (__bf16)p1};
        return __builtin_bit_cast(uint32_t, h);
    }
}

// Online row statistics of one lane (one query): fold the valid logits of a
// tile (raw dot products acc[j], j in [0, 16) x NT tiles; MASKED: only keys
// lo < acc_row(j) <= hi of the tile) into (mt, m, nm, z):
// mt the largest raw logit so far; m <= mt the reference the sum is kept
// against, nm = -round_T(round_T(m) * scaling) * log2(e); z = sum of
// exp2(x * log2(e) + nm) over the logits folded in.  The reference moves (and
// z is rescaled) only when a logit exceeds it by more than span, the raw
// logit distance whose exp2 argument is 32: every term stays below 2^32, the
// sum far from overflow, and most tiles skip the rescale.  The row's true
// maximum is applied once at the end.
template <int DT, int NT, bool MASKED, bool MAP = false, bool WIN = false>
__device__ __forceinline__ void row_fold(const f32x16 (&acc)[NT], float scaling, float span, int lo, int hi, int g,
                                         float& mt, float& m, float& nm, float& z, const uint16_t* map = nullptr) {
    auto valid = [&](int j) { return (!WIN || lo < acc_row(j, 32 * g)) && acc_row(j, 32 * g) <= hi; };
    float tm = -__builtin_inff();
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j)
            tm = fmaxf(tm, (!MASKED || valid(j)) ? acc[t][j] : -__builtin_inff());
    mt = fmaxf(mt, tm);
    if (tm > m + span) {  // per lane: move the reference to this tile's maximum, rescale the sum
        const float nm_new = -(eager_logit<DT, MAP>(tm, scaling, map) * kLog2e);
        z = m == -__builtin_inff() ? 0.0f : z * __builtin_amdgcn_exp2f(nm_new - nm);
        m = tm;
        nm = nm_new;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            float x0, x1;
            exp_args2<DT, MAP>(acc[t][j], acc[t][j + 1], scaling, nm, nm, x0, x1, map);
            const float e0 = __builtin_amdgcn_exp2f(x0), e1 = __builtin_amdgcn_exp2f(x1);
            if constexpr (MASKED) {
                z += valid(j) ? e0 : 0.0f;
                z += valid(j + 1) ? e1 : 0.0f;
            } else {
                z += e0;
                z += e1;
            }
        }
}

// Which rows of a wave's 32 queries [q0, q0 + 31] see the keys of 32-key tile
// kt under the causal mask with window W (query i sees i - W < key <= i):
// every row sees every key (whole), none does (none), or each lane tests its
// keys against (i - W - 32 kt, i - 32 kt] (the rest).
template <bool WIN>
__device__ __forceinline__ bool tile_whole(int kt, int my_diag, int q0, int W) {
    if constexpr (WIN) return kt < my_diag && kt * 32 > q0 + 31 - W;
    return kt < my_diag;
}
// tiles past the diagonal, and (WIN) tiles wholly left of the window
template <bool WIN>
__device__ __forceinline__ bool tile_left(int kt, int q0, int W) {
    if constexpr (WIN) return kt * 32 + 31 <= q0 - W;
    return false;
}

// WIN instantiations take a.window; the others fold the plain causal mask.
template <int DT, int D, bool MAP = false, bool WIN = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 4 : 1))) void real_rowstats(
    RealArgs a) {
    __shared__ __align__(16) char lds0[RealTile<D>::BUF];
    __shared__ __align__(16) char lds1[RealTile<D>::BUF];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 5, c = lane & 31;
    // items ordered (batch x kv head, query block from the last, query head of
    // the group): an XCD range covers whole KV groups, whose keys stay in its L2
    const int item = xcd_item(a);
    if (item >= a.n_items) return;
    const int n_blocks = (a.seq + 127) / 128;
    const int grp = a.hq / a.hkv;
    const int hh = item % grp;
    const int rest = item / grp;
    const int qb = n_blocks - 1 - rest % n_blocks;   // longest rows first
    const int bg = rest / n_blocks;                  // batch * hkv + kv head
    const int b = bg / a.hkv, hk = bg - b * a.hkv;
    const int hq = hk * grp + hh;
    const int bhq = b * a.hq + hq;
    const uint16_t* qbase = static_cast<const uint16_t*>(a.q) + (size_t)bhq * a.seq * D;
    const uint16_t* kbase = static_cast<const uint16_t*>(a.k) + ((size_t)b * a.hkv + hk) * a.seq * D;
    const int q0 = qb * 128 + wave * 32;             // this wave's first query row
    const bool live = q0 < a.seq;                    // wave-uniform
    const int my_diag = q0 / 32;                     // the key tile on this wave's diagonal
    const int last_key = min(qb * 128 + 127, a.seq - 1);
    const int n_it = last_key / 64 + 1;              // 64-key stages
    const int W = WIN ? a.window : kNoWindow;
    const int it_lo = WIN ? max(qb * 128 - W + 1, 0) / 64 : 0;  // the first stage any row of the block sees
    uint4 qa[RealTile<D>::KS];
    row_operand<D>(qbase, q0 + c, a.seq, g, qa);
    // this lane: query q0 + c, keys tile * 32 + acc_row(j, g)
    float mt = -__builtin_inff(), m = -__builtin_inff(), nm = 0.0f, z = 0.0f;
    // raw logit distance with exp2 argument 32 (|round_T| error is far below
    // it; a soft-cap map only shrinks distances)
    const float span = 32.0f / (a.scaling * kLog2e);
    const DmaPlan<D> plan;
    tile_dma<D>(plan, kbase, it_lo * 64, a.seq, lds0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    auto stage = [&](int it, const char* cur, char* nxt) {
        if (it + 1 < n_it) tile_dma<D>(plan, kbase, (it + 1) * 64, a.seq, nxt);
        if (live) {
            const int kt0 = 2 * it;
            // both tiles wholly before this wave's queries (and inside its window): no mask
            if (kt0 + 1 < my_diag && tile_whole<WIN>(kt0, my_diag, q0, W)) {
                f32x16 acc[2];
                acc[0] = logits_lds_regs<DT, D>(cur, qa, c, g);
                acc[1] = logits_lds_regs<DT, D>(cur + 32 * RealTile<D>::ROWB, qa, c, g);
                row_fold<DT, 2, false, MAP>(acc, a.scaling, span, 0, 0, g, mt, m, nm, z, a.logit_map);
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int kt = kt0 + h;
                    if (kt > my_diag) break;
                    if (tile_left<WIN>(kt, q0, W)) continue;
                    f32x16 acc[1];
                    acc[0] = logits_lds_regs<DT, D>(cur + h * 32 * RealTile<D>::ROWB, qa, c, g);
                    if (tile_whole<WIN>(kt, my_diag, q0, W))
                        row_fold<DT, 1, false, MAP>(acc, a.scaling, span, 0, 0, g, mt, m, nm, z, a.logit_map);
                    else  // query - W < key <= query
                        row_fold<DT, 1, true, MAP, WIN>(acc, a.scaling, span, q0 + c - W - 32 * kt, q0 + c - 32 * kt,
                                                        g, mt, m, nm, z, a.logit_map);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this thread's part of the next stage has landed
        __syncthreads();
    };
#pragma unroll 1
    for (int it = it_lo; it < n_it; it += 2) {
        stage(it, lds0, lds1);
        if (it + 1 < n_it) stage(it + 1, lds1, lds0);
    }
    if (!live) return;
    // lanes c and c + 32 hold the same query over disjoint keys: the row
    // maximum, and both sums moved from their references to it
    const float M = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float nmM = -(eager_logit<DT, MAP>(M, a.scaling, a.logit_map) * kLog2e);
    float zs = m == -__builtin_inff() ? 0.0f : z * __builtin_amdgcn_exp2f(nmM - nm);
    const float m_o = __shfl_xor(m, 32, 64), nm_o = __shfl_xor(nm, 32, 64), z_o = __shfl_xor(z, 32, 64);
    zs += m_o == -__builtin_inff() ? 0.0f : z_o * __builtin_amdgcn_exp2f(nmM - nm_o);
    const int i = q0 + c;
    if (g == 0 && i < a.seq) {
        const size_t stat = (size_t)bhq * a.seq;
        a.row_max[stat + i] = nmM;
        a.row_sum[stat + i] = 1.0f / zs;
    }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16(uint4 a, uint4 b, f32x4 acc) {
    if constexpr (DT == NQ_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                      acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
}

// Column sums of one 32 x 32 tile of a lane's key column (queries = rows
// acc_row(j, g)): p = round_T(exp2(x * log2(e) + nm[row]) * rz[row]) with x the
// eager logit, then colacc += P^T . B on the matrix cores with two 16x16x32
// MFMAs (8 rounded values per lane each).  As their A operand, lane l's 8
// values are row l % 16, K slice l / 16; that lane holds key l % 32 = row +
// 16 ((l / 16) & 1).  B (ones_sel) is 1 where column 0 meets the slices of key
// row and column 1 those of key row + 16, else 0, so column 0 of the result
// accumulates the sums of keys 0..15 and column 1 those of keys 16..31, in
// fp32.  That is half the matrix-core passes of summing against an all-ones
// 32x32x16 operand.  MASKED: rows r with r < key_off (row before the key) or
// r >= row_end (past seq, or at or past key + window) contribute 0.
template <int DT, bool MASKED, bool MAP = false>
__device__ __forceinline__ void col_fold(const f32x16& acc, const float* nm_rows, const float* rz_rows, float scaling,
                                         int key_off, int row_end, int g, const uint4& ones_sel, f32x4& colacc,
                                         const uint16_t* map = nullptr) {
    uint32_t pk[8];
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
        const int r0 = 8 * jq + 4 * g;  // rows r0 .. r0 + 3 of the 32-row block
        const float4 nm4 = *reinterpret_cast<const float4*>(&nm_rows[r0]);
        const float4 rz4 = *reinterpret_cast<const float4*>(&rz_rows[r0]);
        const float nm[4] = {nm4.x, nm4.y, nm4.z, nm4.w};
        const float rz[4] = {rz4.x, rz4.y, rz4.z, rz4.w};
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
            const int j = 4 * jq + u;
            float x0, x1;
            exp_args2<DT, MAP>(acc[j], acc[j + 1], scaling, nm[u], nm[u + 1], x0, x1, map);
            float p0 = __builtin_amdgcn_exp2f(x0) * rz[u];
            float p1 = __builtin_amdgcn_exp2f(x1) * rz[u + 1];
            if constexpr (MASKED) {
                const int r = r0 + u;
                p0 = key_off <= r && r < row_end ? p0 : 0.0f;
                p1 = key_off <= r + 1 && r + 1 < row_end ? p1 : 0.0f;
            }
            pk[j / 2] = round_pair<DT>(p0, p1);
        }
    }
    colacc = mfma16x16<DT>(make_uint4(pk[0], pk[1], pk[2], pk[3]), ones_sel, colacc);
    colacc = mfma16x16<DT>(make_uint4(pk[4], pk[5], pk[6], pk[7]), ones_sel, colacc);
}

template <int DT, int D, bool MAP = false, bool WIN = false>
__global__ __launch_bounds__(256) void real_colsum(RealArgs a) {
    __shared__ __align__(16) char lds0[RealTile<D>::BUF];
    __shared__ __align__(16) char lds1[RealTile<D>::BUF];
    __shared__ __align__(16) float st_nm0[64], st_rz0[64], st_nm1[64], st_rz1[64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 5, c = lane & 31;
    // items ordered (batch x query head, key block): an XCD range walks its
    // query heads one after the other, so the streamed queries stay in its L2
    const int item = xcd_item(a);
    if (item >= a.n_items) return;
    const int n_blocks = (a.seq + 127) / 128;
    const int kb = item % n_blocks;                  // first key blocks see the most queries
    const int bhq = item / n_blocks;
    const int b = bhq / a.hq, hq = bhq - b * a.hq;
    const int hk = hq / (a.hq / a.hkv);
    const uint16_t* qbase = static_cast<const uint16_t*>(a.q) + (size_t)bhq * a.seq * D;
    const uint16_t* kbase = static_cast<const uint16_t*>(a.k) + ((size_t)b * a.hkv + hk) * a.seq * D;
    const size_t stat = (size_t)bhq * a.seq;
    const int k0 = kb * 128 + wave * 32;            // this wave's first key
    const int key = k0 + c;
    const int my_first = k0 / 32;                    // first 32-row query block that sees these keys
    const int it0 = kb * 2;                          // first 64-row query stage of the block
    const int W = WIN ? a.window : kNoWindow;
    // one past the last 64-row stage holding a query that sees a key of the block
    // (key j is seen by queries j .. j + W - 1)
    const int n_it = WIN ? min((a.seq + 63) / 64, (kb * 128 + 126 + W) / 64 + 1) : (a.seq + 63) / 64;
    const bool live = k0 < a.seq;
    // a query tile is whole for this wave's keys [k0, k0 + 31] when all its rows
    // come after them, lie below seq and (WIN) before k0 + W; none when all its
    // rows come before the keys or (WIN) at or past k0 + 31 + W
    auto q_whole = [&](int qt) {
        return qt > my_first && qt * 32 + 32 <= a.seq && (!WIN || qt * 32 + 31 < k0 + W);
    };
    auto q_none = [&](int qt) { return qt < my_first || (WIN && qt * 32 >= k0 + 31 + W); };
    uint4 kr[RealTile<D>::KS];
    row_operand<D>(kbase, key, a.seq, g, kr);
    f32x4 colacc = {0.0f, 0.0f, 0.0f, 0.0f};
    // 16x16x32 B operand: column n of lane l is l % 16, its K slice l / 16; a
    // slice holds key (l % 32) = row + 16 ((l / 16) & 1), so column 0 sums the
    // slices of key row and column 1 those of key row + 16
    uint4 ones_sel;
    {
        constexpr uint32_t one2 = DT == NQ_F16 ? 0x3C003C00u : 0x3F803F80u;
        const uint32_t v = (lane & 15) == ((lane >> 4) & 1) ? one2 : 0u;
        ones_sel = make_uint4(v, v, v, v);
    }
    // One stage: 64 query rows by direct-to-LDS loads, and (wave 0) their row
    // statistics, one dword per lane.  Two buffers in fixed roles as in
    // real_rowstats; each thread waits for its own loads before the barrier.
    const DmaPlan<D> plan;
    auto load_stage = [&](int it, char* buf, float* nm, float* rz) {
        tile_dma<D>(plan, qbase, it * 64, a.seq, buf);
        if (wave == 0) {
            const int i = min(it * 64 + lane, a.seq - 1);
            __builtin_amdgcn_global_load_lds((global_void_t*)(a.row_max + stat + i), (lds_void_t*)nm, 4, 0, 0);
            __builtin_amdgcn_global_load_lds((global_void_t*)(a.row_sum + stat + i), (lds_void_t*)rz, 4, 0, 0);
        }
    };
    load_stage(it0, lds0, st_nm0, st_rz0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    auto stage = [&](int it, const char* cur, const float* cnm, const float* crz, char* nxt, float* nnm,
                     float* nrz) {
        if (it + 1 < n_it) load_stage(it + 1, nxt, nnm, nrz);
        if (live) {
            const int qt0 = 2 * it;
            if (qt0 > my_first && qt0 * 32 + 64 <= a.seq && (!WIN || qt0 * 32 + 63 < k0 + W)) {
                // both blocks interior: one basic block, so the second tile's
                // MFMAs run under the first tile's VALU work
                const f32x16 acc0 = logits_lds_regs<DT, D>(cur, kr, c, g);
                const f32x16 acc1 = logits_lds_regs<DT, D>(cur + 32 * RealTile<D>::ROWB, kr, c, g);
                col_fold<DT, false, MAP>(acc0, cnm, crz, a.scaling, 0, 0, g, ones_sel, colacc, a.logit_map);
                col_fold<DT, false, MAP>(acc1, cnm + 32, crz + 32, a.scaling, 0, 0, g, ones_sel, colacc,
                                         a.logit_map);
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int qt = qt0 + h;
                    if (q_none(qt)) continue;
                    const f32x16 acc = logits_lds_regs<DT, D>(cur + h * 32 * RealTile<D>::ROWB, kr, c, g);
                    if (q_whole(qt))
                        col_fold<DT, false, MAP>(acc, cnm + 32 * h, crz + 32 * h, a.scaling, 0, 0, g, ones_sel,
                                                 colacc, a.logit_map);
                    else
                        col_fold<DT, true, MAP>(acc, cnm + 32 * h, crz + 32 * h, a.scaling, key - qt * 32,
                                                WIN ? min(a.seq, key + W) - qt * 32 : a.seq - qt * 32, g, ones_sel,
                                                colacc, a.logit_map);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this thread's part of the next stage has landed
        __syncthreads();
    };
#pragma unroll 1
    for (int it = it0; it < n_it; it += 2) {
        stage(it, lds0, st_nm0, st_rz0, lds1, st_nm1, st_rz1);
        if (it + 1 < n_it) stage(it + 1, lds1, st_nm1, st_rz1, lds0, st_nm0, st_rz0);
    }
    // lane l (column n = l % 16 < 2) holds the sums of keys k0 + 4 (l / 16) + i + 16 n
    if ((lane & 15) < 2 && live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kk = k0 + 4 * (lane >> 4) + i + 16 * (lane & 15);
            if (kk < a.seq) a.colsum[stat + kk] = colacc[i];
        }
    }
}

// ---------------------------------------------------------------------------
// Attention output of the scoring pass, O = round_T(P V) with P the same
// rounded probabilities the column sums use (eager_attention_forward:
// matmul(softmax_fp32(w).to(T), repeat_kv(V))), without materialising P.
//
// The matrix cores contract over keys, so V is first written transposed, Vt
// [batch * hkv, D, s64] (s64 = seq rounded up to 64, zero past seq), with the
// keys of every 32-key block in "slot order": position 16 kk + 8 g + e holds
// key 16 kk + (e < 4 ? 4 g + e : 8 + 4 g + e - 4).  That is the order in which
// a logit accumulator lane (query c, half g) holds its keys (acc_row), so the
// lane's rounded probabilities are directly the A operand of the P V product
// (rows = queries, K = keys) and its B operand (K = keys, columns = D) is one
// 16-byte read of a Vt row.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int slot_key(int p) {  // key (within its 32-key block) at slot position p
    const int kk = p >> 4, g = (p >> 3) & 1, e = p & 7;
    return 16 * kk + (e < 4 ? 4 * g + e : 8 + 4 * g + e - 4);
}

// Vt rows of one 64-key stage of one (batch, kv head): V tile in LDS, then
// each thread packs 8 slot-ordered keys of one d into a 16-byte store.
template <int D>
__global__ __launch_bounds__(256) void vt_slots_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                       int seq, int s64) {
    __shared__ uint16_t tile[64][D + 2];
    const int st = blockIdx.x, bh = blockIdx.y;
    const uint16_t* src = v + (size_t)bh * seq * D;
    for (int u = threadIdx.x; u < 64 * D / 8; u += 256) {
        const int r = u / (D / 8), c8 = (u % (D / 8)) * 8;
        const int key = 64 * st + r;
        uint4 x = make_uint4(0u, 0u, 0u, 0u);
        if (key < seq) x = *reinterpret_cast<const uint4*>(src + (size_t)key * D + c8);
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tile[r][c8 + 2 * i] = (uint16_t)w[i];
            tile[r][c8 + 2 * i + 1] = (uint16_t)(w[i] >> 16);
        }
    }
    __syncthreads();
    uint16_t* dst = vt + (size_t)bh * D * s64 + 64 * st;
    for (int u = threadIdx.x; u < D * 8; u += 256) {
        const int d = u >> 3, p0 = (u & 7) * 8;  // slots p0 .. p0 + 7 of the stage
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int a = p0 + 2 * i, b = a + 1;
            const uint32_t lo = tile[32 * (a >> 5) + slot_key(a & 31)][d];
            const uint32_t hi = tile[32 * (b >> 5) + slot_key(b & 31)][d];
            w[i] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(dst + (size_t)d * s64 + p0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Direct-to-LDS plan for a 64-key stage of Vt: D rows of 128 bytes, padded to
// 144 in LDS (9 units, the last masked), windows of 64 units as in DmaPlan.
template <int D>
struct VtPlan {
    static constexpr int UPR = 9;
    static constexpr int ROWB = 144;
    static constexpr int WINDOWS = (D * UPR + 63) / 64;
    static constexpr int NW = (WINDOWS + 3) / 4;
    static constexpr int BUF = D * ROWB;
    uint32_t off[NW];
    bool ok[NW];
    __device__ __forceinline__ VtPlan(int s64) {
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const int w = 4 * k + wave;
            const int slot = 64 * w + lane;
            const int r = slot / UPR, u = slot - r * UPR;
            ok[k] = w < WINDOWS && r < D && u < 8;
            off[k] = ok[k] ? (uint32_t)(r * s64 * 2 + 16 * u) : 0u;
        }
    }
};

template <int D>
__device__ __forceinline__ void vt_dma(const VtPlan<D>& plan, const uint16_t* vt_bh, int it, char* buf) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const char* stage = reinterpret_cast<const char*>(vt_bh + 64 * it);  // wave-uniform
#pragma unroll
    for (int k = 0; k < VtPlan<D>::NW; ++k) {
        const int w = 4 * k + wave;
        if (w < VtPlan<D>::WINDOWS && plan.ok[k])
            __builtin_amdgcn_global_load_lds((global_void_t*)(stage + plan.off[k]), (lds_void_t*)(buf + 1024 * w), 16,
                                             0, 0);
    }
}

struct OutArgs {
    RealArgs r;
    const uint16_t* vt;  // [batch * hkv, D, s64]
    void* out;           // [batch, hq, seq, D] in the model dtype
    int32_t s64;
};

// Rounded probabilities of one 32 x 32 logit tile for this lane's query (nm,
// rz its row statistics), packed for the two 16-deep K steps of P V.
// MASKED: keys outside lo < acc_row(j, g) <= hi (the lane's query's window
// within the tile) are 0.
template <int DT, bool MASKED, bool MAP = false, bool WIN = false>
__device__ __forceinline__ void out_probs(const f32x16& acc, float nm, float rz, float scaling, int lo, int hi, int g,
                                          uint4 (&pa)[2], const uint16_t* map = nullptr) {
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
        float x0, x1;
        exp_args2<DT, MAP>(acc[j], acc[j + 1], scaling, nm, nm, x0, x1, map);
        float p0 = __builtin_amdgcn_exp2f(x0) * rz;
        float p1 = __builtin_amdgcn_exp2f(x1) * rz;
        if constexpr (MASKED) {
            p0 = (!WIN || lo < acc_row(j, 32 * g)) && acc_row(j, 32 * g) <= hi ? p0 : 0.0f;
            p1 = (!WIN || lo < acc_row(j + 1, 32 * g)) && acc_row(j + 1, 32 * g) <= hi ? p1 : 0.0f;
        }
        pk[j / 2] = round_pair<DT>(p0, p1);
    }
    pa[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    pa[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
}

// One 32-key tile of P V: for each 32-wide column block, two MFMAs (K = the
// tile's two slot-ordered key halves).  vbuf: the stage's Vt rows in LDS,
// tile t of the stage at byte 64 t of a row.
template <int DT, int D>
__device__ __forceinline__ void out_pv(const uint4 (&pa)[2], const char* vbuf, int t, int c, int g,
                                       f32x16 (&oacc)[D / 32]) {
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
        const char* row = vbuf + (32 * db + c) * VtPlan<D>::ROWB + 64 * t + 16 * g;
        oacc[db] = mfma16<DT>(pa[0], *reinterpret_cast<const uint4*>(row), oacc[db]);
        oacc[db] = mfma16<DT>(pa[1], *reinterpret_cast<const uint4*>(row + 32), oacc[db]);
    }
}

// A workgroup owns 128 query rows of one query head (wave w: rows 32 w ..),
// queries resident as the QK^T B operand as in real_rowstats, and streams
// 64-key stages of K (logits) and Vt (values) through two LDS buffers each.
template <int DT, int D, bool MAP = false, bool WIN = false>
__global__ __launch_bounds__(256) void real_output(OutArgs o) {
    __shared__ __align__(16) char k0buf[RealTile<D>::BUF];
    __shared__ __align__(16) char k1buf[RealTile<D>::BUF];
    __shared__ __align__(16) char v0buf[VtPlan<D>::BUF];
    __shared__ __align__(16) char v1buf[VtPlan<D>::BUF];
    const RealArgs& a = o.r;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 5, c = lane & 31;
    const int item = xcd_item(a);
    if (item >= a.n_items) return;
    const int n_blocks = (a.seq + 127) / 128;
    const int grp = a.hq / a.hkv;
    const int hh = item % grp;
    const int rest = item / grp;
    const int qb = n_blocks - 1 - rest % n_blocks;
    const int bg = rest / n_blocks;
    const int b = bg / a.hkv, hk = bg - b * a.hkv;
    const int hq = hk * grp + hh;
    const int bhq = b * a.hq + hq;
    const uint16_t* qbase = static_cast<const uint16_t*>(a.q) + (size_t)bhq * a.seq * D;
    const uint16_t* kbase = static_cast<const uint16_t*>(a.k) + ((size_t)b * a.hkv + hk) * a.seq * D;
    const uint16_t* vt_bh = o.vt + ((size_t)b * a.hkv + hk) * D * o.s64;
    const int q0 = qb * 128 + wave * 32;
    const bool live = q0 < a.seq;
    const int my_diag = q0 / 32;
    const int last_key = min(qb * 128 + 127, a.seq - 1);
    const int n_it = last_key / 64 + 1;
    const int W = WIN ? a.window : kNoWindow;
    const int it_lo = WIN ? max(qb * 128 - W + 1, 0) / 64 : 0;
    uint4 qa[RealTile<D>::KS];
    row_operand<D>(qbase, q0 + c, a.seq, g, qa);
    const size_t stat = (size_t)bhq * a.seq;
    const int qi = min(q0 + c, a.seq - 1);
    const float nm = a.row_max[stat + qi], rz = a.row_sum[stat + qi];
    f32x16 oacc[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) oacc[db] = f32x16{};
    const DmaPlan<D> kplan;
    const VtPlan<D> vplan(o.s64);
    tile_dma<D>(kplan, kbase, it_lo * 64, a.seq, k0buf);
    vt_dma<D>(vplan, vt_bh, it_lo, v0buf);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    auto stage = [&](int it, const char* ck, const char* cv, char* nk, char* nv) {
        if (it + 1 < n_it) {
            tile_dma<D>(kplan, kbase, (it + 1) * 64, a.seq, nk);
            vt_dma<D>(vplan, vt_bh, it + 1, nv);
        }
        if (live) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int kt = 2 * it + t;
                if (kt > my_diag) break;
                if (tile_left<WIN>(kt, q0, W)) continue;
                const f32x16 acc = logits_lds_regs<DT, D>(ck + t * 32 * RealTile<D>::ROWB, qa, c, g);
                uint4 pa[2];
                if (tile_whole<WIN>(kt, my_diag, q0, W))
                    out_probs<DT, false, MAP>(acc, nm, rz, a.scaling, 0, 0, g, pa, a.logit_map);
                else
                    out_probs<DT, true, MAP, WIN>(acc, nm, rz, a.scaling, q0 + c - W - 32 * kt, q0 + c - 32 * kt, g,
                                                  pa, a.logit_map);
                out_pv<DT, D>(pa, cv, t, c, g, oacc);
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
    };
#pragma unroll 1
    for (int it = it_lo; it < n_it; it += 2) {
        stage(it, k0buf, v0buf, k1buf, v1buf);
        if (it + 1 < n_it) stage(it + 1, k1buf, v1buf, k0buf, v0buf);
    }
    if (!live) return;
    // lane (c, g) holds O[q0 + acc_row(j, g)][32 db + c]
    uint16_t* out = static_cast<uint16_t*>(o.out) + (size_t)bhq * a.seq * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int qrow = q0 + acc_row(j, 32 * g);
            if (qrow < a.seq) {
                const float y = oacc[db][j];
                uint16_t h;
                if constexpr (DT == NQ_F16) h = __builtin_bit_cast(uint16_t, (__fp16)y);
                else h = (uint16_t)(__builtin_bit_cast(uint32_t, round_bf16(y)) >> 16);
                out[(size_t)qrow * D + 32 * db + c] = h;
            }
        }
}

// importance[b, i] += mean over heads of colsum[b, h, i], the heads summed in
// order; 64-thread blocks spread a row over many CUs, and the loads go out 8
// heads at a time ahead of their adds.
constexpr int kHeadMeanThreads = 64;

__global__ __launch_bounds__(kHeadMeanThreads) void head_mean_accumulate(const float* colsum, float* importance,
                                                                         int hq, int seq) {
    const int i = blockIdx.x * kHeadMeanThreads + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= seq) return;
    const float* col = colsum + (size_t)b * hq * seq + i;
    float s = 0.0f;
    int h = 0;
    for (; h + 8 <= hq; h += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = col[(size_t)(h + u) * seq];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; h < hq; ++h) s += col[(size_t)h * seq];
    importance[(size_t)b * seq + i] += s / (float)hq;
}

template <int DT, int D>
static hipError_t launch_real(const RealArgs& a, hipStream_t st) {
    if constexpr (DT == NQ_F32) {
        const int n_tiles = (a.seq + 31) / 32;
        dim3 grid(n_tiles, a.batch * a.hq);
        hipLaunchKernelGGL((real_sweep<DT, D, 0>), grid, dim3(64), 0, st, a);
        hipLaunchKernelGGL((real_sweep<DT, D, 1>), grid, dim3(64), 0, st, a);
        hipLaunchKernelGGL((real_sweep<DT, D, 2>), grid, dim3(64), 0, st, a);
    } else {
        RealArgs w = a;
        const int n_blocks = (a.seq + 127) / 128;
        w.n_items = n_blocks * a.batch * a.hq;
        w.per_xcd = (w.n_items + 7) / 8;
        dim3 grid(8 * w.per_xcd);
        if (a.logit_map) {
            hipLaunchKernelGGL((real_rowstats<DT, D, true, true>), grid, dim3(256), 0, st, w);
            hipLaunchKernelGGL((real_colsum<DT, D, true, true>), grid, dim3(256), 0, st, w);
        } else if (a.window != kNoWindow) {
            hipLaunchKernelGGL((real_rowstats<DT, D, false, true>), grid, dim3(256), 0, st, w);
            hipLaunchKernelGGL((real_colsum<DT, D, false, true>), grid, dim3(256), 0, st, w);
        } else {
            hipLaunchKernelGGL((real_rowstats<DT, D>), grid, dim3(256), 0, st, w);
            hipLaunchKernelGGL((real_colsum<DT, D>), grid, dim3(256), 0, st, w);
        }
    }
    hipLaunchKernelGGL(head_mean_accumulate, dim3((a.seq + kHeadMeanThreads - 1) / kHeadMeanThreads, a.batch),
                       dim3(kHeadMeanThreads), 0, st, a.colsum, a.importance, a.hq, a.seq);
    return hipGetLastError();
}

template <int DT, int D>
static hipError_t launch_attention(const RealArgs& a, const void* v, void* out, uint16_t* vt, int s64,
                                   bool with_importance, hipStream_t st) {
    RealArgs w = a;
    const int n_blocks = (a.seq + 127) / 128;
    w.n_items = n_blocks * a.batch * a.hq;
    w.per_xcd = (w.n_items + 7) / 8;
    dim3 grid(8 * w.per_xcd);
    const bool map = a.logit_map != nullptr, win = a.window != kNoWindow;
    if (map) hipLaunchKernelGGL((real_rowstats<DT, D, true, true>), grid, dim3(256), 0, st, w);
    else if (win) hipLaunchKernelGGL((real_rowstats<DT, D, false, true>), grid, dim3(256), 0, st, w);
    else hipLaunchKernelGGL((real_rowstats<DT, D>), grid, dim3(256), 0, st, w);
    if (with_importance) {
        if (map) hipLaunchKernelGGL((real_colsum<DT, D, true, true>), grid, dim3(256), 0, st, w);
        else if (win) hipLaunchKernelGGL((real_colsum<DT, D, false, true>), grid, dim3(256), 0, st, w);
        else hipLaunchKernelGGL((real_colsum<DT, D>), grid, dim3(256), 0, st, w);
        hipLaunchKernelGGL(head_mean_accumulate, dim3((a.seq + kHeadMeanThreads - 1) / kHeadMeanThreads, a.batch),
                           dim3(kHeadMeanThreads), 0, st, a.colsum, a.importance, a.hq, a.seq);
    }
    hipLaunchKernelGGL((vt_slots_kernel<D>), dim3(s64 / 64, a.batch * a.hkv), dim3(256), 0, st,
                       static_cast<const uint16_t*>(v), vt, a.seq, s64);
    OutArgs o;
    o.r = w;
    o.vt = vt;
    o.out = out;
    o.s64 = s64;
    if (map) hipLaunchKernelGGL((real_output<DT, D, true, true>), grid, dim3(256), 0, st, o);
    else if (win) hipLaunchKernelGGL((real_output<DT, D, false, true>), grid, dim3(256), 0, st, o);
    else hipLaunchKernelGGL((real_output<DT, D>), grid, dim3(256), 0, st, o);
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

}  // namespace nq

extern "C" int64_t nq_score_real_workspace(int32_t batch, int32_t q_heads, int32_t seq) {
    return (int64_t)batch * q_heads * seq * 4 * 3;
}

extern "C" int nq_score_real(const void* q, const void* k, int32_t dtype, int32_t batch, int32_t q_heads,
                             int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling, int32_t sliding_window,
                             const uint16_t* logit_map, float* importance, void* workspace, int64_t workspace_bytes,
                             void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(q && k && importance && workspace, "nq_score_real: NULL pointer");
    NQ_CHECK_ARG(sliding_window >= 0, "nq_score_real: negative sliding window");
    NQ_CHECK_ARG(logit_map == nullptr || dtype != NQ_F32,
                 "nq_score_real: a logit map takes fp16 or bf16 models (65536 model-dtype values)");
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
    a.window = sliding_window > 0 && sliding_window < kNoWindow ? sliding_window : kNoWindow;
    a.logit_map = logit_map;
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

extern "C" int64_t nq_attention_real_workspace(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t seq,
                                               int32_t head_dim) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0 || head_dim <= 0) return 0;
    const int64_t stats = (nq_score_real_workspace(batch, q_heads, seq) + 255) / 256 * 256;
    const int64_t s64 = ((int64_t)seq + 63) / 64 * 64;
    return stats + (int64_t)batch * kv_heads * head_dim * s64 * 2;
}

extern "C" int nq_attention_real(const void* q, const void* k, const void* v, int32_t dtype, int32_t batch,
                                 int32_t q_heads, int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling,
                                 int32_t sliding_window, const uint16_t* logit_map, float* importance, void* out,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(q && k && v && out && workspace, "nq_attention_real: NULL pointer");
    NQ_CHECK_ARG(sliding_window >= 0, "nq_attention_real: negative sliding window");
    NQ_CHECK_ARG(batch > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
                 "nq_attention_real: q_heads must be a positive multiple of kv_heads");
    NQ_CHECK_ARG((int64_t)batch * q_heads <= 65535 && seq >= 0, "nq_attention_real: bad shape");
    NQ_CHECK_ARG(head_dim == 64 || head_dim == 128, "nq_attention_real: head_dim %d unsupported (64, 128)",
                 head_dim);
    NQ_CHECK_ARG(dtype == NQ_F16 || dtype == NQ_BF16, "nq_attention_real: dtype must be fp16 or bf16");
    NQ_CHECK_ARG((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)workspace) & 15) == 0,
                 "nq_attention_real: tensors must be 16-byte aligned");
    if (seq == 0) return NQ_OK;
    NQ_CHECK_ARG((int64_t)seq * head_dim < (1ll << 31), "nq_attention_real: seq too long");
    const int64_t need = nq_attention_real_workspace(batch, q_heads, kv_heads, seq, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= need, "nq_attention_real: workspace %lld bytes < %lld",
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
    a.window = sliding_window > 0 && sliding_window < kNoWindow ? sliding_window : kNoWindow;
    a.logit_map = logit_map;
    const int64_t stats = (nq_score_real_workspace(batch, q_heads, seq) + 255) / 256 * 256;
    uint16_t* vt = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + stats);
    const int s64 = (seq + 63) / 64 * 64;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    const bool imp = importance != nullptr;
    if (dtype == NQ_F16)
        e = head_dim == 64 ? launch_attention<NQ_F16, 64>(a, v, out, vt, s64, imp, st)
                           : launch_attention<NQ_F16, 128>(a, v, out, vt, s64, imp, st);
    else
        e = head_dim == 64 ? launch_attention<NQ_BF16, 64>(a, v, out, vt, s64, imp, st)
                           : launch_attention<NQ_BF16, 128>(a, v, out, vt, s64, imp, st);
    NQ_CHECK_HIP(e);
    return NQ_OK;
}
