// Decode attention straight from compressed pages (the vLLM compressor's
// int8 2p codes, fp16 row scales and int32 positions) on gfx950.
//
// The host cuts every sequence's pages into chunks of at most kChunk tokens;
// one workgroup of 4 waves takes one (chunk, kv head) and all G query heads
// that read that kv head, and writes a partial softmax state per query head:
// the chunk's running max m, its sum of exp l and the unnormalised value sum
// y.  A combine kernel merges the chunks of a row.
//
//  1. Keys, a quad of lanes per token (the page decoder's layout): exact
//     fp16 Walsh-Hadamard of the integer codes without the top stage, one
//     scale multiply, the merged top stage + forward RoPE at the stored
//     position, rounding to fp16 -- bit for bit the keys the page decoder
//     writes -- then q . k divided by fl(sqrt(head_dim)): a 16x16x32 fp16 MFMA
//     per 32 coordinates for fp16 queries with 8 heads per kv head, else
//     v_dot2_f32_f16 (fp16 queries) or fp32 FMAs.  Logits go to LDS.
//  2. Per query head the chunk max x_m of the unscaled logits and
//     e = exp((x - x_m) / scale_divisor), l = sum e (fixed order); LDS keeps
//     the weight e * scale_v / 2 per token as an fp16 pair hi + lo.
//  3. Values are never reconstructed per token: the inverse Hadamard is
//     linear, so sum_t e_t v_t = h_D * S (sum_t e_t (scale_t / 2) c_t) with
//     c_t the integer codes (exact in fp16).  The matrix cores accumulate
//     weights x codes over the chunk, 32 tokens per MFMA; the combine kernel
//     weights the chunks' sums, applies S and h_D once per (row, query head)
//     and divides by the softmax sum.
//
// Work items are (chunk, kv head) with the kv head fastest, and block 8k + x
// takes item x * per_xcd + k: the kv heads of one chunk run on one XCD and
// share the chunk's RoPE table rows in its L2.
//
// Against the reference (which rounds every decoded value to fp16 before the
// weighted sum, vllm_backend.py:748-763) the result differs by that rounding
// (below 2^-11 of a value, averaged by the weights) and by summation order.
#include "nq_rowmath.h"

namespace nq {

constexpr int kChunk = 512;  // tokens per chunk (logits held in LDS)

struct AttnArgs {
    const void* query;
    void* out;
    const int32_t* units;        // [unit * 16]: the unit records (see nq_attn_desc)
    const int32_t* chunk_units;  // [chunk + 1]
    const int32_t* chunk_row;
    const int32_t* chunk_tokens;
    const int32_t* row_chunks;   // [row + 1]
    float* part;                 // [chunk * q_heads * (D + 2)]: m, l, S y[D]
    const float* rope_cos;
    const float* rope_sin;
    const float* rope_dm;
    const float* rope_dp;
    uint32_t q_heads, kv_heads, rope_n_pos;
    uint32_t work, per_xcd;      // n_chunks * kv_heads items, ceil(work / 8)
    float inv_scale;             // 1 / scale_divisor
    float hscale;
};

// One unit record: up to 16 consecutive tokens of one page, addressed for kv
// head 0 (head kh adds kh * stride rows).
struct UnitRec {
    const int8_t* kc;
    const int8_t* vc;
    const uint16_t* ks;
    const uint16_t* vs;
    const int32_t* pos;
    int32_t stride, n, coff;
};

__device__ __forceinline__ UnitRec unit_rec(const AttnArgs& a, int u) {
    u = __builtin_amdgcn_readfirstlane(u);  // one record per wave: scalar loads
    const int4* r = reinterpret_cast<const int4*>(a.units + 16 * u);
    const int4 r0 = r[0], r1 = r[1], r2 = r[2];
    auto ptr = [](int lo, int hi) { return (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32); };
    UnitRec x;
    x.kc = gptr<const int8_t>(ptr(r0.x, r0.y));
    x.vc = gptr<const int8_t>(ptr(r0.z, r0.w));
    x.ks = gptr<const uint16_t>(ptr(r1.x, r1.y));
    x.vs = gptr<const uint16_t>(ptr(r1.z, r1.w));
    x.pos = gptr<const int32_t>(ptr(r2.x, r2.y));
    x.stride = r2.z;
    x.n = r2.w;
    x.coff = a.units[16 * u + 12];
    return x;
}

// int8 codes of one dword -> two exact fp16 pairs (see codes_to_f16 in nq_page.hip)
__device__ __forceinline__ void attn_codes_f16(uint32_t w, half2v& lo, half2v& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const half2v bias = {(__fp16)-1152.0f, (__fp16)-1152.0f};
    lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(u, 0x64646464u, 0x00050004u)) + bias;
    hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(u, 0x64646464u, 0x00070006u)) + bias;
}

template <int DT>
__device__ __forceinline__ float attn_load_f32(const void* p, size_t i) {
    if constexpr (DT == NQ_F32) return static_cast<const float*>(p)[i];
    else if constexpr (DT == NQ_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    else return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// wave-wide reductions (64 lanes) through LDS-free cross-lane moves
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int D, int G, int QDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 4 : 2))) void paged_attn_kernel(
    AttnArgs a) {
    constexpr int C = D / 32;
    constexpr bool QF16 = QDT == NQ_F16;
    __shared__ __attribute__((aligned(16))) float s_w[kChunk * G];  // [token][head]: logits, then e * scale_v / 2
    __shared__ float s_a[kChunk];       // scale_v / 2 per token
    __shared__ float s_red[4][G];   // per wave: each head's max, then
    __shared__ float s_sum[4][G];   // its sum of exp
    __shared__ float s_acc[4][G][D];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane & 3;
    const int quad = lane >> 2;
    const uint32_t w_item = (blockIdx.x & 7u) * a.per_xcd + (blockIdx.x >> 3);
    if (w_item >= a.work) return;  // whole block
    const uint32_t chunk = w_item / a.kv_heads;
    const uint32_t kh = w_item % a.kv_heads;
    const uint32_t row = (uint32_t)a.chunk_row[chunk];
    const int u0 = a.chunk_units[chunk], u1 = a.chunk_units[chunk + 1];
    const int n_tok = a.chunk_tokens[chunk] < kChunk ? a.chunk_tokens[chunk] : kChunk;

    // the G query heads of this kv head in LDS (fp16 queries as fp16, others as
    // fp32); every quad reads the same slices, so the reads are broadcasts
    using qreg_t = typename std::conditional<QF16, half2v, float>::type;
    constexpr int QR = QF16 ? 4 : 8;  // registers per 8 coordinates
    __shared__ __attribute__((aligned(16))) qreg_t s_q[G][C][4][QR];
    for (int i = threadIdx.x; i < G * D; i += 256) {
        const int g = i / D, j = i % D;
        const size_t qi = ((size_t)row * a.q_heads + kh * G + g) * D + j;
        const int c = j / 32, qq = (j / 8) % 4, k = j % 8;
        if constexpr (QF16) {
            reinterpret_cast<uint16_t*>(&s_q[g][c][qq][0])[k] = static_cast<const uint16_t*>(a.query)[qi];
        } else {
            s_q[g][c][qq][k] = attn_load_f32<QDT>(a.query, qi);
        }
    }
    __syncthreads();
    const float qsig = quad_sign(q);

    // fp16 queries with 8 heads per kv head take q . k on the matrix cores: per
    // unit and chunk c one 16x16x32 fp16 MFMA with the unit's 16 keys as the A
    // rows and the query heads as the B columns (heads 8..15 zero).  Lane l
    // holds B for head l % 16 over coordinates 32c + 8 (l / 16) .. + 7.
    constexpr bool QK_MFMA = QF16 && G == 8;
    half8v qb[QK_MFMA ? C : 1];
    if constexpr (QK_MFMA) {
        const int n = lane & 15, kg = lane >> 4;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const uint4 v = n < G ? *reinterpret_cast<const uint4*>(&s_q[n][c][kg][0]) : make_uint4(0u, 0u, 0u, 0u);
            qb[c] = __builtin_bit_cast(half8v, v);
        }
    }

    // ---- 1. keys and logits, one token per quad, 16 tokens per unit ----
    // The next unit's record and key codes are loaded while the current one is
    // decoded (indices clamped, so every load is unconditional and in bounds).
    struct KeyIn {
        uint2 w[C];
        uint32_t ks, vs;
        int32_t pos;
    };
    auto load_keys = [&](const UnitRec& r, KeyIn& k) {
        const int t = quad < r.n ? quad : 0;
        const size_t row = (size_t)kh * r.stride + t;
        const int8_t* crow = r.kc + row * D;
#pragma unroll
        for (int c = 0; c < C; ++c) k.w[c] = *reinterpret_cast<const uint2*>(crow + 32 * c + 8 * q);
        k.ks = r.ks[row];
        k.vs = r.vs[row];
        k.pos = r.pos[t];
    };
    int u = u0 + wave;
    UnitRec rc = unit_rec(a, u < u1 ? u : u0);
    KeyIn kin;
    load_keys(rc, kin);
    for (; u < u1; u += 4) {
        const int un = u + 4 < u1 ? u + 4 : u;
        const UnitRec rn = unit_rec(a, un);
        KeyIn knext;
        load_keys(rn, knext);

        const int t = quad;
        const bool valid = t < rc.n && rc.coff + t < kChunk;
        half2v h[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            attn_codes_f16(kin.w[c].x, h[c][0], h[c][1]);
            attn_codes_f16(kin.w[c].y, h[c][2], h[c][3]);
        }
        const float g = qsig * ((0.5f * f16_bits_to_f32(kin.ks)) * a.hscale);
        const uint32_t pos = kin.pos < 0 ? 0u : ((uint32_t)kin.pos >= a.rope_n_pos ? a.rope_n_pos - 1u : (uint32_t)kin.pos);
        float dm[C / 2][8], dp[C / 2][8];
        load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, pos, q, dm, dp);
        fwht_row_f16<C, false>(h, q);
        float x[C][8];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x[c][2 * k] = __builtin_fmaf((float)h[c][k].x, g, 0.0f);
                x[c][2 * k + 1] = __builtin_fmaf((float)h[c][k].y, g, 0.0f);
            }
        rope_stage_merged<C>(x, dm, dp);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) asm("" : "+v"(x[c][i]));  // fp32, then fp16: two roundings
        half2v kf[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) kf[c][k] = half2v{(__fp16)x[c][2 * k], (__fp16)x[c][2 * k + 1]};

        if constexpr (QK_MFMA) {
            // keys to the MFMA A layout: lane 16g + t takes token t's coordinates
            // 32c + 8g .. + 7 from lane 4t + g (the quad layout)
            const int addr_in = 4 * (4 * (lane & 15) + (lane >> 4));
            float4v lg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < C; ++c) {
                u32x4v bw;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    bw[k] = (uint32_t)__builtin_amdgcn_ds_bpermute(addr_in, (int)__builtin_bit_cast(uint32_t, kf[c][k]));
                lg = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, bw), qb[c], lg, 0, 0, 0);
            }
            // lane l holds the logits of tokens 4 (l / 16) + i for head l % 16
            const int n = lane & 15;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tt = 4 * (lane >> 4) + i;
                const float v = lg[i];
                if (n < G && tt < rc.n && rc.coff + tt < kChunk) s_w[(rc.coff + tt) * G + n] = v;
            }
        } else {
#pragma unroll
            for (int gq = 0; gq < G; ++gq) {
                float acc = 0.0f;
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    qreg_t qv[QR];
#pragma unroll
                    for (int k = 0; k < QR; ++k) qv[k] = s_q[gq][c][q][k];
                    if constexpr (QF16) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_fdot2(kf[c][k], qv[k], acc, false);
                    } else {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            acc = __builtin_fmaf((float)kf[c][k].x, qv[2 * k], acc);
                            acc = __builtin_fmaf((float)kf[c][k].y, qv[2 * k + 1], acc);
                        }
                    }
                }
                acc += dpp_f32<kQuadXor1>(acc);
                acc += dpp_f32<kQuadXor2>(acc);
                if (valid && q == 0) s_w[(rc.coff + t) * G + gq] = acc;
            }
        }
        if (valid && q == 1) s_a[rc.coff + t] = 0.5f * f16_bits_to_f32(kin.vs);
        rc = rn;
        kin = knext;
    }
    __syncthreads();

    // ---- 2. chunk max, exp, sum (fixed order) ----
    // s_w is [token][head]; a thread's entries i, i + 256, ... all belong to head
    // i % G (G divides 256), so lanes of one head reduce with xor offsets >= G.
    const int my_g = threadIdx.x % G;
    __shared__ float s_amax[4];
    {
        float v = -__builtin_inff();
        for (int i = threadIdx.x; i < n_tok * G; i += 256) v = __builtin_fmaxf(v, s_w[i]);
#pragma unroll
        for (int o = 32; o >= G; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
        if (lane < G) s_red[wave][lane] = v;
        float am = 0.0f;
        for (int t = threadIdx.x; t < n_tok; t += 256) am = __builtin_fmaxf(am, s_a[t]);
        am = wave_max(am);
        if (lane == 0) s_amax[wave] = am;
    }
    __syncthreads();
    // a head's chunk max and exp sum stay in LDS (read again for the output)
    auto head_max = [&](int gq) {
        return __builtin_fmaxf(__builtin_fmaxf(s_red[0][gq], s_red[1][gq]), __builtin_fmaxf(s_red[2][gq], s_red[3][gq]));
    };
    auto head_sum = [&](int gq) { return (s_sum[0][gq] + s_sum[1][gq]) + (s_sum[2][gq] + s_sum[3][gq]); };
    // Step 3 takes the weights e * scale_v / 2 as an fp16 pair hi + lo (22
    // significant bits), scaled by 2^(14 - x) where 2^x > the chunk's largest
    // scale_v / 2, so the largest weight sits just under 2^14 and small ones
    // stay clear of fp16's subnormals; the sum is scaled back by 2^(x - 14).
    int wexp = 0;
    {
        const float am = __builtin_fmaxf(__builtin_fmaxf(s_amax[0], s_amax[1]), __builtin_fmaxf(s_amax[2], s_amax[3]));
        if (am > 0.0f) (void)__builtin_frexpf(am, &wexp);
    }
    const float wmul = __builtin_ldexpf(1.0f, 14 - wexp);
    {
        const float mg = head_max(my_g);
        float v = 0.0f;
        for (int i = threadIdx.x; i < n_tok * G; i += 256) {
            const float e = expf((s_w[i] - mg) * a.inv_scale);
            v += e;
            const float w = (e * s_a[i / G]) * wmul;
            const __fp16 hi = (__fp16)w;
            const __fp16 lo = (__fp16)(w - (float)hi);
            s_w[i] = __builtin_bit_cast(float, half2v{hi, lo});
        }
#pragma unroll
        for (int o = 32; o >= G; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane < G) s_sum[wave][lane] = v;
    }
    __syncthreads();

    // ---- 3. values in the lattice domain, on the matrix cores ----
    // Per pair of units (32 tokens) and column block j one 16x16x32 fp16 MFMA
    // Y_j += W X_j: the K index is (unit, token), W's rows are (part, head) --
    // rows 0..G-1 the heads' hi weights, rows G..2G-1 their lo weights, the
    // rest zero -- and X_j's column n is coordinate NB * n + j.  Lane (n, kg)
    // holds the tokens 8 (kg & 1) .. + 7 of unit kg >> 1: NB consecutive code
    // bytes of each of those 8 rows (one load per row) and the matching weights.
    constexpr int NB = D / 16;
    using cword_t = typename std::conditional<NB == 4, uint32_t,
                                              typename std::conditional<NB == 8, uint2, uint4>::type>::type;
    const int n16 = lane & 15, kg = lane >> 4;
    const bool second = kg >= 2;
    const int tb = 8 * (kg & 1);
    const bool has_w = n16 < 2 * G;
    const int w_half = 2 * (n16 % G) + (n16 >= G ? 1 : 0);  // fp16 index within a token's G hi/lo pairs
    const _Float16* s_wh = reinterpret_cast<const _Float16*>(s_w);
    struct ValRec {
        const int8_t* vc;
        int32_t stride, n, nw, coff;
    };
    // this lane's unit of the pair (pu, pu + 1); a missing second unit reads the
    // first's rows under zero weights
    auto val_rec = [&](int pu) {
        const bool has_b = pu + 1 < u1;
        const UnitRec ra = unit_rec(a, pu);
        const UnitRec rb = unit_rec(a, has_b ? pu + 1 : pu);
        ValRec v;
        v.vc = second ? rb.vc : ra.vc;
        v.stride = second ? rb.stride : ra.stride;
        v.n = second ? rb.n : ra.n;
        v.coff = second ? rb.coff : ra.coff;
        int nw = second ? (has_b ? rb.n : 0) : ra.n;
        if (v.coff + nw > kChunk) nw = kChunk - v.coff;
        v.nw = nw;
        return v;
    };
    auto load_codes = [&](const ValRec& r, uint32_t (&cw)[8][NB / 4]) {
        const int8_t* base = r.vc + (size_t)kh * r.stride * D + NB * n16;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int t = tb + s < r.n ? tb + s : r.n - 1;
            const cword_t x = *reinterpret_cast<const cword_t*>(base + (size_t)t * D);
            const uint32_t* xw = reinterpret_cast<const uint32_t*>(&x);
#pragma unroll
            for (int w = 0; w < NB / 4; ++w) cw[s][w] = xw[w];
        }
    };
    float4v pacc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) pacc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const half2v bias = {(__fp16)-1152.0f, (__fp16)-1152.0f};
    u = u0 + 2 * wave;
    ValRec vr = val_rec(u < u1 ? u : u0);
    uint32_t ccur[8][NB / 4];
    load_codes(vr, ccur);
    for (; u < u1; u += 8) {
        const int un = u + 8 < u1 ? u + 8 : u;
        const ValRec vn = val_rec(un);
        uint32_t cnext[8][NB / 4];
        load_codes(vn, cnext);
        half8v wa;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const bool ok = has_w && tb + s < vr.nw;
            const _Float16 w = s_wh[ok ? 2 * G * (vr.coff + tb + s) + w_half : 0];
            wa[s] = ok ? w : (_Float16)0.0f;
        }
#pragma unroll
        for (int w = 0; w < NB / 4; ++w) {
            // bytes b of dword w of tokens 2p, 2p + 1 -> one fp16 pair of column block 4w + b
            uint32_t hb[4][4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t x0 = ccur[2 * p][w] ^ 0x80808080u, x1 = ccur[2 * p + 1][w] ^ 0x80808080u;
                const uint32_t lo = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // x0.b0 x1.b0 x0.b1 x1.b1
                const uint32_t hi = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // x0.b2 x1.b2 x0.b3 x1.b3
                hb[0][p] = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00050004u);
                hb[1][p] = __builtin_amdgcn_perm(lo, 0x64646464u, 0x00070006u);
                hb[2][p] = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00050004u);
                hb[3][p] = __builtin_amdgcn_perm(hi, 0x64646464u, 0x00070006u);
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                u32x4v xb;
#pragma unroll
                for (int p = 0; p < 4; ++p) xb[p] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, hb[b][p]) + bias);
                pacc[4 * w + b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, __builtin_bit_cast(half8v, xb),
                                                                          pacc[4 * w + b], 0, 0, 0);
            }
        }
        vr = vn;
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int w = 0; w < NB / 4; ++w) ccur[s][w] = cnext[s][w];
    }
    // lane l holds rows 4 kg + i of Y_j at column n16: a head's hi row plus its
    // lo row (G rows further: 4G lanes on for G >= 4, in the same lane below)
    constexpr int RI = G < 4 ? G : 4;  // rows of a lane that hold a head's hi sum
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            if constexpr (G >= 4) pacc[j][i] += __shfl_xor(pacc[j][i], 4 * G, 64);
            else pacc[j][i] += pacc[j][i + G];
        }
    if (4 * kg < G) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < RI; ++i) s_acc[wave][4 * kg + i][NB * n16 + j] = pacc[j][i];
    }
    __syncthreads();
    // the four waves' sums (fixed order), still in the lattice domain: the
    // combine kernel applies the Walsh-Hadamard S once per (row, head) to the
    // weighted sum of the chunks (S is linear)
    const float wunscale = __builtin_ldexpf(1.0f, wexp - 14);
    for (int i = threadIdx.x; i < G * D; i += 256) {
        const int gq = i / D, j = i % D;
        float* pp = a.part + ((size_t)chunk * a.q_heads + kh * G + gq) * (D + 2);
        pp[2 + j] = ((s_acc[0][gq][j] + s_acc[1][gq][j]) + (s_acc[2][gq][j] + s_acc[3][gq][j])) * wunscale;
        if (j == 0) {
            pp[0] = head_max(gq) * a.inv_scale;  // the chunk max in the scaled domain
            pp[1] = head_sum(gq);
        }
    }
}

// Merge the chunks of one (row, query head): a workgroup of 1024 threads,
// thread (group, column) summing the weighted y of every 32nd chunk for the
// D / 32 coordinates column + 32 i (independent chains, so a row of many
// chunks is not one long chain of dependent loads per thread); the groups are
// added in a fixed order, then the Walsh-Hadamard S (in LDS), h_D and the
// softmax sum turn the lattice-domain sum into the attended value.
template <int D, int QDT>
__global__ __launch_bounds__(1024) void paged_attn_combine(AttnArgs a) {
    constexpr int NG = 32, NI = D / 32;
    __shared__ float s_y[NG][D];
    __shared__ float s_l[NG];
    __shared__ float s_m[16];
    const uint32_t row = blockIdx.x / a.q_heads;
    const uint32_t qh = blockIdx.x % a.q_heads;
    const int c0 = a.row_chunks[row], c1 = a.row_chunks[row + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid >> 5, col = tid & 31;
    float M = -__builtin_inff();
    for (int c = c0 + tid; c < c1; c += 1024) M = __builtin_fmaxf(M, a.part[((size_t)c * a.q_heads + qh) * (D + 2)]);
    M = wave_max(M);
    if (lane == 0) s_m[wave] = M;
    __syncthreads();
    M = s_m[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) M = __builtin_fmaxf(M, s_m[w]);
    float y[NI], L = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) y[i] = 0.0f;
#pragma unroll 2
    for (int c = c0 + grp; c < c1; c += NG) {
        const float* pp = a.part + ((size_t)c * a.q_heads + qh) * (D + 2);
        const float f = expf(pp[0] - M);
#pragma unroll
        for (int i = 0; i < NI; ++i) y[i] = __builtin_fmaf(f, pp[2 + col + 32 * i], y[i]);
        L = __builtin_fmaf(f, pp[1], L);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) s_y[grp][col + 32 * i] = y[i];
    if (col == 0) s_l[grp] = L;
    __syncthreads();
    // the groups in order, into s_y[0]; then S over D, in place
    for (int j = tid; j < D; j += 1024) {
        float v = s_y[0][j];
#pragma unroll
        for (int g = 1; g < NG; ++g) v += s_y[g][j];
        s_y[0][j] = v;
    }
#pragma unroll
    for (int len = 1; len < D; len <<= 1) {
        __syncthreads();
        for (int p = tid; p < D / 2; p += 1024) {
            const int i = (p / len) * 2 * len + (p % len);
            const float x0 = s_y[0][i], x1 = s_y[0][i + len];
            s_y[0][i] = x0 + x1;
            s_y[0][i + len] = x0 - x1;
        }
    }
    __syncthreads();
    if (tid >= D) return;
    L = s_l[0];
#pragma unroll
    for (int g = 1; g < NG; ++g) L += s_l[g];
    const int j = tid;
    const size_t o = ((size_t)row * a.q_heads + qh) * D + j;
    // attended value, then fp16 (the reference's .to(float16)), then the output type
    const float val = c1 > c0 ? (s_y[0][j] * a.hscale) / L : 0.0f;
    const uint32_t hb = f32_to_f16_bits(val);
    if constexpr (QDT == NQ_F32) {
        static_cast<float*>(a.out)[o] = f16_bits_to_f32(hb);
    } else if constexpr (QDT == NQ_BF16) {
        // round to nearest even into bf16 (fp16 values are finite or inf)
        const uint32_t u = __builtin_bit_cast(uint32_t, f16_bits_to_f32(hb));
        static_cast<uint16_t*>(a.out)[o] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    } else {
        static_cast<uint16_t*>(a.out)[o] = (uint16_t)hb;
    }
}

template <int D, int G, int QDT>
static hipError_t launch_attn(const AttnArgs& a, uint32_t n_chunks, uint32_t batch, hipStream_t s) {
    if (n_chunks > 0) {
        hipLaunchKernelGGL((paged_attn_kernel<D, G, QDT>), dim3(a.per_xcd * 8u), dim3(256), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((paged_attn_combine<D, QDT>), dim3(batch * a.q_heads), dim3(1024), 0, s, a);
    return hipGetLastError();
}

template <int D, int QDT>
static hipError_t attn_groups(int G, const AttnArgs& a, uint32_t n_chunks, uint32_t batch, hipStream_t s) {
    switch (G) {
        case 1: return launch_attn<D, 1, QDT>(a, n_chunks, batch, s);
        case 2: return launch_attn<D, 2, QDT>(a, n_chunks, batch, s);
        case 4: return launch_attn<D, 4, QDT>(a, n_chunks, batch, s);
        default:
            if constexpr (QDT == NQ_F16) return launch_attn<D, 8, QDT>(a, n_chunks, batch, s);
            return hipErrorInvalidValue;
    }
}

template <int D>
static hipError_t attn_dtype(int qdt, int G, const AttnArgs& a, uint32_t n_chunks, uint32_t batch, hipStream_t s) {
    switch (qdt) {
        case NQ_F16: return attn_groups<D, NQ_F16>(G, a, n_chunks, batch, s);
        case NQ_BF16: return attn_groups<D, NQ_BF16>(G, a, n_chunks, batch, s);
        default: return attn_groups<D, NQ_F32>(G, a, n_chunks, batch, s);
    }
}

}  // namespace nq

extern "C" int32_t nq_paged_attention_chunk_tokens(void) { return nq::kChunk; }

extern "C" int64_t nq_paged_attention_workspace(int32_t n_chunks, int32_t q_heads, int32_t head_dim) {
    if (n_chunks <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
    return (int64_t)n_chunks * q_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

extern "C" int nq_paged_attention(const nq_attn_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_paged_attention: desc is NULL");
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_paged_attention: head_dim %d unsupported (64, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->batch >= 0 && d->q_heads > 0 && d->kv_heads > 0 && d->q_heads % d->kv_heads == 0,
                 "nq_paged_attention: q_heads %d must be a positive multiple of kv_heads %d", d->q_heads,
                 d->kv_heads);
    const int G = d->q_heads / d->kv_heads;
    NQ_CHECK_ARG(G == 1 || G == 2 || G == 4 || (G == 8 && d->q_dtype == NQ_F16),
                 "nq_paged_attention: %d query heads per kv head unsupported (1, 2, 4; 8 with fp16 queries)", G);
    NQ_CHECK_ARG(d->q_dtype == NQ_F16 || d->q_dtype == NQ_BF16 || d->q_dtype == NQ_F32,
                 "nq_paged_attention: unknown query dtype %d", d->q_dtype);
    NQ_CHECK_ARG(d->n_chunks >= 0, "nq_paged_attention: n_chunks %d", d->n_chunks);
    if (d->batch == 0) return NQ_OK;
    NQ_CHECK_ARG(d->query && d->out && d->row_chunks, "nq_paged_attention: query, out and row_chunks are required");
    if (d->n_chunks > 0) {
        NQ_CHECK_ARG(d->units && d->chunk_units && d->chunk_row && d->chunk_tokens,
                     "nq_paged_attention: chunk plan arrays are required");
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin && d->rope_n_pos > 0 && d->rope_n_pos < (1ll << 31),
                     "nq_paged_attention: keys need RoPE tables");
        NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                     "nq_paged_attention: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
        const int64_t need = nq_paged_attention_workspace(d->n_chunks, d->q_heads, d->head_dim);
        NQ_CHECK_ARG(d->workspace != nullptr && d->workspace_bytes >= need,
                     "nq_paged_attention: workspace of %lld bytes needed", (long long)need);
        NQ_CHECK_ARG((uint64_t)d->n_chunks * d->kv_heads + 8 <= max_blocks(256), "nq_paged_attention: grid too large");
        NQ_CHECK_ARG(d->scale_divisor > 0.0f, "nq_paged_attention: scale_divisor must be positive");
    }
    NQ_CHECK_ARG((uint64_t)d->batch * d->q_heads <= max_blocks(1024), "nq_paged_attention: grid too large");
    AttnArgs a = {};
    a.query = d->query;
    a.out = d->out;
    a.units = d->units;
    a.chunk_units = d->chunk_units;
    a.chunk_row = d->chunk_row;
    a.chunk_tokens = d->chunk_tokens;
    a.row_chunks = d->row_chunks;
    a.part = static_cast<float*>(d->workspace);
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.q_heads = (uint32_t)d->q_heads;
    a.kv_heads = (uint32_t)d->kv_heads;
    a.rope_n_pos = (uint32_t)(d->rope_n_pos > 0 ? d->rope_n_pos : 1);
    a.inv_scale = 1.0f / d->scale_divisor;
    a.hscale = d->hadamard_scale;
    a.work = (uint32_t)d->n_chunks * (uint32_t)d->kv_heads;
    a.per_xcd = (a.work + 7u) / 8u;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    switch (d->head_dim) {
        case 64: e = attn_dtype<64>(d->q_dtype, G, a, (uint32_t)d->n_chunks, (uint32_t)d->batch, s); break;
        case 128: e = attn_dtype<128>(d->q_dtype, G, a, (uint32_t)d->n_chunks, (uint32_t)d->batch, s); break;
        default: e = attn_dtype<256>(d->q_dtype, G, a, (uint32_t)d->n_chunks, (uint32_t)d->batch, s); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}
