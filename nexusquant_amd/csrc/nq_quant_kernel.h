// Fused row quantizer for gfx950, the kernel template shared by nq_quant.hip
// (entry points, plain instantiations), nq_quant_list.hip (row-list
// instantiations) and nq_quant_gather.hip (gather instantiations): inverse
// RoPE -> Walsh-Hadamard -> per-row scale -> relaxed E8 -> packed codes, and
// the drop-in reconstruction (inverse Hadamard -> rescale -> forward RoPE ->
// fp16) in the same pass.
//
// Layout: one row (one head vector of one token, D <= 256 padded coordinates)
// is owned by a quad of 4 lanes.  Lane q of the quad holds C = D/32 chunks of 8
// consecutive coordinates, chunk c covering coordinates 32c + 8q .. 32c + 8q + 7.
// So an E8 group (8 consecutive coordinates) is one chunk of one lane, the RoPE
// pair (i, i + D/2) is chunk c and c + C/2 of the same lane, and of the
// log2(D) Hadamard butterfly stages the stages on coordinate bits 0-2 and
// 5.. are lane-local while the stages on bits 3 and 4 cross lanes inside the
// quad through DPP quad permutes.  A quad reads/writes 64 contiguous bytes of
// a fp16 row per chunk, and a 256-thread block owns 64 rows.
//
// Arithmetic follows oracle/nq_spec.c step by step (no FMA contraction: the
// file is compiled with -ffp-contract=off; the explicit fmaf calls below are
// exact sign-folded butterflies or the correctly rounded division refinement).
#pragma once

#include "nq_rowmath.h"

namespace nq {

// Per-tensor device address tables (n_tensors entries each; null when the
// output is not written).  The kernel takes them as __restrict__ arguments so
// that, being read-only, their entries load into scalar registers inside the
// sub-item loop.
struct QuantTables {
    const uint64_t* src;
    const uint64_t* recon;
    const uint64_t* syms;
    const uint64_t* cosets;
    const uint64_t* scales;
    const uint64_t* positions;  // pages: per tensor int32 [page_tokens] (keys)
    const uint64_t* codes8;     // pages: per tensor int8 [rows, D]: 2p
    const uint64_t* scales16;   // pages: per tensor fp16 [rows]
};

struct QuantArgs {
    const int32_t* gather;
    const uint8_t* keep;
    const float* rope_cos;
    const float* rope_sin;
    const float* rope_dm;   // optional fl(sin - cos) / fl(cos + sin) tables
    const float* rope_dp;
    uint32_t heads, seq_in, seq_out, n_tensors;
    uint32_t batch, hn, group, n_groups;    // hn = heads * n_tensors sub-items per batch row, in groups
    uint32_t n_tiles, work, per_xcd;        // work items = n_tiles * batch * n_groups, n_tiles = ceil(seq_out/64)
    float hscale;
    int32_t keep_mode;                      // NQ_KEEP_*
    // page encoding (PAGE instantiations only): rows are a page's (head, token)
    // rows flattened, token = row % page_tokens; keys rotate at positions[token]
    uint32_t page_tokens;
    uint32_t rope_n_pos;
    // row list (mask eviction): per batch row a permutation of its positions,
    // the n_kept[b] kept ones first; output row = source row = the listed position
    const int32_t* order;
    const int32_t* n_kept;
};

// ------------------------------------------------------------------ E8 ----

// min(|e0|, ..., |e7|) in four min3/min instructions.  Written in asm because
// the compiler otherwise quiets every |e| (a max with itself) before the min.
__device__ __forceinline__ float min8_abs(const float (&e)[8]) {
    float m1, m2, m3, m;
    asm("v_min3_f32 %0, |%1|, |%2|, |%3|" : "=v"(m1) : "v"(e[0]), "v"(e[1]), "v"(e[2]));
    asm("v_min3_f32 %0, |%1|, |%2|, |%3|" : "=v"(m2) : "v"(e[3]), "v"(e[4]), "v"(e[5]));
    asm("v_min3_f32 %0, |%1|, |%2|, %3" : "=v"(m3) : "v"(e[6]), "v"(e[7]), "v"(m1));
    asm("v_min_f32 %0, %1, %2" : "=v"(m) : "v"(m2), "v"(m3));
    return m;
}

// r += d in the lanes of `mask` only: one VALU instruction under a narrowed
// EXEC, restored inside the same asm block.
__device__ __forceinline__ void add_in_lanes(float& r, float d, uint64_t mask) {
    uint64_t saved;
    asm volatile("s_and_saveexec_b64 %1, %2\n\t"
                 "v_add_f32 %0, %0, %3\n\t"
                 "s_mov_b64 exec, %1"
                 : "+v"(r), "=&s"(saved)
                 : "s"(mask), "v"(d));
}

// r[j] = rint(x[j] - 0.5) in the lanes of `mask` only.
__device__ __forceinline__ void half_candidates_in_lanes(float (&r)[8], const float (&x)[8], uint64_t mask) {
    uint64_t saved;
    asm volatile("s_and_saveexec_b64 %8, %9\n\t"
                 "v_add_f32 %0, -0.5, %10\n\t"
                 "v_add_f32 %1, -0.5, %11\n\t"
                 "v_add_f32 %2, -0.5, %12\n\t"
                 "v_add_f32 %3, -0.5, %13\n\t"
                 "v_add_f32 %4, -0.5, %14\n\t"
                 "v_add_f32 %5, -0.5, %15\n\t"
                 "v_add_f32 %6, -0.5, %16\n\t"
                 "v_add_f32 %7, -0.5, %17\n\t"
                 "v_rndne_f32 %0, %0\n\t"
                 "v_rndne_f32 %1, %1\n\t"
                 "v_rndne_f32 %2, %2\n\t"
                 "v_rndne_f32 %3, %3\n\t"
                 "v_rndne_f32 %4, %4\n\t"
                 "v_rndne_f32 %5, %5\n\t"
                 "v_rndne_f32 %6, %6\n\t"
                 "v_rndne_f32 %7, %7\n\t"
                 "s_mov_b64 exec, %8"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]),
                   "+v"(r[7]), "=&s"(saved)
                 : "s"(mask), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]),
                   "v"(x[6]), "v"(x[7]));
}

// Relaxed E8 decision for one group (oracle/nq_spec.c nqs_e8_group).  x holds
// the normalised coordinates, already clamped to [-L/2, L/2].  On return x
// holds the chosen candidate before the coset offset and the final clamp:
// the integer point r (with the odd-sum step applied) when the integer coset
// wins, rint(x - 0.5) when the half coset wins (the caller adds 1/2).  The
// odd-sum step goes to the first coordinate whose |x - r| equals the group
// minimum, which is the reference's first argmin, and moves toward x (+1 on a
// zero gap: x - r is never -0).  Returns the half-coset flag.
__device__ __forceinline__ bool e8_select(float (&x)[8]) {
    float r[8], e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        r[j] = __builtin_rintf(x[j]);
        e[j] = x[j] - r[j];
    }
    const float rsum = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));  // exact
    const bool odd = ((int)rsum & 1) != 0;
    const float amin = min8_abs(e);
    const float asum = ((__builtin_fabsf(e[0]) + __builtin_fabsf(e[1])) +
                        (__builtin_fabsf(e[2]) + __builtin_fabsf(e[3]))) +
                       ((__builtin_fabsf(e[4]) + __builtin_fabsf(e[5])) +
                        (__builtin_fabsf(e[6]) + __builtin_fabsf(e[7])));
    const float thr = odd ? __builtin_fmaf(2.0f, amin, 1.0f) : 2.0f;  // 1 + 2*amin, one rounding
    const bool use_half = asum > thr;
    const uint64_t half_lanes = __builtin_amdgcn_ballot_w64(use_half);
    const uint64_t pending = __builtin_amdgcn_ballot_w64(odd) & ~half_lanes;
    uint64_t seen = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint64_t eq = __builtin_amdgcn_ballot_w64(__builtin_fabsf(e[j]) == amin);
        add_in_lanes(r[j], __builtin_copysignf(1.0f, e[j]), eq & pending & ~seen);
        seen |= eq;
    }
    half_candidates_in_lanes(r, x, half_lanes);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = r[j];
    return use_half;
}

// --------------------------------------------------------------- codes ----

template <int L, int C>
__device__ __forceinline__ void store_symbols(uint8_t* row_syms, int q, const float (&p)[C][8],
                                              const int (&coset)[C]) {
    constexpr int B = SymBits<L>::value;
    constexpr float HL = (float)(L / 2);
    constexpr bool ODD_HL = ((L / 2) & 1) != 0;
    constexpr int NB = C * B;  // bytes owned by this lane
    uint64_t slot[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const float adj = (ODD_HL && coset[c]) ? 0.5f : 0.0f;
        uint64_t v = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t s = (uint32_t)(p[c][j] + (HL + adj));
            v |= (uint64_t)s << (B * j);
        }
        slot[c] = v;
    }
    uint8_t* dst = row_syms + q * NB;
    if constexpr (B == 4) {
        uint32_t w[C];
#pragma unroll
        for (int c = 0; c < C; ++c) w[c] = (uint32_t)slot[c];
        if constexpr (C == 2) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
        } else {
#pragma unroll
            for (int c = 0; c < C; c += 4)
                *reinterpret_cast<uint4*>(dst + 4 * c) = make_uint4(w[c], w[c + 1], w[c + 2], w[c + 3]);
        }
    } else {
        uint8_t bytes[NB];
#pragma unroll
        for (int c = 0; c < C; ++c) {
#pragma unroll
            for (int m = 0; m < B; ++m) bytes[c * B + m] = (uint8_t)(slot[c] >> (8 * m));
        }
        if constexpr (NB % 4 == 0) {
#pragma unroll
            for (int k = 0; k < NB; k += 4) {
                uint32_t w = (uint32_t)bytes[k] | ((uint32_t)bytes[k + 1] << 8) |
                             ((uint32_t)bytes[k + 2] << 16) | ((uint32_t)bytes[k + 3] << 24);
                *reinterpret_cast<uint32_t*>(dst + k) = w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < NB; k += 2) {
                uint16_t w = (uint16_t)(bytes[k] | (bytes[k + 1] << 8));
                *reinterpret_cast<uint16_t*>(dst + k) = w;
            }
        }
    }
}

// ------------------------------------------------- packed lattice points ----
//
// For D * L <= 1024 and levels <= 8 the chosen candidates are carried as
// packed fp16 pairs (coordinate k, k + 4 of a group in register k) of
//   U = clamp01((p + L/2) / L),
// computed in one v_pk_fma_f16 with the clamp bit: p is the candidate plus the
// coset offset, so the clamp is the reference's clamp to [-L/2, L/2].  Every
// value is a multiple of 1/(2L) in [0, 1], exact in fp16.

__device__ __forceinline__ uint32_t pk_fma_clamp(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t d;
    asm("v_pk_fma_f16 %0, %1, %2, %3 clamp" : "=v"(d) : "v"(a), "s"(b), "v"(c));
    return d;
}

__device__ __forceinline__ uint32_t pk_f16_bits(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

__device__ __forceinline__ uint32_t splat_f16(float v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (__fp16)v);
    return h | (h << 16);
}

// Symbols of one group from its four U registers.  sym = p + L/2 (integer
// coset), floor(p) + L/2 (half coset, L/2 even) or ceil(p) + L/2 (L/2 odd).
// S = U * (L * 2^-23) + c * 2^-24 is an exact fp16 subnormal whose bit pattern
// is the integer 2(p + L/2) + c (c = 1 only for L = 2), so sym = bits >> 1 in
// every case (the shift is the floor of half-coset points).  Returns the
// group's 8 symbols, symbol j at bit j * bits.
template <int L>
__device__ __forceinline__ uint32_t group_symbols(const uint32_t (&u)[4]) {
    constexpr int B = SymBits<L>::value;
    const half2v scl = {(__fp16)(L * 0x1p-23f), (__fp16)(L * 0x1p-23f)};
    const half2v off = L == 2 ? half2v{(__fp16)0x1p-24f, (__fp16)0x1p-24f} : half2v{(__fp16)0.0f, (__fp16)0.0f};
    uint32_t d[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        d[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2v, u[k]), scl, off));
    if constexpr (B == 4 || B == 3) {
        // fields 2(p + L/2) at bits 0 and 16 of each register; the low bit (set
        // for half-coset points) is dropped so it cannot reach the neighbour
        uint32_t m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = d[k] & 0xfffefffeu;
        if constexpr (B == 4) {
            return (m[0] >> 1) | (m[1] << 3) | (m[2] << 7) | (m[3] << 11);
        } else {
            const uint32_t t = (m[0] >> 1) | (m[1] << 2) | (m[2] << 5) | (m[3] << 8);  // s0..3 @0, s4..7 @16
            return (t & 0xfffu) | ((t >> 4) & 0xfff000u);
        }
    } else {
        static_assert(B == 2, "packed symbols implemented for 2, 3 and 4 bits");
        uint32_t m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = d[k] & 0x00060006u;  // drop the +1 bit
        const uint32_t t = (m[0] >> 1) | (m[1] << 1) | (m[2] << 3) | (m[3] << 5);  // s0..3 @0, s4..7 @16
        return (t & 0xffu) | ((t >> 8) & 0xff00u);
    }
}

// Store the lane's C group words (B bytes each, slot order) at dst.
template <int B, int C>
__device__ __forceinline__ void store_group_words(uint8_t* dst, const uint32_t (&w)[C]) {
    if constexpr (B == 4) {
        if constexpr (C == 2) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
        } else {
#pragma unroll
            for (int c = 0; c < C; c += 4)
                *reinterpret_cast<uint4*>(dst + 4 * c) = make_uint4(w[c], w[c + 1], w[c + 2], w[c + 3]);
        }
    } else if constexpr (B == 2) {
        if constexpr (C == 2) {
            *reinterpret_cast<uint32_t*>(dst) = w[0] | (w[1] << 16);
        } else {
#pragma unroll
            for (int c = 0; c < C; c += 4)
                *reinterpret_cast<uint2*>(dst + 2 * c) =
                    make_uint2(w[c] | (w[c + 1] << 16), w[c + 2] | (w[c + 3] << 16));
        }
    } else {
        static_assert(B == 3, "3-byte groups");
        if constexpr (C == 2) {
            // 6 bytes at a 2-byte aligned address
            uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
            d16[0] = (uint16_t)w[0];
            d16[1] = (uint16_t)((w[0] >> 16) | (w[1] << 8));
            d16[2] = (uint16_t)(w[1] >> 8);
        } else {
#pragma unroll
            for (int c = 0; c < C; c += 4) {
                const uint32_t a = w[c] | (w[c + 1] << 24);
                const uint32_t b = (w[c + 1] >> 8) | (w[c + 2] << 16);
                const uint32_t e = (w[c + 2] >> 16) | (w[c + 3] << 8);
                *reinterpret_cast<uint3*>(dst + 3 * c) = make_uint3(a, b, e);
            }
        }
    }
}

// -------------------------------------------------------------- kernel ----

// Staging of a sub-item's source rows through LDS.  A wave's 16 rows arrive as
// NSEG direct-to-LDS loads of 16 bytes per lane (segment s of the wave holds
// lane l's bytes at 16 l), issued one sub-item ahead so that the HBM reads of
// the next rows overlap the arithmetic on the current ones without holding
// VGPRs.  Blocks whose staging would exceed 32 KB (fp32 rows of 256) load
// straight into registers instead.
template <int D, int DR, int DT>
struct RowStaging {
    static constexpr int in_bytes = DT == NQ_F32 ? 4 : 2;
    static constexpr int chunks = (DR + 31) / 32;   // chunks that hold source data
    static constexpr int parts = in_bytes / 2;      // 16-byte pieces per chunk
    static constexpr int nseg = chunks * parts;     // loads per lane per sub-item
    static constexpr bool pipe = 4 * nseg * 1024 <= 32768;
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// One sub-item's outputs (null when not written).
struct RowOut {
    uint16_t* recon;
    uint8_t* syms;
    uint8_t* cosets;
    float* scales;
    int8_t* codes8;
    uint16_t* scales16;
};

// The row computation of one sub-item: x holds the source row (zero padded,
// zeroed for evicted rows); cs / sn the source position's RoPE rows for keys.
// With a gather list the forward rotation takes the output position's rows:
// co / so for the merged layout, loaded per sub-item for the padded one.
template <int D, int L, bool IS_KEY, int DR, bool PAGE, bool GATHER>
__device__ __forceinline__ void quant_row_body(const QuantArgs& a, float (&x)[D / 32][8],
                                               float (&cs)[RopeChunks<D, DR>::value][8],
                                               float (&sn)[RopeChunks<D, DR>::value][8],
                                               const float (&co)[RopeChunks<D, DR>::value][8],
                                               const float (&so)[RopeChunks<D, DR>::value][8], int q, const RowOut& o,
                                               uint32_t bh, uint32_t t_in, uint32_t t_out, bool active,
                                               const float* lds_rope = nullptr) {
    constexpr int C = D / 32;
    constexpr int RC = RopeChunks<D, DR>::value;
    // Keys with DR == D: inverse RoPE and the top Hadamard stage in one step
    // (their pairs coincide); the other stages follow in fwht_row.
    constexpr bool MERGED = IS_KEY && DR == D;
    if constexpr (MERGED) {
        rope_stage_merged<C>(x, cs, sn);
    } else if constexpr (IS_KEY) {
        if constexpr (!PAGE && DR != D) load_rope_row<D, DR, RC>(lds_rope, q, cs, sn);  // staged in LDS
        apply_rope<D, DR, RC, true>(x, q, cs, sn);
    }

    fwht_row<C, !MERGED>(x, q);  // x = sigma(q) * S x
    constexpr float HL = (float)(L / 2);
    const float sigma = quad_sign(q);
    float umax = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) umax = __builtin_fmaxf(umax, __builtin_fabsf(x[c][i]));
    umax = __builtin_fmaxf(umax, dpp_f32<kQuadXor1>(umax));
    umax = __builtin_fmaxf(umax, dpp_f32<kQuadXor2>(umax));
    // Row scale as the reference: amax of the normalised rotation, clamped at
    // 1e-8 (rounding is monotone, so fl(max|u| h) is the max of fl(|u| h)).
    const float amax_raw = umax * a.hscale;
    const bool tiny = !(amax_raw >= 1e-8f);
    const float amax = tiny ? 1e-8f : amax_raw;
    const float scale = amax * (2.0f / (float)L);
    // Normalisation factor: the smallest f >= fl((L/2) / umax) with
    // fl(umax * f) >= L/2, so the row maximum lands on +-L/2 after the clamp;
    // fl(h / scale) for rows whose amax was clamped.  One correctly rounded
    // division per row.
    float f = (tiny ? a.hscale : HL) / (tiny ? scale : umax);
    if (!tiny && umax * f < HL) f = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, f) + 1u);
    const float fs = sigma * f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[c][i] = __builtin_amdgcn_fmed3f(x[c][i] * fs, -HL, HL);

    bool coset[C];
#pragma unroll
    for (int c = 0; c < C; ++c) coset[c] = e8_select(x[c]);

    const size_t out_row = (size_t)bh * a.seq_out + t_out;
    uint32_t cbits = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) cbits |= (uint32_t)coset[c] << (4 * c + q);
    cbits |= dpp_u32<kQuadXor1>(cbits);
    cbits |= dpp_u32<kQuadXor2>(cbits);
    if (active && q == 0) {
        if (o.cosets) {
            uint8_t* cdst = o.cosets + out_row * (D / 64);
            if constexpr (D == 64) *cdst = (uint8_t)cbits;
            else if constexpr (D == 128) *reinterpret_cast<uint16_t*>(cdst) = (uint16_t)cbits;
            else *reinterpret_cast<uint32_t*>(cdst) = cbits;
        }
        if (o.scales) o.scales[out_row] = scale;
    }
    if constexpr (PAGE) {
        // int8 codes 2p and the fp16 row scale, the page format of the vLLM
        // compressor (vllm_backend.py:305-314, 366-373)
        if (!active) return;
        if (q == 0 && o.scales16) o.scales16[out_row] = (uint16_t)f32_to_f16_bits(scale);
        int8_t* cdst = o.codes8 + out_row * D;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const float off = coset[c] ? 0.5f : 0.0f;
            uint32_t w[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                uint32_t v = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = __builtin_amdgcn_fmed3f(x[c][4 * k + j] + off, -HL, HL);
                    v |= ((uint32_t)(int32_t)(2.0f * p) & 0xffu) << (8 * j);
                }
                w[k] = v;
            }
            *reinterpret_cast<uint2*>(cdst + 32 * c + 8 * q) = make_uint2(w[0], w[1]);
        }
        return;
    } else {
    constexpr int B = SymBits<L>::value;
    constexpr int ROW_BYTES = D / 8 * B;
    const float g = sigma * (a.hscale * scale);  // reconstruction multiplier, sign folded

    constexpr bool PACKED = D * L <= 1024 && B <= 4;
    if constexpr (PACKED) {
        // U = clamp01((candidate + offset + L/2) / L); offset 1/2 for the half coset
        const uint32_t inv_l = splat_f16(1.0f / (float)L);
        const uint32_t off_int = splat_f16(HL / (float)L);
        const uint32_t off_half = splat_f16((HL + 0.5f) / (float)L);
        uint32_t u[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const uint32_t off = coset[c] ? off_half : off_int;
#pragma unroll
            for (int k = 0; k < 4; ++k) u[c][k] = pk_fma_clamp(pk_f16_bits(x[c][k], x[c][k + 4]), inv_l, off);
        }
        if (o.syms && active) {
            uint32_t wds[C];
#pragma unroll
            for (int c = 0; c < C; ++c) wds[c] = group_symbols<L>(u[c]);
            uint8_t* dst = o.syms + out_row * ROW_BYTES + q * (C * B);
            store_group_words<B, C>(dst, wds);
        }
        if (!o.recon) return;
        // Walsh-Hadamard of U in fp16 (exact: multiples of 1/(2L), |.| <= D).
        // S U = (S p)/L + (D/2) e_0, so every output but coordinate 0 (lane 0,
        // chunk 0, register 0 low half) is (S p)/L; that one is corrected by
        // subtracting (L/2) D after the exact multiply by L.  Without the top
        // stage (MERGED) the constant lands as (L/2)(D/2) on coordinates 0 and
        // D/2 (lane 0, chunks 0 and C/2).
        const float gl = g * (float)L;  // exact
        const float dc = q == 0 ? HL * (float)(MERGED ? D / 2 : D) : 0.0f;
        half2v hp[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) hp[c][k] = __builtin_bit_cast(half2v, u[c][k]);
        fwht_row_f16<C, !MERGED>(hp, q);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k == 0 && (c == 0 || (MERGED && c == C / 2))) {
                    const float t = __builtin_fmaf((float)hp[c][0].x, (float)L, -dc);  // exact
                    x[c][0] = t * g;
                } else {
                    x[c][k] = __builtin_fmaf((float)hp[c][k].x, gl, 0.0f);
                }
                x[c][k + 4] = __builtin_fmaf((float)hp[c][k].y, gl, 0.0f);
            }
    } else {
        // candidate + coset offset, clamped, as fp32 lattice points
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const float off = coset[c] ? 0.5f : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = __builtin_amdgcn_fmed3f(x[c][i] + off, -HL, HL);
        }
        if (o.syms && active) {
            int cs[C];
#pragma unroll
            for (int c = 0; c < C; ++c) cs[c] = coset[c] ? 1 : 0;
            uint8_t* dst = o.syms + out_row * ROW_BYTES;
            store_symbols<L, C>(dst, q, x, cs);
        }
        if (!o.recon) return;
        constexpr bool EXACT_F16 = D * (L / 2) <= 1024;
        if constexpr (EXACT_F16) {
            half2v hp[C][4];
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    hp[c][k] = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(x[c][2 * k], x[c][2 * k + 1]));
            fwht_row_f16<C, !MERGED>(hp, q);
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    x[c][2 * k] = __builtin_fmaf((float)hp[c][k].x, g, 0.0f);
                    x[c][2 * k + 1] = __builtin_fmaf((float)hp[c][k].y, g, 0.0f);
                }
        } else {
            fwht_row<C, !MERGED>(x, q);  // exact on half-integer lattice points
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int i = 0; i < 8; ++i) x[c][i] = x[c][i] * g;
        }
    }

    if constexpr (MERGED) {
        // the top inverse Hadamard stage and forward RoPE in one step.  The tables
        // stay live through the quantizer: reloading them here cuts 8 VGPRs but
        // not the occupancy, and the extra loads cost more than they save.  With a
        // gather list, co / so hold the output position's rows.
        if constexpr (GATHER) {
            rope_stage_merged<C>(x, co, so);
        } else {
            rope_stage_merged<C>(x, cs, sn);
        }
    } else if constexpr (IS_KEY) {
        if constexpr (GATHER) {
            // the padded layout loads the output position's rows here (holding
            // them for the work item would cost a wave of occupancy)
            float cg[RC][8], sg[RC][8];
            load_rope<D, DR, RC>(a.rope_cos, a.rope_sin, t_out, q, cg, sg);
            apply_rope<D, DR, RC, false>(x, q, cg, sg);
        } else {
            if constexpr (!PAGE && DR != D) load_rope_row<D, DR, RC>(lds_rope, q, cs, sn);
            apply_rope<D, DR, RC, false>(x, q, cs, sn);
        }
    }
    if (!active) return;
    uint16_t* dst = o.recon + out_row * DR;
    // The fp32 result is rounded to fp16 in a second step, as the reference does
    // (fp32 tensor, then .half()).  The empty asm pins the fp32 value: without it
    // the backend folds fma + convert into v_fma_mix{lo,hi}_f16, which rounds
    // the exact product-sum to fp16 once and differs at fp16 rounding ties.
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) asm("" : "+v"(x[c][i]));
#pragma unroll
    for (int c = 0; c < C; ++c) {
        if (32 * c >= DR) continue;  // padding coordinates are not part of the output
        half2v hv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) hv[k] = half2v{(__fp16)x[c][2 * k], (__fp16)x[c][2 * k + 1]};
        uint4 w;
        w.x = __builtin_bit_cast(uint32_t, hv[0]);
        w.y = __builtin_bit_cast(uint32_t, hv[1]);
        w.z = __builtin_bit_cast(uint32_t, hv[2]);
        w.w = __builtin_bit_cast(uint32_t, hv[3]);
        *reinterpret_cast<uint4*>(dst + 32 * c + 8 * q) = w;
    }
    }  // !PAGE
}

// The outputs of an evicted row under mask eviction, stored without reading
// or transforming it: a zeroed row quantizes to the integer point 0 (every
// symbol L/2, coset bits 0), its amax is clamped to 1e-8, so its scale is
// 1e-8 * (2/L) (exact: 2/L is a power of two), and its reconstruction is 0.
// Same lanes and store widths as quant_row_body's stores.
template <int D, int L, int DR>
__device__ __forceinline__ void store_evicted_row(const RowOut& o, size_t out_row, int q) {
    constexpr int C = D / 32;
    if (o.recon) {
        uint16_t* dst = o.recon + out_row * DR;
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (32 * c < DR) *reinterpret_cast<uint4*>(dst + 32 * c + 8 * q) = make_uint4(0u, 0u, 0u, 0u);
    }
    if (o.syms) {
        float p[C][8];
        int cs[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            cs[c] = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) p[c][i] = 0.0f;
        }
        store_symbols<L, C>(o.syms + out_row * (D / 8 * SymBits<L>::value), q, p, cs);
    }
    if (q == 0) {
        if (o.cosets) {
            uint8_t* cdst = o.cosets + out_row * (D / 64);
            if constexpr (D == 64) *cdst = 0;
            else if constexpr (D == 128) *reinterpret_cast<uint16_t*>(cdst) = 0;
            else *reinterpret_cast<uint32_t*>(cdst) = 0u;
        }
        if (o.scales) o.scales[out_row] = 1e-8f * (2.0f / (float)L);
    }
}

// lgkmcnt(0) / vmcnt(0) with the other counters left open (gfx9 s_waitcnt encoding)
constexpr int kWaitLgkm0 = 0xc07f;
constexpr int kWaitVm0 = 0x0f70;

// Row selection, one set of instantiations each, so that every path keeps its
// own register budget: kSelNone (output row t reads source row t, optionally
// zeroed or filtered by a keep list), kSelList (QuantArgs::order, mask
// eviction without work on evicted rows) and kSelGather (QuantArgs::gather,
// truncation: keys hold the source position's RoPE rows for the work item, and
// the output position's too where the merged layout applies; the padded layout
// loads the output rows per sub-item).
constexpr int kSelNone = 0;
constexpr int kSelList = 1;
constexpr int kSelGather = 2;

// Keys with the padded RoPE layout (head_dim 96): the row-list instantiation
// (mask eviction, the Phi-3 workload) fits 4 waves per SIMD without spills
// (126 VGPRs); the others keep their natural 3 waves rather than spill at 4.
template <int D, int L, bool IS_KEY, int DT, int DR, bool PAGE = false, int SEL = kSelNone>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((IS_KEY && !PAGE && DR != D && SEL == kSelList) ? 4 : 1))) void
quant_rows_kernel(QuantArgs a, const uint64_t* __restrict__ tab_src,
                                                         const uint64_t* __restrict__ tab_recon,
                                                         const uint64_t* __restrict__ tab_syms,
                                                         const uint64_t* __restrict__ tab_cosets,
                                                         const uint64_t* __restrict__ tab_scales,
                                                         const uint64_t* __restrict__ tab_positions,
                                                         const uint64_t* __restrict__ tab_codes8,
                                                         const uint64_t* __restrict__ tab_scales16) {
    static_assert(!PAGE || DR == D, "page encoding takes power-of-two head dims");
    static_assert(!PAGE || SEL == kSelNone, "pages take no row selection");
    constexpr bool LIST = SEL == kSelList;
    constexpr bool GATHER = SEL == kSelGather;
    constexpr int C = D / 32;
    constexpr int RC = RopeChunks<D, DR>::value;
    constexpr bool MERGED = IS_KEY && DR == D;
    using ST = RowStaging<D, DR, DT>;
    const int q = threadIdx.x & 3;
    // Block -> work item.  Consecutive block ids go round-robin to the 8 XCDs, so
    // block 8k + x takes work item x * per_xcd + k: each XCD walks a contiguous
    // range.  A work item is one 64-token tile of one batch row and a group of
    // sub-items j, the (head, tensor) pairs of that row with the tensor fastest,
    // which every wave runs back to back for its 16 tokens.  Items are ordered
    // (group, batch, tile) with the tile fastest: the blocks resident on one XCD
    // at a time cover consecutive tiles of one group, so they stream a few
    // contiguous regions of the group's tensors instead of one small piece of
    // every tensor (measured: 6% faster on the 80-layer 128K cache, and less
    // sensitive to where the buffers land in physical memory).  Keys with a
    // gather list take the group fastest instead: their groups are small and
    // each work item loads two positions' RoPE rows, which the blocks of one
    // tile then share in the XCD's L2 (the tile-fastest order re-fetched them
    // per group, 0.3 GB of a truncation launch's 0.7 GB of reads; 5% faster).
    // The whole block exits together.
    const uint32_t w = (blockIdx.x & 7u) * a.per_xcd + (blockIdx.x >> 3);
    if (w >= a.work) return;
    uint32_t tile, rest;
    if constexpr (GATHER && IS_KEY) {
        tile = w / (a.batch * a.n_groups);
        rest = w - tile * (a.batch * a.n_groups);
    } else {
        tile = w % a.n_tiles;
        rest = w / a.n_tiles;
    }
    const uint32_t b = rest % a.batch;
    const uint32_t grp = rest / a.batch;
    const uint32_t j0 = grp * a.group;
    const uint32_t j1 = j0 + a.group < a.hn ? j0 + a.group : a.hn;
    const uint32_t t_raw = tile * 64u + (threadIdx.x >> 2);
    const bool in_range = t_raw < a.seq_out;
    uint32_t t_out = in_range ? t_raw : a.seq_out - 1u;  // idle quads recompute a valid row
    uint32_t t_in = t_out;
    bool keep = true;
    if constexpr (LIST) {
        // Row list: entry t_raw of the batch row's list; the first n_kept are kept.
        // Tiles wholly past n_kept hold evicted rows only: they store the
        // zero-row outputs and read nothing (the branch is uniform per block).
        // The host validates the list; clamp anyway so that a bad entry cannot
        // reach outside the tensors.
        const int32_t nk = a.n_kept[b];
        const uint32_t n_list = nk < 0 ? 0u : ((uint32_t)nk > a.seq_in ? a.seq_in : (uint32_t)nk);
        const int32_t li = a.order[(size_t)b * a.seq_in + t_out];
        t_in = t_out = li < 0 ? 0u : ((uint32_t)li >= a.seq_in ? a.seq_in - 1u : (uint32_t)li);
        keep = t_raw < n_list;
        if (tile * 64u >= n_list) {
            for (uint32_t j = j0; j < j1 && in_range; ++j) {
                const uint32_t tensor = j % a.n_tensors;
                RowOut o = {};
                o.recon = tab_recon ? gptr<uint16_t>(tab_recon[tensor]) : nullptr;
                o.syms = tab_syms ? gptr<uint8_t>(tab_syms[tensor]) : nullptr;
                o.cosets = tab_cosets ? gptr<uint8_t>(tab_cosets[tensor]) : nullptr;
                o.scales = tab_scales ? gptr<float>(tab_scales[tensor]) : nullptr;
                const uint32_t bh = b * a.heads + j / a.n_tensors;
                store_evicted_row<D, L, DR>(o, (size_t)bh * a.seq_out + t_out, q);
            }
            return;
        }
    } else {
        if constexpr (GATHER) {
            // the host validates the list; clamp anyway so a bad index cannot read out of bounds
            const int32_t gi = a.gather[(size_t)b * a.seq_out + t_out];
            t_in = gi < 0 ? 0u : ((uint32_t)gi >= a.seq_in ? a.seq_in - 1u : (uint32_t)gi);
        }
        if (a.keep) keep = a.keep[(size_t)b * a.seq_in + t_in] != 0;
    }
    // rows this launch writes: all, or (soft eviction) only the kept / only the evicted ones
    const bool active = in_range && (a.keep_mode == NQ_KEEP_ZERO || keep == (a.keep_mode == NQ_KEEP_WRITE_KEPT));
    if (a.keep_mode != NQ_KEEP_ZERO) keep = true;  // selected rows are quantized as they are

    // Keys: the RoPE rows of the source position, loaded once for the work item
    // (pages rotate at per-page positions, loaded per sub-item).
    float cs[RC][8], sn[RC][8];  // cos / sin, or fl(sin - cos) / fl(cos + sin) when MERGED
    auto load_tables = [&](uint32_t pos) {
        if constexpr (MERGED) load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, pos, q, cs, sn);
        else load_rope<D, DR, RC>(a.rope_cos, a.rope_sin, pos, q, cs, sn);
    };

    auto row_elems = [&](uint32_t j) -> int64_t {  // element offset of this lane's first coordinate
        const uint32_t bh = b * a.heads + j / a.n_tensors;
        return ((int64_t)bh * a.seq_in + t_in) * DR + 8 * q;
    };
    __shared__ __attribute__((aligned(16))) uint8_t stage[ST::pipe ? 4 * ST::nseg * 1024 : 16];
    uint8_t* wstage = stage + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * (ST::nseg * 1024);
    const uint32_t lane = threadIdx.x & 63u;
    auto stage_rows = [&](uint32_t j) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(tab_src[j % a.n_tensors]) + row_elems(j) * ST::in_bytes;
#pragma unroll
        for (int c = 0; c < ST::chunks; ++c)
#pragma unroll
            for (int h = 0; h < ST::parts; ++h)
                __builtin_amdgcn_global_load_lds((global_void_t*)(p + 32 * c * ST::in_bytes + 16 * h),
                                                 (lds_void_t*)(wstage + (c * ST::parts + h) * 1024), 16, 0, 0);
    };

    // Keys with the padded RoPE layout (head_dim 96) read their RoPE rows from
    // LDS at each rotation instead of holding them in registers for the whole
    // work item (48 VGPRs, a wave of occupancy): the block stages its 64 rows'
    // cos and sin (48 + 48 floats each, 24 KiB) once, before the sub-items.
    constexpr bool LDS_ROPE = IS_KEY && !PAGE && DR != D;
    __shared__ __attribute__((aligned(16))) float s_rope[LDS_ROPE ? 2 * 64 * (DR / 2) : 4];
    const float* my_rope = nullptr;
    if constexpr (LDS_ROPE) {
        constexpr int H = DR / 2;  // table columns per row
        const int r = threadIdx.x >> 2;
        const float* ct = a.rope_cos + (size_t)t_in * H + (H / 4) * q;
        const float* st = a.rope_sin + (size_t)t_in * H + (H / 4) * q;
        float* dc = s_rope + r * H + (H / 4) * q;
        float* ds = s_rope + 64 * H + r * H + (H / 4) * q;
#pragma unroll
        for (int k = 0; k < H / 4; k += 4) {
            *reinterpret_cast<float4*>(dc + k) = *reinterpret_cast<const float4*>(ct + k);
            *reinterpret_cast<float4*>(ds + k) = *reinterpret_cast<const float4*>(st + k);
        }
        __syncthreads();
        my_rope = s_rope + r * H;
    } else if constexpr (IS_KEY && !PAGE) {
        load_tables(t_in);
    }
    // With a gather list, merged-layout keys also hold the output position's
    // rows for the work item (loading them per sub-item measured 11% slower).
    constexpr bool HOLD_OUT = GATHER && MERGED;
    float co[HOLD_OUT ? RC : 1][8], so[HOLD_OUT ? RC : 1][8];
    if constexpr (HOLD_OUT) load_rope_merged<D>(a.rope_cos, a.rope_sin, a.rope_dm, a.rope_dp, t_out, q, co, so);
    if constexpr (ST::pipe) stage_rows(j0);
    for (uint32_t j = j0; j < j1; ++j) {
        const uint32_t tensor = j % a.n_tensors;
        const uint32_t bh = b * a.heads + j / a.n_tensors;
        float x[C][8];
        if constexpr (ST::pipe) {
            // the wave's own loads of this sub-item's rows have landed (each wave
            // reads back only what it staged, so no barrier is needed)
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            uint4 raw[ST::nseg];
#pragma unroll
            for (int s = 0; s < ST::nseg; ++s) raw[s] = *reinterpret_cast<const uint4*>(wstage + s * 1024 + lane * 16);
#pragma unroll
            for (int c = 0; c < ST::chunks; ++c) cvt8<DT>(&raw[c * ST::parts], x[c]);
            // the reads have landed before the next sub-item's loads overwrite the segments
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            if (j + 1 < j1) stage_rows(j + 1);
        } else {
            const void* src = reinterpret_cast<const void*>(tab_src[tensor]);
            const int64_t off = row_elems(j);
#pragma unroll
            for (int c = 0; c < ST::chunks; ++c) load8<DT>(src, off + 32 * c, x[c]);
        }
#pragma unroll
        for (int c = ST::chunks; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = 0.0f;  // zero padding to D
        if (!keep) {
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int i = 0; i < 8; ++i) x[c][i] = 0.0f;
        }
        if constexpr (IS_KEY && PAGE) {
            // the host validates positions against the table; clamp anyway so a bad
            // position cannot read outside it
            const int32_t pp = gptr<const int32_t>(tab_positions[tensor])[t_in % a.page_tokens];
            load_tables(pp < 0 ? 0u : ((uint32_t)pp >= a.rope_n_pos ? a.rope_n_pos - 1u : (uint32_t)pp));
        }
        RowOut o;
        o.recon = tab_recon ? gptr<uint16_t>(tab_recon[tensor]) : nullptr;
        o.syms = tab_syms ? gptr<uint8_t>(tab_syms[tensor]) : nullptr;
        o.cosets = tab_cosets ? gptr<uint8_t>(tab_cosets[tensor]) : nullptr;
        o.scales = tab_scales ? gptr<float>(tab_scales[tensor]) : nullptr;
        if constexpr (PAGE) {
            o.codes8 = gptr<int8_t>(tab_codes8[tensor]);
            o.scales16 = tab_scales16 ? gptr<uint16_t>(tab_scales16[tensor]) : nullptr;
        } else {
            o.codes8 = nullptr;
            o.scales16 = nullptr;
        }
        if constexpr (HOLD_OUT)
            quant_row_body<D, L, IS_KEY, DR, PAGE, GATHER>(a, x, cs, sn, co, so, q, o, bh, t_in, t_out, active, my_rope);
        else
            quant_row_body<D, L, IS_KEY, DR, PAGE, GATHER>(a, x, cs, sn, cs, sn, q, o, bh, t_in, t_out, active, my_rope);
    }
}

// ---------------------------------------------------------------- host ----

// Sub-items per work item, at most max_group, fewer while the grid would fall
// below min_blocks (8192 = 32 per CU by default).  Values take 8 (16 and 1
// measured slower).  Keys take 64: a work item loads its tile's RoPE rows
// once, so with the tile-fastest order the rows are fetched once per group, 10
// times per tile on an 80-layer cache instead of 80.  Keys with a gather list
// load two positions' rows per work item and keep larger groups on small
// caches (4096 blocks: 8% faster on a 32-layer truncation than 8192, 2048 the
// same; plain and row-list launches measured slower at 4096).  Sets group,
// n_groups, hn, n_tiles, work and per_xcd from heads, n_tensors and batch;
// returns the work item count (the caller rejects counts beyond the grid limit
// before launching).
constexpr uint32_t kMaxGroup = 8;
constexpr uint32_t kKeyGroup = 64;
constexpr uint64_t kMinBlocks = 8192;
constexpr uint64_t kGatherKeyMinBlocks = 4096;

static uint64_t plan_work(QuantArgs& a, uint64_t tiles, uint32_t max_group, uint64_t min_blocks = kMinBlocks) {
    a.hn = a.heads * a.n_tensors;
    uint32_t g = a.hn < max_group ? a.hn : max_group;
    while (g > 1 && tiles * a.batch * ((a.hn + g - 1) / g) < min_blocks) g >>= 1;
    a.group = g;
    a.n_groups = (a.hn + g - 1) / g;
    a.n_tiles = (uint32_t)tiles;
    const uint64_t work = tiles * a.batch * a.n_groups;
    a.work = (uint32_t)work;
    a.per_xcd = (uint32_t)((work + 7) / 8);
    return work;
}

template <int D, int L, bool K, int DT, int DR, bool PAGE = false, int SEL = kSelNone>
static hipError_t launch_quant(const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    hipLaunchKernelGGL((quant_rows_kernel<D, L, K, DT, DR, PAGE, SEL>), dim3(a.per_xcd * 8u), dim3(256), 0, s, a,
                       t.src, t.recon, t.syms, t.cosets, t.scales, t.positions, t.codes8, t.scales16);
    return hipGetLastError();
}

template <int D, int L, bool K, int DR, int SEL>
static hipError_t dispatch_dtype(int dt, const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    switch (dt) {
        case NQ_F16: return launch_quant<D, L, K, NQ_F16, DR, false, SEL>(a, t, s);
        case NQ_BF16: return launch_quant<D, L, K, NQ_BF16, DR, false, SEL>(a, t, s);
        default: return launch_quant<D, L, K, NQ_F32, DR, false, SEL>(a, t, s);
    }
}

template <int D, int L, int DR, int SEL>
static hipError_t dispatch_key(bool key, int dt, const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    return key ? dispatch_dtype<D, L, true, DR, SEL>(dt, a, t, s) : dispatch_dtype<D, L, false, DR, SEL>(dt, a, t, s);
}

template <int D, int DR, int SEL>
static hipError_t dispatch_levels(int L, bool key, int dt, const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    switch (L) {
        case 2: return dispatch_key<D, 2, DR, SEL>(key, dt, a, t, s);
        case 4: return dispatch_key<D, 4, DR, SEL>(key, dt, a, t, s);
        case 8: return dispatch_key<D, 8, DR, SEL>(key, dt, a, t, s);
        default: return dispatch_key<D, 16, DR, SEL>(key, dt, a, t, s);
    }
}

// Launch of one nq_quantize call on the already planned arguments, by head_dim.
template <int SEL>
static hipError_t dispatch_quant(int head_dim, int L, bool key, int dt, const QuantArgs& a, const QuantTables& t,
                                 hipStream_t s) {
    switch (head_dim) {
        case 64: return dispatch_levels<64, 64, SEL>(L, key, dt, a, t, s);
        case 96: return dispatch_levels<128, 96, SEL>(L, key, dt, a, t, s);
        case 128: return dispatch_levels<128, 128, SEL>(L, key, dt, a, t, s);
        default: return dispatch_levels<256, 256, SEL>(L, key, dt, a, t, s);
    }
}

// The row-list and gather instantiations, each compiled in a translation unit
// of its own (nq_quant_list.hip, nq_quant_gather.hip) so the sets build in
// parallel.
hipError_t dispatch_quant_list(int head_dim, int L, bool key, int dt, const QuantArgs& a, const QuantTables& t,
                               hipStream_t s);
hipError_t dispatch_quant_gather(int head_dim, int L, bool key, int dt, const QuantArgs& a, const QuantTables& t,
                                 hipStream_t s);

}  // namespace nq
