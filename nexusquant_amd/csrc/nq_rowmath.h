// Row math shared by the quantizer and the code kernels: the quad-per-row
// layout (lane q of a quad owns chunks c of 8 coordinates 32c + 8q .. +7),
// 16-byte loads, Walsh-Hadamard butterflies and symbol widths.
#pragma once

#include "nq_common.h"

namespace nq {

template <int L>
struct SymBits {
    static constexpr int value = L == 2 ? 2 : L == 4 ? 3 : L == 8 ? 4 : 5;
};

// ------------------------------------------------------------- loads ------

// 8 coordinates from their raw bytes: one uint4 of fp16 / bf16, two of fp32.
template <int DT>
__device__ __forceinline__ void cvt8(const uint4* r, float* out) {
    if constexpr (DT == NQ_F32) {
        const uint4 a = r[0], b = r[1];
        const uint32_t ws[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = __builtin_bit_cast(float, ws[k]);
    } else {
        const uint4 w = r[0];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (DT == NQ_BF16) {
                out[2 * k] = __builtin_bit_cast(float, ws[k] << 16);
                out[2 * k + 1] = __builtin_bit_cast(float, ws[k] & 0xffff0000u);
            } else {
                out[2 * k] = f16_bits_to_f32(ws[k] & 0xffffu);
                out[2 * k + 1] = f16_bits_to_f32(ws[k] >> 16);
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t elem_off, float* out) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(base) +
                                                    elem_off * (DT == NQ_F32 ? 4 : 2));
    uint4 r[2];
    r[0] = p[0];
    if constexpr (DT == NQ_F32) r[1] = p[1];
    cvt8<DT>(r, out);
}

__device__ __forceinline__ void load8f(const float* p, float* out) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// ------------------------------------------------------------ Hadamard ----

typedef __fp16 half2v __attribute__((ext_vector_type(2)));

#define NQ_GLOBAL __attribute__((address_space(1)))

// A device address as a pointer the compiler knows to be global memory (it is
// made in the global address space, then cast to a generic pointer, which
// address-space inference folds back): accesses through it compile to global
// rather than flat instructions, and stores count on vmcnt only.
template <class T>
__device__ __forceinline__ T* gptr(uint64_t addr) {
    return (T*)(NQ_GLOBAL T*)addr;
}

// Quad butterfly v <- v + c * partner(v) with the partner read through DPP in
// the same v_fmac_f32 instruction.  The DPP read of a VGPR needs two wait
// states after the VALU write that produced it; s_nop 1 provides them for the
// first instruction, and the other seven read registers written before it.
#define NQ_FMAC_DPP8(PERM, x, c)                                                       \
    asm("s_nop 1\n\t"                                                                  \
        "v_fmac_f32_dpp %0, %0, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %1, %1, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %2, %2, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %3, %3, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %4, %4, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %5, %5, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %6, %6, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
        "v_fmac_f32_dpp %7, %7, %8 " PERM " row_mask:0xf bank_mask:0xf bound_ctrl:1"     \
        : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),       \
          "+v"(x[6]), "+v"(x[7])                                                       \
        : "v"(c))

// Unnormalised Walsh-Hadamard over the quad's row.  Stage order follows
// coordinate bits 0,1,2 (in chunk), 3,4 (across the quad), 5.. (across chunks);
// TOP = false leaves out the stage on the top bit (pairs i, i + D/2), which
// the merged RoPE step below performs.
// The quad stages compute v + c * partner with c = +-1 per lane, the exact
// butterfly up to a sign; every lane's values end multiplied by
// sigma(q) = (-1)^popcount(q), which the caller folds into the next multiply.
template <int C, bool TOP = true>
__device__ __forceinline__ void fwht_row(float (&x)[C][8], int q) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int len = 1; len < 8; len <<= 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (i & len) continue;
                float a = x[c][i], b = x[c][i + len];
                x[c][i] = a + b;
                x[c][i + len] = a - b;
            }
        }
    }
    const float s3 = (q & 1) ? -1.0f : 1.0f;
    const float s4 = (q & 2) ? -1.0f : 1.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) NQ_FMAC_DPP8("quad_perm:[1,0,3,2]", x[c], s3);
#pragma unroll
    for (int c = 0; c < C; ++c) NQ_FMAC_DPP8("quad_perm:[2,3,0,1]", x[c], s4);
#pragma unroll
    for (int len = 1; len < (TOP ? C : C / 2); len <<= 1) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if (c & len) continue;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float a = x[c][i], b = x[c + len][i];
                x[c][i] = a + b;
                x[c + len][i] = a - b;
            }
        }
    }
}

// The same transform on lattice points packed two per register as fp16
// (coordinates 2k, 2k+1 of a chunk in register k).  Every value stays a
// multiple of 1/2 of magnitude <= D*L/2 <= 1024, so fp16 holds it exactly and
// the result equals the fp32 transform in any stage order.  Output carries the
// same sigma(q) sign.
template <int C, bool TOP = true>
__device__ __forceinline__ void fwht_row_f16(half2v (&h)[C][4], int q) {
    const half2v pm = {(__fp16)1.0f, (__fp16)-1.0f};
#pragma unroll
    for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) h[c][k] = __builtin_elementwise_fma(h[c][k], pm, h[c][k].yx);
#pragma unroll
        for (int len = 1; len < 4; len <<= 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k & len) continue;
                half2v a = h[c][k], b = h[c][k + len];
                h[c][k] = a + b;
                h[c][k + len] = a - b;
            }
        }
    }
    const __fp16 f3 = (q & 1) ? (__fp16)-1.0f : (__fp16)1.0f;
    const __fp16 f4 = (q & 2) ? (__fp16)-1.0f : (__fp16)1.0f;
    const half2v s3 = {f3, f3}, s4 = {f4, f4};
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            half2v p = __builtin_bit_cast(half2v, dpp_u32<kQuadXor1>(__builtin_bit_cast(uint32_t, h[c][k])));
            h[c][k] = __builtin_elementwise_fma(s3, p, h[c][k]);
        }
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            half2v p = __builtin_bit_cast(half2v, dpp_u32<kQuadXor2>(__builtin_bit_cast(uint32_t, h[c][k])));
            h[c][k] = __builtin_elementwise_fma(s4, p, h[c][k]);
        }
#pragma unroll
    for (int len = 1; len < (TOP ? C : C / 2); len <<= 1) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if (c & len) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                half2v a = h[c][k], b = h[c + len][k];
                h[c][k] = a + b;
                h[c + len][k] = a - b;
            }
        }
    }
}

__device__ __forceinline__ float quad_sign(int q) {
    return ((q ^ (q >> 1)) & 1) ? -1.0f : 1.0f;
}

// ------------------------------------------------------------------ RoPE ----
//
// Split-half RoPE pairs coordinate i with i + DR/2 (DR = real head dim).  With
// DR == D the pair is chunk c and c + C/2 of the same lane.  With DR = 96
// padded to D = 128 the partner of every live coordinate sits in quad lane
// q ^ 2: for q < 2 chunks (0, 1, 2) pair with that lane's chunks (1, 2, 0), for
// q >= 2 with (2, 0, 1); chunk 3 is padding.  rope_col gives the table column
// of the pair's first coordinate for each of the lane's RoPE chunks.

template <int D, int DR>
struct RopeChunks {
    static constexpr int value = DR == D ? D / 64 : 3;
};

template <int D, int DR>
__device__ __forceinline__ int rope_col(int c, int q) {
    if constexpr (DR == D) {
        return 32 * c + 8 * q;
    } else {
        static_assert(D == 128 && DR == 96, "padded RoPE layout implemented for 96 -> 128");
        const bool lowq = q < 2;
        return c == 0 ? 8 * q : (c == 1 ? (lowq ? 32 + 8 * q : 8 * (q - 2)) : (lowq ? 16 + 8 * q : 32 + 8 * (q - 2)));
    }
}

template <int D, int DR, int RC>
__device__ __forceinline__ void load_rope(const float* cos_t, const float* sin_t, uint32_t pos, int q,
                                          float (&cs)[RC][8], float (&sn)[RC][8]) {
    const float* ct = cos_t + (size_t)pos * (DR / 2);
    const float* st = sin_t + (size_t)pos * (DR / 2);
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        load8f(ct + rope_col<D, DR>(c, q), cs[c]);
        load8f(st + rope_col<D, DR>(c, q), sn[c]);
    }
}

// The same columns from one token's row staged in LDS: cos at row[0, DR / 2),
// sin 64 rows (64 * DR / 2 floats) further on.
template <int D, int DR, int RC>
__device__ __forceinline__ void load_rope_row(const float* row, int q, float (&cs)[RC][8], float (&sn)[RC][8]) {
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        const int col = rope_col<D, DR>(c, q);
        const float4 c0 = *reinterpret_cast<const float4*>(row + col), c1 = *reinterpret_cast<const float4*>(row + col + 4);
        const float4 s0 = *reinterpret_cast<const float4*>(row + 64 * (DR / 2) + col);
        const float4 s1 = *reinterpret_cast<const float4*>(row + 64 * (DR / 2) + col + 4);
        cs[c][0] = c0.x; cs[c][1] = c0.y; cs[c][2] = c0.z; cs[c][3] = c0.w;
        cs[c][4] = c1.x; cs[c][5] = c1.y; cs[c][6] = c1.z; cs[c][7] = c1.w;
        sn[c][0] = s0.x; sn[c][1] = s0.y; sn[c][2] = s0.z; sn[c][3] = s0.w;
        sn[c][4] = s1.x; sn[c][5] = s1.y; sn[c][6] = s1.z; sn[c][7] = s1.w;
    }
}

// INVERSE (input side): lo' = fma(lo, c, hi*s), hi' = fma(hi, c, -(lo*s)).
// Forward (output side): lo' = fma(lo, c, -(hi*s)), hi' = fma(lo, s, hi*c).
template <int D, int DR, int RC, bool INVERSE>
__device__ __forceinline__ void apply_rope(float (&x)[D / 32][8], int q, const float (&cs)[RC][8],
                                           const float (&sn)[RC][8]) {
    constexpr int C = D / 32;
    if constexpr (DR == D) {
#pragma unroll
        for (int c = 0; c < C / 2; ++c) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float lo = x[c][i], hi = x[c + C / 2][i];
                if constexpr (INVERSE) {
                    x[c][i] = __builtin_fmaf(lo, cs[c][i], hi * sn[c][i]);
                    x[c + C / 2][i] = __builtin_fmaf(hi, cs[c][i], -(lo * sn[c][i]));
                } else {
                    x[c][i] = __builtin_fmaf(lo, cs[c][i], -(hi * sn[c][i]));
                    x[c + C / 2][i] = __builtin_fmaf(lo, sn[c][i], hi * cs[c][i]);
                }
            }
        }
    } else {
        float P[3][8];
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) P[c][i] = dpp_f32<kQuadXor2>(x[c][i]);
        const bool lowq = q < 2;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const bool is_lo = c == 0 || (c == 1 && lowq);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p = c == 0 ? (lowq ? P[1][i] : P[2][i])
                                       : (c == 1 ? (lowq ? P[2][i] : P[0][i]) : (lowq ? P[0][i] : P[1][i]));
                const float v = x[c][i];
                if constexpr (INVERSE) {
                    const float ps = p * sn[c][i];
                    x[c][i] = __builtin_fmaf(v, cs[c][i], is_lo ? ps : -ps);
                } else {
                    x[c][i] = is_lo ? __builtin_fmaf(v, cs[c][i], -(p * sn[c][i]))
                                    : __builtin_fmaf(p, sn[c][i], v * cs[c][i]);
                }
            }
        }
    }
}

// --------------------------------------------------- merged RoPE + top stage ----
//
// With DR == D the RoPE pair (i, i + D/2) is also the pair of the top
// Walsh-Hadamard stage, and rotation followed by that butterfly is
//   (lo, hi) -> (lo (c - s) + hi (c + s), lo (c + s) - hi (c - s))
// on the input side (inverse RoPE, then the stage), and the same map on the
// output side (the inverse stage, then forward RoPE).  With dm = fl(c - s)
// and dp = fl(c + s):  lo' = fma(lo, dm, fl(hi dp)), hi' = fma(lo, dp, -fl(hi dm)).
// The tables hold nm = fl(s - c) = -dm instead, so both products need no
// negated operand: lo' = fma(-lo, nm, fl(hi dp)), hi' = fma(lo, dp, fl(hi nm)),
// the same numbers (negation is exact).

template <int D>
__device__ __forceinline__ void load_rope_merged(const float* cos_t, const float* sin_t, const float* dm_t,
                                                 const float* dp_t, uint32_t pos, int q, float (&dm)[D / 64][8],
                                                 float (&dp)[D / 64][8]) {
    constexpr int RC = D / 64;
    const size_t base = (size_t)pos * (D / 2);
    if (dm_t) {
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            load8f(dm_t + base + 32 * c + 8 * q, dm[c]);
            load8f(dp_t + base + 32 * c + 8 * q, dp[c]);
        }
    } else {
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            float cs[8], sn[8];
            load8f(cos_t + base + 32 * c + 8 * q, cs);
            load8f(sin_t + base + 32 * c + 8 * q, sn);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dm[c][i] = sn[i] - cs[i];  // fl(s - c)
                dp[c][i] = cs[i] + sn[i];
            }
        }
    }
}

template <int C>
__device__ __forceinline__ void rope_stage_merged(float (&x)[C][8], const float (&dm)[C / 2][8],
                                                  const float (&dp)[C / 2][8]) {
#pragma unroll
    for (int c = 0; c < C / 2; ++c) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float lo = x[c][i], hi = x[c + C / 2][i];
            x[c][i] = __builtin_fmaf(-lo, dm[c][i], hi * dp[c][i]);  // dm holds fl(s - c)
            x[c + C / 2][i] = __builtin_fmaf(lo, dp[c][i], hi * dm[c][i]);
        }
    }
}

}  // namespace nq
