// Fused row quantizer for gfx950: inverse RoPE -> Walsh-Hadamard -> per-row
// scale -> relaxed E8 -> packed codes, and the drop-in reconstruction
// (inverse Hadamard -> rescale -> forward RoPE -> fp16) in the same pass.
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
#include "nq_rowmath.h"

namespace nq {

struct QuantArgs {
    const uint64_t* src;
    const uint64_t* recon;
    const uint64_t* syms;
    const uint64_t* cosets;
    const uint64_t* scales;
    const int32_t* gather;
    const uint8_t* keep;
    const float* rope_cos;
    const float* rope_sin;
    uint32_t heads, seq_in, seq_out, rows;
    uint32_t n_tensors, bh, work, per_xcd;  // work items = ceil(seq_out/64) * bh * n_tensors
    float hscale;
};

// ------------------------------------------------------------------ E8 ----

// Relaxed E8 (oracle/nq_spec.c nqs_e8_group): returns the coset flag and
// overwrites x with the clamped lattice point.  The odd-sum step goes to the
// first coordinate whose |x - r| equals the group minimum, which is the
// reference's first argmin.
template <int L>
__device__ __forceinline__ int e8_group(float (&x)[8]) {
    constexpr float HL = (float)(L / 2);
    float r[8], e[8], a[8];
    int isum = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        r[j] = __builtin_rintf(x[j]);
        e[j] = x[j] - r[j];
        a[j] = __builtin_fabsf(e[j]);
        isum += (int)r[j];
    }
    const bool odd = (isum & 1) != 0;
    const float amin = __builtin_fminf(__builtin_fminf(__builtin_fminf(a[0], a[1]), __builtin_fminf(a[2], a[3])),
                                       __builtin_fminf(__builtin_fminf(a[4], a[5]), __builtin_fminf(a[6], a[7])));
    const float asum = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    const float thr = odd ? (1.0f + 2.0f * amin) : 2.0f;
    const bool use_half = asum > thr;
    bool pending = odd && !use_half;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float h = __builtin_rintf(x[j] - 0.5f) + 0.5f;
        const bool hit = pending && (a[j] == amin);
        pending = pending && !hit;
        const float rs = r[j] + __builtin_copysignf(1.0f, e[j]);  // e is never -0
        float v = use_half ? h : (hit ? rs : r[j]);
        x[j] = __builtin_fminf(__builtin_fmaxf(v, -HL), HL);
    }
    return use_half ? 1 : 0;
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

// -------------------------------------------------------------- kernel ----

template <int D, int L, bool IS_KEY, int DT, int DR>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantArgs a) {
    constexpr int C = D / 32;
    constexpr int RC = RopeChunks<D, DR>::value;
    const int q = threadIdx.x & 3;
    // Block -> work item.  Consecutive block ids go round-robin to the 8 XCDs, so
    // block 8k + x takes work item x * per_xcd + k: each XCD walks a contiguous
    // range.  Work items are ordered (token tile, batch*head, tensor) with the
    // tensor fastest, so the blocks that read one token tile's RoPE rows run back
    // to back on one XCD and find them in its L2.  The whole block exits together.
    const uint32_t w = (blockIdx.x & 7u) * a.per_xcd + (blockIdx.x >> 3);
    if (w >= a.work) return;
    const uint32_t tensor = w % a.n_tensors;
    const uint32_t rest = w / a.n_tensors;
    const uint32_t bh = rest % a.bh;
    const uint32_t tile = rest / a.bh;
    const uint32_t t_raw = tile * 64u + (threadIdx.x >> 2);
    const bool active = t_raw < a.seq_out;
    const uint32_t t_out = active ? t_raw : a.seq_out - 1u;  // idle quads recompute a valid row
    const uint32_t b = bh / a.heads;
    uint32_t t_in = t_out;
    if (a.gather) {
        // the host validates the list; clamp anyway so a bad index cannot read out of bounds
        const int32_t gi = a.gather[(size_t)b * a.seq_out + t_out];
        t_in = gi < 0 ? 0u : ((uint32_t)gi >= a.seq_in ? a.seq_in - 1u : (uint32_t)gi);
    }
    bool keep = true;
    if (a.keep) keep = a.keep[(size_t)b * a.seq_in + t_in] != 0;

    float x[C][8];
    const void* src = reinterpret_cast<const void*>(a.src[tensor]);
    const int64_t in_off = ((int64_t)bh * a.seq_in + t_in) * DR;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        if (32 * c < DR) {
            load8<DT>(src, in_off + 32 * c + 8 * q, x[c]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = 0.0f;  // zero padding to D
        }
    }
    if (!keep) {
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = 0.0f;
    }

    float cs[RC][8], sn[RC][8];
    if constexpr (IS_KEY) {
        load_rope<D, DR, RC>(a.rope_cos, a.rope_sin, t_in, q, cs, sn);
        apply_rope<D, DR, RC, true>(x, q, cs, sn);
    }

    fwht_row<C>(x, q);
    const float sigma = quad_sign(q);
    const float hs = sigma * a.hscale;
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[c][i] = x[c][i] * hs;
            amax = __builtin_fmaxf(amax, __builtin_fabsf(x[c][i]));
        }
    amax = __builtin_fmaxf(amax, dpp_f32<kQuadXor1>(amax));
    amax = __builtin_fmaxf(amax, dpp_f32<kQuadXor2>(amax));
    amax = __builtin_fmaxf(amax, 1e-8f);
    const float scale = amax * (2.0f / (float)L);
    const float rcp = 1.0f / scale;  // correctly rounded reciprocal

    int coset[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // correctly rounded x / scale by one refinement of the reciprocal
            float q0 = x[c][i] * rcp;
            float rem = __builtin_fmaf(-q0, scale, x[c][i]);
            x[c][i] = __builtin_fmaf(rem, rcp, q0);
        }
        coset[c] = e8_group<L>(x[c]);
    }

    const size_t out_row = (size_t)bh * a.seq_out + t_out;
    if (a.syms && active) {
        constexpr int ROW_BYTES = D / 8 * SymBits<L>::value;
        uint8_t* dst = reinterpret_cast<uint8_t*>(a.syms[tensor]) + out_row * ROW_BYTES;
        store_symbols<L, C>(dst, q, x, coset);
    }
    uint32_t cbits = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) cbits |= (uint32_t)coset[c] << (4 * c + q);
    cbits |= dpp_u32<kQuadXor1>(cbits);
    cbits |= dpp_u32<kQuadXor2>(cbits);
    if (active && q == 0) {
        if (a.cosets) {
            uint8_t* cdst = reinterpret_cast<uint8_t*>(a.cosets[tensor]) + out_row * (D / 64);
            if constexpr (D == 64) *cdst = (uint8_t)cbits;
            else if constexpr (D == 128) *reinterpret_cast<uint16_t*>(cdst) = (uint16_t)cbits;
            else *reinterpret_cast<uint32_t*>(cdst) = cbits;
        }
        if (a.scales) reinterpret_cast<float*>(a.scales[tensor])[out_row] = scale;
    }

    if (!a.recon) return;
    const float g = sigma * (a.hscale * scale);
    constexpr bool EXACT_F16 = D * (L / 2) <= 1024;
    if constexpr (EXACT_F16) {
        half2v hp[C][4];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                hp[c][k] = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(x[c][2 * k], x[c][2 * k + 1]));
        fwht_row_f16<C>(hp, q);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x[c][2 * k] = __builtin_fmaf((float)hp[c][k].x, g, 0.0f);
                x[c][2 * k + 1] = __builtin_fmaf((float)hp[c][k].y, g, 0.0f);
            }
    } else {
        fwht_row<C>(x, q);  // exact on half-integer lattice points
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[c][i] = x[c][i] * g;
    }

    if constexpr (IS_KEY) {
        if (a.gather && t_out != t_in) load_rope<D, DR, RC>(a.rope_cos, a.rope_sin, t_out, q, cs, sn);
        apply_rope<D, DR, RC, false>(x, q, cs, sn);
    }
    if (!active) return;
    half2v* dst = reinterpret_cast<half2v*>(reinterpret_cast<uint16_t*>(a.recon[tensor]) + out_row * DR);
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
        half2v o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = half2v{(__fp16)x[c][2 * k], (__fp16)x[c][2 * k + 1]};
        uint4 w;
        w.x = __builtin_bit_cast(uint32_t, o[0]);
        w.y = __builtin_bit_cast(uint32_t, o[1]);
        w.z = __builtin_bit_cast(uint32_t, o[2]);
        w.w = __builtin_bit_cast(uint32_t, o[3]);
        *reinterpret_cast<uint4*>(dst + (32 * c + 8 * q) / 2) = w;
    }
}

// ---------------------------------------------------------------- host ----

template <int D, int L, bool K, int DT, int DR>
static hipError_t launch_quant(const QuantArgs& a, uint32_t n_tensors, hipStream_t s) {
    (void)n_tensors;
    dim3 grid(a.per_xcd * 8u);
    hipLaunchKernelGGL((quant_rows_kernel<D, L, K, DT, DR>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int D, int L, bool K, int DR>
static hipError_t dispatch_dtype(int dt, const QuantArgs& a, uint32_t n, hipStream_t s) {
    switch (dt) {
        case NQ_F16: return launch_quant<D, L, K, NQ_F16, DR>(a, n, s);
        case NQ_BF16: return launch_quant<D, L, K, NQ_BF16, DR>(a, n, s);
        default: return launch_quant<D, L, K, NQ_F32, DR>(a, n, s);
    }
}

template <int D, int L, int DR>
static hipError_t dispatch_key(bool key, int dt, const QuantArgs& a, uint32_t n, hipStream_t s) {
    return key ? dispatch_dtype<D, L, true, DR>(dt, a, n, s) : dispatch_dtype<D, L, false, DR>(dt, a, n, s);
}

template <int D, int DR = D>
static hipError_t dispatch_levels(int L, bool key, int dt, const QuantArgs& a, uint32_t n, hipStream_t s) {
    switch (L) {
        case 2: return dispatch_key<D, 2, DR>(key, dt, a, n, s);
        case 4: return dispatch_key<D, 4, DR>(key, dt, a, n, s);
        case 8: return dispatch_key<D, 8, DR>(key, dt, a, n, s);
        default: return dispatch_key<D, 16, DR>(key, dt, a, n, s);
    }
}

}  // namespace nq

extern "C" int nq_quantize(const nq_quant_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_quantize: desc is NULL");
    NQ_CHECK_ARG(d->n_tensors >= 0 && d->n_tensors <= 65535, "nq_quantize: n_tensors %d out of range", d->n_tensors);
    if (d->n_tensors == 0) return NQ_OK;
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 96 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_quantize: head_dim %d unsupported by this entry point (64, 96, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->levels == 2 || d->levels == 4 || d->levels == 8 || d->levels == 16,
                 "nq_quantize: levels must be 2, 4, 8 or 16 (got %d)", d->levels);
    NQ_CHECK_ARG(d->dtype == NQ_F16 || d->dtype == NQ_BF16 || d->dtype == NQ_F32,
                 "nq_quantize: unknown dtype %d", d->dtype);
    NQ_CHECK_ARG(d->batch > 0 && d->heads > 0 && d->seq_in >= 0 && d->seq_out >= 0,
                 "nq_quantize: bad geometry");
    NQ_CHECK_ARG(d->gather != nullptr || d->seq_out == d->seq_in,
                 "nq_quantize: seq_out must equal seq_in without a gather list");
    NQ_CHECK_ARG(d->src != nullptr, "nq_quantize: src is NULL");
    const uint64_t rows = (uint64_t)d->batch * d->heads * d->seq_out;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq_quantize: %llu rows per tensor exceeds 2^31", (unsigned long long)rows);
    if (rows == 0) return NQ_OK;
    if (d->is_key) {
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin, "nq_quantize: keys need RoPE tables");
        NQ_CHECK_ARG(d->rope_n_pos >= d->seq_in && d->rope_n_pos >= d->seq_out,
                     "nq_quantize: RoPE table has %lld positions, need %d",
                     (long long)d->rope_n_pos, d->seq_in > d->seq_out ? d->seq_in : d->seq_out);
    }
    QuantArgs a;
    a.src = d->src;
    a.recon = d->recon;
    a.syms = d->syms;
    a.cosets = d->cosets;
    a.scales = d->scales;
    a.gather = d->gather;
    a.keep = d->keep;
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.heads = (uint32_t)d->heads;
    a.seq_in = (uint32_t)d->seq_in;
    a.seq_out = (uint32_t)d->seq_out;
    a.rows = (uint32_t)rows;
    a.hscale = d->hadamard_scale;
    a.n_tensors = (uint32_t)d->n_tensors;
    a.bh = (uint32_t)d->batch * (uint32_t)d->heads;
    const uint64_t work = (uint64_t)((d->seq_out + 63) / 64) * a.bh * a.n_tensors;
    NQ_CHECK_ARG(work < (1ull << 32) - 8, "nq_quantize: %llu work items exceed the grid limit",
                 (unsigned long long)work);
    a.work = (uint32_t)work;
    a.per_xcd = (uint32_t)((work + 7) / 8);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    switch (d->head_dim) {
        case 64: e = dispatch_levels<64>(d->levels, d->is_key != 0, d->dtype, a, d->n_tensors, s); break;
        case 96: e = dispatch_levels<128, 96>(d->levels, d->is_key != 0, d->dtype, a, d->n_tensors, s); break;
        case 128: e = dispatch_levels<128>(d->levels, d->is_key != 0, d->dtype, a, d->n_tensors, s); break;
        default: e = dispatch_levels<256>(d->levels, d->is_key != 0, d->dtype, a, d->n_tensors, s); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}
