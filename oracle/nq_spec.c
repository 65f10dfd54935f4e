/*
 * Tier-B oracle: the row quantizer restated in plain C with a fixed arithmetic
 * order.  TEST INFRASTRUCTURE ONLY -- the product library never links it.
 *
 * It restates the reference's per-row pipeline
 *   keys  : inverse RoPE -> Hadamard -> relaxed E8 (per-row scale) -> Hadamard -> RoPE
 *   values:                 Hadamard -> relaxed E8 (per-row scale) -> Hadamard
 * (jagmarques/nexusquant pipeline.py:232-265, e8_lattice.py:27-124,
 *  rope_utils.py:75-249, hadamard.py:23-43) and fixes every rounding step so
 * that the HIP kernel can be compared with it bit for bit:
 *
 *  1. Inverse RoPE with one fused multiply-add per coordinate.  For d = D
 *     (power-of-two head dims) the RoPE pair (i, i + D/2) is also the pair of
 *     the top Hadamard stage, and the two are done as one step with dm =
 *     fl(c - s), dp = fl(c + s):  lo' = fma(lo, dm, fl(hi*dp)),
 *     hi' = fma(lo, dp, -fl(hi*dm)), after which stage 3 leaves out that top
 *     stage.  For d = 96 (padded): lo' = fma(lo, c, fl(hi*s)),
 *     hi' = fma(hi, c, -fl(lo*s)).  The reference rounds every product and sum
 *     separately (rope_utils.py:75-112, dense GEMM); the differences are a few
 *     ulp of the rotated value, below what moves a code except at a near tie.
 *  2. Zero-pad to D = next power of two (the reference raises for d = 96,
 *     hadamard.py:35-36; padding is this build's definition).
 *  3. Unnormalised Walsh-Hadamard butterflies u = S x, stages on index bit
 *     0,1,..., log2(D)-1 in that order (the top one already done for d = D
 *     keys), each (a, b) -> (a + b, a - b) in fp32.
 *     The reference uses a dense fp32 GEMM with the normalised matrix h_D * S
 *     here, so the two differ in the last ulp; the resulting code disagreement
 *     is measured in tests (about 1e-6 of groups).
 *  4. Row scale exactly as the reference's amax of the normalised rotation:
 *     amax = fl(max|u| * h_D) (rounding is monotone, so this equals the max of
 *     the rounded products), clamped at fp32(1e-8); scale = amax/(L/2) (exact)
 *     (e8_lattice.py:114-116).  Normalised coordinates xn = clamp(fl(u * f),
 *     -L/2, L/2): one multiply per coordinate in place of the reference's
 *     multiply by h_D and division by scale, within a few ulp of it.  f is the
 *     smallest float >= fl((L/2) / max|u|) with fl(max|u| * f) >= L/2, so the
 *     row's largest coordinate lands exactly on +-L/2 after the clamp, as it
 *     does in the reference (amax / scale == L/2 exactly).  Rows whose amax is
 *     clamped to 1e-8 use f = fl(h_D / scale) and never reach L/2.
 *  5. Relaxed E8 per 8-group (e8_lattice.py:36-69): r = rint(x); on odd sum
 *     the first smallest |x - r| coordinate steps toward x (zero gap: +1);
 *     h = rint(x - 0.5) + 0.5.  The choice d_half < d_int is evaluated in the
 *     algebraically identical closed form (d_half - d_int = 2 - sum|x - r| on
 *     even sums, 1 + 2 min|x - r| - sum|x - r| on odd sums), with the sum of
 *     |x - r| added as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) in fp32.  It differs
 *     from the reference's rounded fp32 distance sums only when the two
 *     distances are within about 1e-6 of each other (a near tie).
 *  6. Clamp to [-L/2, L/2] after the choice (e8_lattice.py:120).
 *  7. Reconstruction: w = S * p is exact in fp32 for every order (p is a
 *     half-integer of magnitude <= 8), then recon = w * fl(h_D * scale).  Keys
 *     with d = D stop w before the top stage and finish with the merged step
 *     of 1. on the output-position tables (the top inverse stage followed by
 *     forward RoPE is the same map); d = 96 keys apply forward RoPE
 *     lo' = fma(lo, c, -fl(hi*s)), hi' = fma(lo, s, fl(hi*c)).  The reference
 *     rounds every product separately; the difference is below fp16
 *     resolution except at fp16 rounding ties.  Keep the first d outputs,
 *     round to fp16 (round to nearest even).
 *
 *  8. Page decode (the vLLM compressor's int8 2p codes and fp16 scales,
 *     vllm_backend.py:394-429): w = S c on the integer codes c = 2p is exact in
 *     fp32 in any order; then w * g with g = fl(fl(0.5 * scale) * h_D)
 *     (0.5 * scale is exact), so each coordinate is rounded once where the
 *     reference's dense GEMM rounds every product and partial sum.  Keys stop
 *     w before the top stage and finish with the merged step of 1. at the
 *     stored position; fp16 round to nearest even.
 *
 * Code symbols: the group's coset bit is 1 when the half-integer candidate was
 * chosen.  Integer coset: sym = p + L/2.  Half coset: the clamp folds one edge
 * point onto +-L/2 (the top edge when L/2 is even, the bottom edge when L/2 is
 * odd, because rint rounds half to even), so sym = floor(p) + L/2 when L/2 is
 * even and ceil(p) + L/2 when L/2 is odd; sym is always in [0, L].  Decoding:
 * p = sym - L/2 (integer), min(sym - L/2 + 1/2, L/2) (half, L/2 even),
 * max(sym - L/2 - 1/2, -L/2) (half, L/2 odd).
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define NQS_MAXD 256

/* ---------------------------------------------------------------- fp16 -- */

uint16_t nqs_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {                      /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) {                      /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx < 0x38800000u) {                       /* below fp16 normal range */
        if (absx < 0x33000000u) return (uint16_t)sign;       /* < 2^-25: rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                  /* 14 - (e - 127) + ... */
        /* value = m * 2^(e-150); fp16 subnormal unit 2^-24 -> q = m >> (126-e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u;              /* rebias 127 -> 15 */
    uint32_t m = absx & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float nqs_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float v = (float)m * 0x1p-24f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------ E8 -- */

/* One 8-group.  x: normalised coordinates.  Outputs clamped lattice point p,
 * coset flag, and a tie margin: the smallest distance of this group's input to
 * any decision boundary of the rule (rint boundaries, argmin runner-up, the
 * half/integer choice).  Returns nothing; all outputs by pointer. */
void nqs_e8_group(const float* x, float half_levels, float* p, int* coset, float* margin) {
    float r[8], e[8], a[8], hh[8];
    int parity = 0;
    for (int j = 0; j < 8; ++j) {
        r[j] = rintf(x[j]);
        e[j] = x[j] - r[j];
        a[j] = fabsf(e[j]);
        parity += (int)r[j];
        float t = x[j] - 0.5f;
        hh[j] = rintf(t) + 0.5f;
    }
    int odd = parity & 1;
    int imin = 0;
    float amin = a[0];
    for (int j = 1; j < 8; ++j) {
        if (a[j] < amin) { amin = a[j]; imin = j; }
    }
    float asum = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    float thr = odd ? (1.0f + 2.0f * amin) : 2.0f;
    int use_half = asum > thr;
    for (int j = 0; j < 8; ++j) {
        float v;
        if (use_half) {
            v = hh[j];
        } else {
            v = r[j];
            if (odd && j == imin) v += (e[j] >= 0.0f) ? 1.0f : -1.0f;
        }
        if (v > half_levels) v = half_levels;
        if (v < -half_levels) v = -half_levels;
        p[j] = v;
    }
    *coset = use_half;
    if (margin) {
        float m = fabsf(asum - thr);
        for (int j = 0; j < 8; ++j) {
            float b1 = fabsf(a[j] - 0.5f);           /* rint boundary of r */
            if (b1 < m) m = b1;
            /* rint boundary of h; the row's amax coordinate is exactly +-L/2 in
             * every implementation, so it is not a perturbable boundary */
            if (fabsf(x[j]) != half_levels && a[j] < m) m = a[j];
            if (odd && j != imin) {
                float b3 = a[j] - amin;              /* argmin runner-up */
                if (b3 < m) m = b3;
            }
        }
        *margin = m;
    }
}

/* ----------------------------------------------------------- row quant -- */

static int coset_of(const uint8_t* flags, int i) { return flags[i >> 3]; }

static float next_up(float f) { /* f > 0, finite */
    uint32_t b;
    memcpy(&b, &f, 4);
    ++b;
    memcpy(&f, &b, 4);
    return f;
}

/* butterfly stages on index bits 0, 1, ... up to (not including) the bit of `top` */
static void fwht_stages(float* v, int D, int top) {
    for (int len = 1; len < top; len <<= 1) {
        for (int i = 0; i < D; ++i) {
            if (i & len) continue;
            float a = v[i], b = v[i + len];
            v[i] = a + b;
            v[i + len] = a - b;
        }
    }
}

/*
 * Quantize n rows.
 *   x        [n][d] fp32 input rows (exact conversions of fp16/bf16/fp32)
 *   cos_in, sin_in   [n][d/2] tables at each row's source position (keys) or NULL
 *   cos_out, sin_out [n][d/2] tables at each row's output position (keys) or NULL
 *   D        padded power-of-two width (>= d, <= 256), L levels (2,4,8,16)
 *   hD       Hadamard normalisation constant for width D
 * Outputs (any may be NULL):
 *   xn_out   [n][D] normalised rotated rows
 *   p_out    [n][D] clamped lattice points
 *   sym_out  [n][D] uint8 symbols floor(p) + L/2
 *   coset_out[n][D/8] uint8 coset flags
 *   scale_out[n] fp32 row scale
 *   recon_out[n][d] fp16 bits of the reconstruction
 *   margin_out [n][D/8] tie margins
 */
void nqs_quant_rows(int64_t n, int d, int D, int L, float hD,
                    const float* x,
                    const float* cos_in, const float* sin_in,
                    const float* cos_out, const float* sin_out,
                    float* xn_out, float* p_out, uint8_t* sym_out, uint8_t* coset_out,
                    float* scale_out, uint16_t* recon_out, float* margin_out) {
    const int half = d / 2;
    const float half_levels = (float)(L / 2);
    const int G = D / 8;
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < n; ++row) {
        float v[NQS_MAXD], xn[NQS_MAXD], p[NQS_MAXD];
        const float* xr = x + row * d;
        for (int i = 0; i < D; ++i) v[i] = 0.0f;
        const int merged = cos_in && d == D;  /* RoPE pairs are the top Hadamard pairs */
        if (merged) {
            const float* c = cos_in + row * half;
            const float* s = sin_in + row * half;
            for (int i = 0; i < half; ++i) {
                float lo = xr[i], hi = xr[i + half];
                float dm = c[i] - s[i], dp = c[i] + s[i];
                v[i] = fmaf(lo, dm, hi * dp);
                v[i + half] = fmaf(lo, dp, -(hi * dm));
            }
        } else if (cos_in) {
            const float* c = cos_in + row * half;
            const float* s = sin_in + row * half;
            for (int i = 0; i < half; ++i) {
                float lo = xr[i], hi = xr[i + half];
                v[i] = fmaf(lo, c[i], hi * s[i]);
                v[i + half] = fmaf(hi, c[i], -(lo * s[i]));
            }
        } else {
            for (int i = 0; i < d; ++i) v[i] = xr[i];
        }
        fwht_stages(v, D, merged ? D / 2 : D);
        float umax = 0.0f;
        for (int i = 0; i < D; ++i) {
            float av = fabsf(v[i]);
            if (av > umax) umax = av;
        }
        float amax = umax * hD;
        float f;
        if (amax >= 1e-8f) {
            /* smallest f >= fl(L/2 / umax) with fl(umax * f) >= L/2: the quotient
             * is within half an ulp, so one step up always suffices */
            f = half_levels / umax;
            if (umax * f < half_levels) f = next_up(f);
        } else {
            amax = 1e-8f;
            f = hD / (amax / half_levels);
        }
        float scale = amax / half_levels;
        for (int i = 0; i < D; ++i) {
            float t = v[i] * f;
            xn[i] = t > half_levels ? half_levels : (t < -half_levels ? -half_levels : t);
        }
        uint8_t coset_flags[NQS_MAXD / 8];
        for (int g = 0; g < G; ++g) {
            int cs;
            float mg;
            nqs_e8_group(xn + 8 * g, half_levels, p + 8 * g, &cs, &mg);
            coset_flags[g] = (uint8_t)cs;
            if (coset_out) coset_out[row * G + g] = (uint8_t)cs;
            /* a coordinate the clamp moved onto +-L/2 that is not the row maximum
             * sits one ulp from where the reference puts it: a tie for the
             * direction of the odd-sum step */
            for (int j = 0; j < 8 && mg > 0.0f; ++j)
                if (fabsf(xn[8 * g + j]) == half_levels && fabsf(v[8 * g + j]) != umax) mg = 0.0f;
            if (margin_out) margin_out[row * G + g] = mg;
        }
        if (xn_out) memcpy(xn_out + row * D, xn, sizeof(float) * D);
        if (p_out) memcpy(p_out + row * D, p, sizeof(float) * D);
        if (sym_out) {
            const int odd_hl = (L / 2) & 1;
            for (int i = 0; i < D; ++i) {
                int half_cs = coset_of(coset_flags, i);
                float f = (half_cs && odd_hl) ? ceilf(p[i]) : floorf(p[i]);
                sym_out[row * D + i] = (uint8_t)(int)(f + half_levels);
            }
        }
        if (scale_out) scale_out[row] = scale;
        if (recon_out) {
            float w[NQS_MAXD];
            memcpy(w, p, sizeof(float) * D);
            fwht_stages(w, D, merged ? D / 2 : D);  /* exact on half-integer points */
            float g = hD * scale;
            for (int i = 0; i < D; ++i) w[i] = w[i] * g;
            uint16_t* out = recon_out + row * d;
            if (merged) {
                /* top inverse stage and forward RoPE in one step (same map as the input side) */
                const float* c = cos_out + row * half;
                const float* s = sin_out + row * half;
                for (int i = 0; i < half; ++i) {
                    float lo = w[i], hi = w[i + half];
                    float dm = c[i] - s[i], dp = c[i] + s[i];
                    out[i] = nqs_f32_to_f16(fmaf(lo, dm, hi * dp));
                    out[i + half] = nqs_f32_to_f16(fmaf(lo, dp, -(hi * dm)));
                }
            } else if (cos_out) {
                const float* c = cos_out + row * half;
                const float* s = sin_out + row * half;
                for (int i = 0; i < half; ++i) {
                    /* output side: one fused multiply-add per coordinate; the result
                     * is rounded to fp16 next, which hides the fp32 difference from
                     * the reference's separate products except at fp16 ties */
                    float lo = w[i], hi = w[i + half];
                    float t2 = hi * s[i];
                    float t4 = hi * c[i];
                    out[i] = nqs_f32_to_f16(fmaf(lo, c[i], -t2));
                    out[i + half] = nqs_f32_to_f16(fmaf(lo, s[i], t4));
                }
            } else {
                for (int i = 0; i < d; ++i) out[i] = nqs_f32_to_f16(w[i]);
            }
        }
    }
}


/* Page decode (item 8 above): codes int8 [n, D] (2p), scales fp16 [n]; keys
 * read cos/sin rows [n, D/2] at their stored positions. */
void nqs_page_decode(int64_t n, int D, int is_key, float hD, const int8_t* codes, const uint16_t* scales16,
                     const float* cos_rows, const float* sin_rows, uint16_t* out) {
    const int half = D / 2;
    for (int64_t row = 0; row < n; ++row) {
        float w[NQS_MAXD];
        for (int i = 0; i < D; ++i) w[i] = (float)codes[row * D + i];
        fwht_stages(w, D, is_key ? half : D);
        const float g = (0.5f * nqs_f16_to_f32(scales16[row])) * hD;
        for (int i = 0; i < D; ++i) w[i] = w[i] * g;
        uint16_t* o = out + row * D;
        if (is_key) {
            const float* c = cos_rows + row * half;
            const float* s = sin_rows + row * half;
            for (int i = 0; i < half; ++i) {
                float lo = w[i], hi = w[i + half];
                float dm = c[i] - s[i], dp = c[i] + s[i];
                o[i] = nqs_f32_to_f16(fmaf(lo, dm, hi * dp));
                o[i + half] = nqs_f32_to_f16(fmaf(lo, dp, -(hi * dm)));
            }
        } else {
            for (int i = 0; i < D; ++i) o[i] = nqs_f32_to_f16(w[i]);
        }
    }
}
