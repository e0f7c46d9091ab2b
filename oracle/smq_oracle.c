/* CPU oracle for the quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the
 * reference's arithmetic contract, written from its specification. Only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark may load
 * it, and only as the checker. The GPU product never links or calls it.
 *
 * Every function names the reference lines it restates (paths relative to
 * the reference tree). Build: see oracle/Makefile (gcc -O2 -ffp-contract=off
 * -fno-fast-math, so no multiply-add is ever fused).
 *
 * Pinning (what checks each function, beyond retyping its formula):
 *   orc_f16_to_f32 / orc_f32_to_f16 : numpy's IEEE half conversion over all
 *       65,536 halves and random floats; the reference's constants
 *       (tests/test_kernels.c:58-60, tests/convert-quant.test.ts:117-132).
 *   orc_quantize_q8 : closed-form properties (tests/test_kernels.c:89-107),
 *       a numpy restatement, and the compiled reference (oracle/_ref).
 *   orc_dot_* / orc_gemm_* : float64 closed form (tests/test_kernels.c:109-127),
 *       exact-integer lane sums, the FMA probe (0.0f exact / 0x1p-12f fast,
 *       tests/test_kernels.c:223-249), and the compiled reference.
 *   orc_q8_weight_rows : SHA-256 goldens tests/goldens/convert-q8.json.
 *   orc_quantize_q5_row : brute-force minimum search on tiny blocks, and the
 *       compiled reference.
 *   orc_gemm_blockwise : exact equality with a float64 evaluation where every
 *       step is exact (power-of-two scales), and 1e-5 normwise of orc_gemm.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "smq_oracle.h"

#if defined(FLT_EVAL_METHOD) && FLT_EVAL_METHOD != 0
#  error "the oracle needs plain binary32 evaluation"
#endif

/* ---- little-endian field readers ------------------------------------- */

static uint32_t le_u32(const unsigned char *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static float le_f32(const unsigned char *p) {
    uint32_t u = le_u32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t le_u16(const unsigned char *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- binary16 (src/f16.h:10-55) -------------------------------------- */

/* f16.h:10-27. Exact widening, derived from the value formula rather than
 * bit surgery: normal = (1024 + m) * 2^(e - 25), subnormal = m * 2^-24. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    int neg = (h >> 15) & 1;
    float v;
    if (e == 31u) {
        uint32_t bits = ((uint32_t)neg << 31) | 0x7f800000u | (m << 13);
        memcpy(&v, &bits, 4);
        return v;
    }
    if (e == 0u) v = ldexpf((float)m, -24);
    else v = ldexpf((float)(1024u + m), (int)e - 25);
    return neg ? -v : v;
}

/* f16.h:30-55. Round to nearest, ties to even; overflow gives infinity.
 * Computed as: find the half-precision quantum for |f|, round |f|/quantum to
 * an integer in double (exact: the quotient has at most 24 significant bits
 * plus the shift), and re-encode. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t bits;
    uint16_t sign;
    double a, q, r;
    int e;
    memcpy(&bits, &f, 4);
    sign = (uint16_t)((bits >> 16) & 0x8000u);
    if ((bits & 0x7f800000u) == 0x7f800000u) /* inf or NaN */
        return (uint16_t)(sign | 0x7c00u | ((bits & 0x7fffffu) ? 0x200u : 0u));
    a = fabs((double)f);
    if (a == 0.0) return sign;
    (void)frexp(a, &e); /* a = mant * 2^e, mant in [0.5, 1) */
    e -= 1;             /* a = 1.x * 2^e */
    if (e < -14) e = -14; /* subnormal range shares the 2^-24 quantum */
    q = ldexp(1.0, e - 10);
    r = nearbyint(a / q); /* default rounding mode: ties to even */
    a = r * q;
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u); /* rounded past the largest half */
    if (a < ldexp(1.0, -14)) return (uint16_t)(sign | (uint16_t)r); /* subnormal: r = mantissa */
    (void)frexp(a, &e);
    e -= 1;
    /* a = (1 + m/1024) * 2^e exactly */
    return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)(ldexp(a, 10 - e) - 1024.0));
}

/* ---- activation quantizer (src/kernels.c:912-935) -------------------- */

int orc_quantize_q8(const float *x, uint32_t n, float *d, int8_t *q) {
    uint32_t nblocks = (n + 31u) / 32u, b, j;
    for (b = 0; b < nblocks; ++b) {
        const float *xb = x + (size_t)b * 32u;
        int8_t *qb = q + (size_t)b * 32u;
        uint32_t valid = n - b * 32u;
        float amax = 0.0f, scale, inv;
        if (valid > 32u) valid = 32u;
        for (j = 0; j < valid; ++j) {
            float a = fabsf(xb[j]);
            if (!(a <= FLT_MAX)) return -1; /* inf or NaN: kernels.c:921 */
            if (a > amax) amax = a;
        }
        scale = amax / 127.0f;
        inv = (scale >= FLT_MIN) ? 1.0f / scale : 0.0f; /* kernels.c:912 */
        d[b] = scale;
        for (j = 0; j < 32u; ++j) {
            long v = 0;
            if (j < valid) {
                float prod = xb[j] * inv;
                v = lrintf(prod);
            }
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            qb[j] = (int8_t)v;
        }
    }
    return 0;
}

/* ---- block decoding --------------------------------------------------- */

/* Q5 block (docs/FORMAT.md:124-134; kernels.c:53-60): f16 scale, u32 high
 * plane (bit j = bit 4 of element j), 16 nibble bytes (byte j holds element
 * j low and element j+16 high). Value = q - 16. */
void orc_unpack_q5(const unsigned char *blk, int8_t out[32]) {
    uint32_t high = le_u32(blk + 2), j;
    const unsigned char *nib = blk + 6;
    for (j = 0; j < 32u; ++j) {
        uint32_t lo = j < 16u ? (nib[j] & 15u) : (uint32_t)(nib[j - 16u] >> 4);
        uint32_t hi = (high >> j) & 1u;
        out[j] = (int8_t)((int)(lo | (hi << 4)) - 16);
    }
}

/* ---- dot-product contract (src/kernels.c:36-50, 62-79, 107-173) ------- */

/* One block into the eight lane accumulators: lane l = exact int sum of
 * products 4l..4l+3; then acc[l] = acc[l] + d * float(sum) with two roundings,
 * or a single fmaf in the fast contract (kernels.c:43-50, 116-121). */
static void lanes_update(float acc[8], const int8_t *wq, const int8_t *xq, float d, int fast) {
    int l, k;
    for (l = 0; l < 8; ++l) {
        int32_t s = 0;
        for (k = 0; k < 4; ++k) s += (int32_t)wq[4 * l + k] * (int32_t)xq[4 * l + k];
        if (fast) {
            acc[l] = fmaf(d, (float)s, acc[l]);
        } else {
            float p = d * (float)s;
            acc[l] = acc[l] + p;
        }
    }
}

/* kernels.c:36-39: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). */
static float lanes_reduce(const float a[8]) {
    float p04 = a[0] + a[4], p15 = a[1] + a[5], p26 = a[2] + a[6], p37 = a[3] + a[7];
    float even = p04 + p26, odd = p15 + p37;
    return even + odd;
}

static float dot_q8_impl(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, int fast) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t b;
    for (b = 0; b < nb; ++b) {
        const unsigned char *blk = w + (size_t)b * ORC_Q8_BLOCK;
        float d = le_f32(blk) * xd[b];
        lanes_update(acc, (const int8_t *)(blk + 4), xq + (size_t)b * 32u, d, fast);
    }
    return lanes_reduce(acc);
}

static float dot_q5_impl(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, int fast) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int8_t wq[32];
    uint32_t b;
    for (b = 0; b < nb; ++b) {
        const unsigned char *blk = w + (size_t)b * ORC_Q5_BLOCK;
        float d = orc_f16_to_f32(le_u16(blk)) * xd[b];
        orc_unpack_q5(blk, wq);
        lanes_update(acc, wq, xq + (size_t)b * 32u, d, fast);
    }
    return lanes_reduce(acc);
}

float orc_dot_q8(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_q8_impl(w, xd, xq, nb, 0);
}
float orc_dot_q5(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_q5_impl(w, xd, xq, nb, 0);
}
float orc_dot_q8_fast(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_q8_impl(w, xd, xq, nb, 1);
}
float orc_dot_q5_fast(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_q5_impl(w, xd, xq, nb, 1);
}

/* kernels.c:81-93: one row, four activations `stride` blocks apart. */
void orc_dot_x4(int q5, int fast, const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb,
                uint32_t stride, float out[4]) {
    uint32_t t;
    for (t = 0; t < 4u; ++t) {
        const float *d = xd + (size_t)t * stride;
        const int8_t *q = xq + (size_t)t * stride * 32u;
        out[t] = q5 ? dot_q5_impl(w, d, q, nb, fast) : dot_q8_impl(w, d, q, nb, fast);
    }
}

/* kernels.c:95-105: four rows `row_bytes` apart, one activation. */
void orc_dot_r4(int q5, int fast, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                uint32_t nb, float out[4]) {
    uint32_t i;
    for (i = 0; i < 4u; ++i) {
        const unsigned char *row = w + i * row_bytes;
        out[i] = q5 ? dot_q5_impl(row, xd, xq, nb, fast) : dot_q8_impl(row, xd, xq, nb, fast);
    }
}

/* kernels.c:175-201 (GemmQ8, kernels.h:60-65): out[t * stride + r] is the dot
 * of weight row r with activation t; activations are packed nb blocks apart.
 * Visiting order never changes a value, so a plain double loop restates it. */
void orc_gemm(int q5, int fast, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
              uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride) {
    uint32_t r, t;
    for (t = 0; t < ntok; ++t) {
        const float *d = xd + (size_t)t * nb;
        const int8_t *q = xq + (size_t)t * nb * 32u;
        for (r = 0; r < nrows; ++r) {
            const unsigned char *row = w + (size_t)r * row_bytes;
            out[(size_t)t * stride + r] = q5 ? dot_q5_impl(row, d, q, nb, fast) : dot_q8_impl(row, d, q, nb, fast);
        }
    }
}

/* Per-block exact integer sums (all 32 products), the quantity the
 * relaxed-order prefill path must reproduce bit for bit:
 * sums[(t * nrows + r) * nb + b]. */
void orc_block_sums(int q5, const unsigned char *w, size_t row_bytes, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, int32_t *sums) {
    uint32_t r, t, b, j;
    int8_t wq[32];
    for (t = 0; t < ntok; ++t)
        for (r = 0; r < nrows; ++r)
            for (b = 0; b < nb; ++b) {
                const unsigned char *blk = w + (size_t)r * row_bytes + (size_t)b * (q5 ? ORC_Q5_BLOCK : ORC_Q8_BLOCK);
                const int8_t *xb = xq + ((size_t)t * nb + b) * 32u;
                int32_t s = 0;
                if (q5) orc_unpack_q5(blk, wq);
                else memcpy(wq, blk + 4, 32);
                for (j = 0; j < 32u; ++j) s += (int32_t)wq[j] * (int32_t)xb[j];
                sums[((size_t)t * nrows + r) * nb + b] = s;
            }
}

/* The relaxed-order prefill contract as the GPU's MFMA kernels evaluate it:
 * per output, the blocks in order of acc = fmaf(wscale * xscale, S, acc),
 * S the exact integer block sum (orc_block_sums). The reference has no such
 * order (its GEMM keeps eight lane sums); the GPU GEMMs that do not split K
 * must equal this bit for bit. */
void orc_gemm_blockwise(int q5, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                        uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride) {
    uint32_t r, t, b, j;
    int8_t wq[32];
    for (t = 0; t < ntok; ++t)
        for (r = 0; r < nrows; ++r) {
            float acc = 0.0f;
            for (b = 0; b < nb; ++b) {
                const unsigned char *blk = w + (size_t)r * row_bytes + (size_t)b * (q5 ? ORC_Q5_BLOCK : ORC_Q8_BLOCK);
                const int8_t *xb = xq + ((size_t)t * nb + b) * 32u;
                const float ws = q5 ? orc_f16_to_f32(le_u16(blk)) : le_f32(blk);
                int32_t sum = 0;
                if (q5) orc_unpack_q5(blk, wq);
                else memcpy(wq, blk + 4, 32);
                for (j = 0; j < 32u; ++j) sum += (int32_t)wq[j] * (int32_t)xb[j];
                acc = fmaf(ws * xd[(size_t)t * nb + b], (float)sum, acc);
            }
            out[(size_t)t * stride + r] = acc;
        }
}

/* ---- caller glue (src/model.c:252-310) -------------------------------- */

/* threadpool.h:19-23 */
void orc_split_range(uint32_t total, uint32_t index, uint32_t count, uint32_t *begin, uint32_t *end) {
    *begin = (uint32_t)((uint64_t)total * index / count);
    *end = (uint32_t)((uint64_t)total * (index + 1u) / count);
}

/* model.c:252-266 for one item over all its rows: gemm, then y += bias[r],
 * then a finiteness check. Returns 1 when every cell is finite. */
int orc_mat_item(int q5, int fast, const unsigned char *w, size_t row_bytes, uint32_t rows, const float *bias,
                 const float *xd, const int8_t *xq, uint32_t ntok, uint32_t nb, float *y) {
    uint32_t t, r;
    int ok = 1;
    orc_gemm(q5, fast, w, row_bytes, xd, xq, rows, ntok, nb, y, rows);
    for (t = 0; t < ntok; ++t)
        for (r = 0; r < rows; ++r) {
            float *cell = &y[(size_t)t * rows + r];
            if (bias) *cell = *cell + bias[r];
            ok &= fabs((double)*cell) <= DBL_MAX; /* finite.h:11 */
        }
    return ok;
}

/* model.c:334-342: sequential f32 sum of squares, one reciprocal square root,
 * y = (x * inv) * w. Returns -1 when the sum or the scale is not finite. */
int orc_rmsnorm(const float *x, const float *w, float *y, uint32_t n, float eps) {
    float sq = 0.0f, inv;
    uint32_t i;
    for (i = 0; i < n; ++i) {
        float p = x[i] * x[i];
        sq = sq + p;
    }
    inv = 1.0f / sqrtf(sq / (float)n + eps);
    if (!(fabsf(sq) <= FLT_MAX) || !(fabsf(inv) <= FLT_MAX)) return -1;
    for (i = 0; i < n; ++i) {
        float t = x[i] * inv;
        y[i] = t * w[i];
    }
    return 0;
}

/* ---- deterministic exp and the gated activations (src/vecmath.c:19-93) - */

/* vecmath.c:44-52: bits of 2^(j/32) (correctly rounded binary64) minus j<<47;
 * regenerated from the mathematics by oracle/gen_exp_table.py. */
static const uint64_t ORC_EXP2[32] = {
    0x3ff0000000000000u, 0x3fefd9b0d3158574u, 0x3fefb5586cf9890fu, 0x3fef9301d0125b51u,
    0x3fef72b83c7d517bu, 0x3fef54873168b9aau, 0x3fef387a6e756238u, 0x3fef1e9df51fdee1u,
    0x3fef06fe0a31b715u, 0x3feef1a7373aa9cbu, 0x3feedea64c123422u, 0x3feece086061892du,
    0x3feebfdad5362a27u, 0x3feeb42b569d4f82u, 0x3feeab07dd485429u, 0x3feea47eb03a5585u,
    0x3feea09e667f3bcdu, 0x3fee9f75e8ec5f74u, 0x3feea11473eb0187u, 0x3feea589994cce13u,
    0x3feeace5422aa0dbu, 0x3feeb737b0cdc5e5u, 0x3feec49182a3f090u, 0x3feed503b23e255du,
    0x3feee89f995ad3adu, 0x3feeff76f2fb5e47u, 0x3fef199bdd85529cu, 0x3fef3720dcef9069u,
    0x3fef5818dcfba487u, 0x3fef7c97337b9b5fu, 0x3fefa4afa2a490dau, 0x3fefd0765b6e4540u,
};

const uint64_t *orc_exp2_table(void) { return ORC_EXP2; }

/* vecmath.c:61-76: e^x = 2^(k/32) * e^(r ln2/32) with k = round(32x/ln2)
 * taken from the low bits after adding 1.5*2^52, r the remainder, a degree-4
 * Taylor polynomial evaluated with separate multiplies and adds (no FMA),
 * everything in binary64, one rounding to binary32. Clamped to [-104, 89]. */
float orc_exp_det(float x) {
    const double inv_ln2_n = 0x1.71547652b82fep+5, shift = 0x1.8p+52;
    const double a = 0x1.62e42fefa39efp-1 / 32;
    const double c1 = a, c2 = a * a / 2, c3 = a * a * a / 6, c4 = a * a * a * a / 24;
    double z, kd, r, p, scale;
    uint64_t ki, sb;
    if (x != x) return x;
    if (x > 89.0f) x = 89.0f;
    if (x < -104.0f) x = -104.0f;
    z = inv_ln2_n * (double)x;
    kd = z + shift;
    memcpy(&ki, &kd, 8);
    kd = kd - shift;
    r = z - kd;
    p = c4 * r + c3;
    p = p * r + c2;
    p = p * r + c1;
    p = p * r + 1.0;
    sb = ORC_EXP2[ki & 31u] + (ki << 47);
    memcpy(&scale, &sb, 8);
    return (float)(p * scale);
}

/* vecmath.c:78-81: up *= gate / (1 + e^-gate). */
void orc_silu_mul(float *up, const float *gate, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) {
        float den = 1.0f + orc_exp_det(-gate[i]);
        float s = gate[i] / den;
        up[i] = up[i] * s;
    }
}

/* vecmath.c:86-93: up *= g / (1 + e^-(1.5957691216 (g + 0.044715 g^3))). */
void orc_gelu_mul(float *up, const float *gate, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) {
        float g = gate[i];
        float g3 = 0.044715f * g * g * g;
        float u = 1.5957691216f * (g + g3);
        float den = 1.0f + orc_exp_det(-u);
        float s = g / den;
        up[i] = up[i] * s;
    }
}

/* model.c:354-362 row_work for `rows` token rows of n values: optional RMSNorm
 * (norm != NULL, into y), optional gated activation (gate != NULL: y *= act),
 * then quantize_q8 into d/q. Returns 1 when every row was finite. y holds the
 * pre-quantization rows (the source rows themselves when no norm is given). */
int orc_row_work(const float *src, const float *norm, float eps, const float *gate, int gelu, uint32_t rows,
                 uint32_t n, float *y, float *d, int8_t *q) {
    uint32_t r, nb = (n + 31u) / 32u;
    int ok = 1;
    for (r = 0; r < rows; ++r) {
        float *row = y + (size_t)r * n;
        if (norm) {
            if (orc_rmsnorm(src + (size_t)r * n, norm, row, n, eps)) {
                ok = 0;
                continue;
            }
        } else if (row != src + (size_t)r * n) {
            memcpy(row, src + (size_t)r * n, (size_t)n * 4);
        }
        if (gate) {
            if (gelu) orc_gelu_mul(row, gate + (size_t)r * n, n);
            else orc_silu_mul(row, gate + (size_t)r * n, n);
        }
        if (orc_quantize_q8(row, n, d + (size_t)r * nb, q + (size_t)r * nb * 32u)) ok = 0;
    }
    return ok;
}

/* ---- attention pieces (src/model.c:425-491, src/kernels.c:1119-1176) ---- */

/* kernels.c:1119-1127: eight lanes over full groups of 8, lane reduction,
 * then the tail added in order. */
float orc_dot_f32(const float *a, const float *b, uint32_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sum;
    uint32_t i, l;
    for (i = 0; i + 8 <= n; i += 8)
        for (l = 0; l < 8; ++l) {
            float p = a[i + l] * b[i + l];
            acc[l] = acc[l] + p;
        }
    sum = lanes_reduce(acc);
    for (; i < n; ++i) {
        float p = a[i] * b[i];
        sum = sum + p;
    }
    return sum;
}

/* model.c:442-450: adjacent pairs (2i, 2i+1), i < pairs, of each head. */
void orc_rope(float *x, uint32_t heads, uint32_t hd, uint32_t pairs, const float *cs, const float *sn) {
    uint32_t h, i;
    for (h = 0; h < heads; ++h, x += hd)
        for (i = 0; i < pairs; ++i) {
            float a = x[2 * i], b = x[2 * i + 1];
            float ac = a * cs[i], bs = b * sn[i], as = a * sn[i], bc = b * cs[i];
            x[2 * i] = ac - bs;
            x[2 * i + 1] = as + bc;
        }
}

/* kernels.c:1154-1176 attend_f32: scores = dot * (1/sqrt(hd)); softmax with
 * the maximum subtracted, exp_det, sequential total, one reciprocal; then
 * out = sum over positions (in order) of (score * inv) * value. */
void orc_attend_f32(const float *q, const float *keys, const float *values, uint32_t stride, uint32_t hd,
                    uint32_t start, uint32_t pos, float *scores, float *out) {
    uint32_t p, j;
    float factor = 1.0f / sqrtf((float)hd), high = -FLT_MAX, total = 0.0f, inv;
    for (p = start; p <= pos; ++p) {
        float s = orc_dot_f32(q, keys + (size_t)p * stride, hd);
        scores[p] = s * factor;
    }
    for (p = start; p <= pos; ++p)
        if (scores[p] > high) high = scores[p];
    for (p = start; p <= pos; ++p) {
        scores[p] = orc_exp_det(scores[p] - high);
        total = total + scores[p];
    }
    inv = 1.0f / total;
    for (j = 0; j < hd; ++j) out[j] = 0.0f;
    for (p = start; p <= pos; ++p) {
        float w = scores[p] * inv;
        const float *v = values + (size_t)p * stride;
        for (j = 0; j < hd; ++j) {
            float t = w * v[j];
            out[j] = out[j] + t;
        }
    }
}

/* sampler.c:57-63: first non-banned id, replaced by any later id whose logit
 * is strictly greater. Returns UINT32_MAX when every id is banned. */
uint32_t orc_argmax(const float *logits, uint32_t n, const unsigned char *banned) {
    uint32_t i, best = UINT32_MAX;
    for (i = 0; i < n; ++i)
        if (!(banned && banned[i]) && (best == UINT32_MAX || logits[i] > logits[best])) best = i;
    return best;
}

/* ---- offline weight rules --------------------------------------------- */

/* tools/q8pack.c:38-44 (also scripts/smoe/quant.ts:73-97): per block
 * scale = f32(max|v| / 127); q = clamp(nearbyint(double(v) / double(scale)),
 * -127, 127), 0 for a zero scale; padding zero. `out` receives rows *
 * ceil(cols/32) 36-byte blocks. */
void orc_q8_weight_rows(const float *x, uint32_t rows, uint32_t cols, unsigned char *out) {
    uint32_t nblocks = (cols + 31u) / 32u, r, b, j;
    for (r = 0; r < rows; ++r) {
        const float *row = x + (size_t)r * cols;
        for (b = 0; b < nblocks; ++b) {
            unsigned char *blk = out + ((size_t)r * nblocks + b) * ORC_Q8_BLOCK;
            uint32_t valid = cols - b * 32u;
            float high = 0.0f, scale;
            if (valid > 32u) valid = 32u;
            for (j = 0; j < valid; ++j)
                if (fabsf(row[b * 32u + j]) > high) high = fabsf(row[b * 32u + j]);
            scale = high / 127.0f;
            memcpy(blk, &scale, 4); /* little-endian host */
            memset(blk + 4, 0, 32);
            for (j = 0; j < valid; ++j) {
                int v = 0;
                if (scale != 0.0f) v = (int)nearbyint((double)row[b * 32u + j] / (double)scale);
                if (v > 127) v = 127;
                if (v < -127) v = -127;
                blk[4 + j] = (unsigned char)(int8_t)v;
            }
        }
    }
}

/* kernels.c:1064-1070: level = clamp(lrintf(v * inv), -16, 15). */
static int q5_level(float v, float inv) {
    float p = v * inv;
    long q = lrintf(p);
    if (q < -16) return -16;
    if (q > 15) return 15;
    return (int)q;
}

/* kernels.c:1083-1117: the signed extreme (largest |x|, first on ties) over
 * 21 divisors -(14.5 + 0.1k); each candidate scale is rounded through f16;
 * zero or non-finite candidates are skipped; squared error in double picks
 * the first minimum. */
void orc_quantize_q5_row(const float *x, uint32_t cols, unsigned char *out) {
    uint32_t nblocks = (cols + 31u) / 32u, b, j, k;
    for (b = 0; b < nblocks; ++b) {
        const float *xb = x + (size_t)b * 32u;
        unsigned char *blk = out + (size_t)b * ORC_Q5_BLOCK;
        uint32_t valid = cols - b * 32u, high = 0;
        float extreme = 0.0f, best_d = 0.0f, inv;
        double best_err = -1.0;
        uint16_t best_h = 0;
        if (valid > 32u) valid = 32u;
        for (j = 0; j < valid; ++j)
            if (fabsf(xb[j]) > fabsf(extreme)) extreme = xb[j];
        if (extreme != 0.0f) {
            for (k = 0; k <= 20u; ++k) {
                float divisor = -(14.5f + 0.1f * (float)k);
                uint16_t h = orc_f32_to_f16(extreme / divisor);
                float d = orc_f16_to_f32(h), dinv;
                double err = 0.0;
                if (d == 0.0f || !(fabsf(d) <= FLT_MAX)) continue;
                dinv = 1.0f / d;
                for (j = 0; j < valid; ++j) {
                    double e = (double)xb[j] - (double)q5_level(xb[j], dinv) * (double)d;
                    err += e * e;
                }
                if (best_err < 0.0 || err < best_err) {
                    best_err = err;
                    best_d = d;
                    best_h = h;
                }
            }
        }
        blk[0] = (unsigned char)(best_h & 0xffu);
        blk[1] = (unsigned char)(best_h >> 8);
        inv = best_d != 0.0f ? 1.0f / best_d : 0.0f;
        memset(blk + 6, 0, 16);
        for (j = 0; j < 32u; ++j) {
            uint32_t u = (uint32_t)(((j < valid && best_d != 0.0f) ? q5_level(xb[j], inv) : 0) + 16);
            high |= ((u >> 4) & 1u) << j;
            if (j < 16u) blk[6 + j] |= (unsigned char)(u & 15u);
            else blk[6 + j - 16u] |= (unsigned char)((u & 15u) << 4);
        }
        blk[2] = (unsigned char)high;
        blk[3] = (unsigned char)(high >> 8);
        blk[4] = (unsigned char)(high >> 16);
        blk[5] = (unsigned char)(high >> 24);
    }
}

/* kernels.c:1044-1062: one row expanded to floats, scale * q. */
void orc_dequantize_row(int q5, const unsigned char *w, uint32_t cols, float *out) {
    uint32_t nblocks = (cols + 31u) / 32u, b, j;
    int8_t q[32];
    for (b = 0; b < nblocks; ++b) {
        uint32_t valid = cols - b * 32u;
        float scale;
        if (valid > 32u) valid = 32u;
        if (q5) {
            const unsigned char *blk = w + (size_t)b * ORC_Q5_BLOCK;
            scale = orc_f16_to_f32(le_u16(blk));
            orc_unpack_q5(blk, q);
        } else {
            const unsigned char *blk = w + (size_t)b * ORC_Q8_BLOCK;
            scale = le_f32(blk);
            memcpy(q, blk + 4, 32);
        }
        for (j = 0; j < valid; ++j) out[b * 32u + j] = scale * (float)q[j];
    }
}
