/* Q5 weight conversion on gfx950 (reference: src/kernels.c:1064-1117,
 * quantize_q5_row, as src/quantize_main.c:107-121 runs it row by row).
 *
 * Per 32-element block: the signed extreme (the first element of largest
 * magnitude; a NaN element is never chosen), then 21 candidate scales
 * d_k = f16(extreme / -(14.5 + 0.1k)) (f32 arithmetic, binary16 rounding to
 * nearest even, k = 0..20; a zero or non-finite d_k is skipped); each
 * candidate's squared error sum_j (x_j - clamp(rint(x_j * (1/d_k)), -16, 15) * d_k)^2
 * is formed in binary64 in element order; the first minimum wins (with a NaN
 * element every sum is NaN and the first kept candidate stays); codes q + 16
 * are packed as 16 nibble bytes (element j low, j + 16 high) after the f16
 * scale and the 32-bit plane of fifth bits (docs/FORMAT.md:124-134).
 *
 * Mapping: half a wave per block. Lane j holds element j (the extreme is a
 * 32-lane reduction over (|x|, -j), so ties keep the first element); lane k < 21
 * then owns candidate k and runs its binary64 error sum over the 32 elements
 * read from LDS in element order, so the 21 serial sums proceed side by side;
 * the winner is the minimum error with ties to the lowest k; lane j quantizes
 * its element with the winner and the half-wave assembles the 22 bytes.
 */
#include <float.h>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t CV_WG = 256;                 /* eight blocks per workgroup */
constexpr uint32_t CV_BLOCKS = CV_WG / 32;

/* lrintf(v * inv) clamped to the 5-bit range (kernels.c:1064-1067). A NaN product takes
 * -16: x86-64's lrintf returns LONG_MIN for it (cvtss2si's "integer indefinite"), which the
 * clamp turns into -16 on the host the reference and the oracle run on. */
__device__ __forceinline__ int q5_level(float v, float inv) {
    const float p = v * inv;
    const float r = __builtin_rintf(p);
    return !(r >= -16.0f) ? -16 : (r > 15.0f ? 15 : (int)r);
}

/* binary32 -> binary16 bits, round to nearest even, overflow to infinity,
 * subnormal results kept (one v_cvt_f16_f32; f16 denormals are on). */
__device__ __forceinline__ uint32_t to_half_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

__global__ __launch_bounds__(CV_WG) void k_quantize_q5(const float *x, uint32_t rows, uint32_t cols,
                                                       unsigned char *out) {
    __shared__ float xs[CV_BLOCKS][32];
    __shared__ double errs[CV_BLOCKS][32];
    const uint32_t tid = threadIdx.x, slot = tid / 32, j = tid % 32;
    const uint32_t nb = (cols + 31) / 32;
    const uint64_t blk = (uint64_t)blockIdx.x * CV_BLOCKS + slot;
    const bool live = blk < (uint64_t)rows * nb; /* uniform per half-wave */
    const uint32_t row = live ? (uint32_t)(blk / nb) : 0, b = live ? (uint32_t)(blk % nb) : 0;
    const uint32_t n = cols - b * 32 < 32 ? cols - b * 32 : 32; /* elements of this block */
    const bool valid = live && j < n;
    const float v = valid ? x[(size_t)row * cols + (size_t)b * 32 + j] : 0.0f;
    xs[slot][j] = v;

    /* the signed extreme: largest |x|, first on ties (kernels.c:1090-1091); a NaN never wins
     * (fabsf(NaN) > m is false there), so it enters as -1 and an all-NaN block keeps extreme 0 */
    float best_a = v == v ? fabsf(v) : -1.0f;
    uint32_t best_j = j;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float oa = __shfl_xor(best_a, off, 32);
        const uint32_t oj = __shfl_xor(best_j, off, 32);
        if (oa > best_a || (oa == best_a && oj < best_j)) {
            best_a = oa;
            best_j = oj;
        }
    }
    __syncthreads(); /* xs */
    const float extreme = best_a > 0.0f ? xs[slot][best_j] : 0.0f;

    /* candidate k = lane j < 21: its scale and its error sum in element order (a NaN element
     * makes every kept candidate's sum NaN) */
    double err = -1.0; /* skipped: no sum of squares is -1 */
    float d = 0.0f;
    uint32_t h = 0;
    if (extreme != 0.0f && j <= 20) {
        const float t = 0.1f * (float)j;
        const float divisor = -(14.5f + t);
        h = to_half_bits(extreme / divisor);
        d = half_to_float(h);
        if (d != 0.0f && fabsf(d) <= FLT_MAX) {
            const float dinv = 1.0f / d;
            double acc = 0.0;
            for (uint32_t e = 0; e < n; ++e) { /* uniform trip count; LDS broadcast reads */
                const float xe = xs[slot][e];
                const double q = (double)q5_level(xe, dinv);
                const double pe = q * (double)d;
                const double de = (double)xe - pe;
                const double sq = de * de;
                acc = acc + sq;
            }
            err = acc;
        }
    }
    errs[slot][j] = err;
    __syncthreads();
    /* first minimum over the kept candidates, as `best < 0 || err < best` (kernels.c:1099): the
     * first kept one is taken whatever its error, so NaN sums leave the first kept candidate */
    uint32_t win = 32;
    double best = -1.0;
    for (uint32_t k = 0; k <= 20; ++k) {
        const double e = errs[slot][k];
        if (e != -1.0 && (best < 0.0 || e < best)) {
            best = e;
            win = k;
        }
    }
    const uint32_t wh = __shfl(h, win < 32 ? win : 0, 32);
    const float wd = win < 32 ? __shfl(d, win, 32) : 0.0f;
    const uint32_t half = win < 32 ? wh : 0u;
    const float inv = wd != 0.0f ? 1.0f / wd : 0.0f;
    const uint32_t u = (uint32_t)((valid && wd != 0.0f ? q5_level(v, inv) : 0) + 16);

    /* pack: high plane bit j = bit 4 of code j; byte 6 + j (j < 16) = code j | code j+16 << 4 */
    const uint64_t hb = __ballot((u >> 4) & 1u);
    const uint32_t high = (uint32_t)(((tid & 63u) < 32 ? hb : hb >> 32) & 0xffffffffu);
    const uint32_t upper = __shfl_down(u, 16, 32);
    if (!live) return;
    unsigned char *o = out + (size_t)row * nb * Q5_BYTES + (size_t)b * Q5_BYTES;
    if (j < 16) o[6 + j] = (unsigned char)((u & 15u) | ((upper & 15u) << 4));
    else if (j < 18) o[j - 16] = (unsigned char)(half >> (8 * (j - 16)));
    else if (j < 22) o[2 + (j - 18)] = (unsigned char)(high >> (8 * (j - 18)));
}

}  // namespace

hipError_t launch_quantize_q5(const float *x, uint32_t rows, uint32_t cols, unsigned char *out, hipStream_t s) {
    const uint64_t blocks = (uint64_t)rows * ((cols + 31) / 32);
    if (!blocks) return hipSuccess;
    const uint64_t grid = (blocks + CV_BLOCKS - 1) / CV_BLOCKS;
    if (grid > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_quantize_q5, dim3((uint32_t)grid), dim3(CV_WG), 0, s, x, rows, cols, out);
    return hipGetLastError();
}

}  // namespace smq
