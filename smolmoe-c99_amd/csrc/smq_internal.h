/* Internal launch interface between the C ABI (smq_api.cpp) and the gfx950
 * kernels (smq_kernels.hip). Not installed; include/smq.h is the public ABI. */
#ifndef SMQ_INTERNAL_H
#define SMQ_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace smq {

constexpr uint32_t QK = 32;
constexpr uint32_t Q8_BYTES = 36;
constexpr uint32_t Q5_BYTES = 22;
constexpr uint32_t MAX_ITEMS = 4;
/* The decode GEMV and the exact GEMM stage the whole activation (or a token
 * tile of it) in LDS; wider rows take the generic kernel. */
constexpr uint32_t MAX_FAST_NB = 512;

/* One matrix of a fused launch: rows of `row_bytes`, output
 * y[t * y_stride + r] (+ bias[r]). */
struct Item {
    const unsigned char *w;
    size_t row_bytes;
    const float *bias;
    float *y;
    size_t y_stride;
    uint32_t rows;
    uint32_t tile_begin; /* first workgroup tile of this item */
};

struct MatArgs {
    Item item[MAX_ITEMS];
    uint32_t nitems;
    const float *xd;
    const int8_t *xq;
    uint32_t nb, ntok;
    uint32_t xstride; /* blocks between consecutive activations (nb when packed) */
    int *flag; /* set to 1 on a non-finite output; may be NULL */
};

/* Launchers; each returns the hipError_t of its launch. */
hipError_t launch_quantize_q8(const float *x, uint32_t rows, uint32_t n, float *d, int8_t *q, int *flag,
                              hipStream_t s);
hipError_t launch_matmul(const MatArgs &a, bool q5, bool fast, hipStream_t s);
/* Int8-MFMA prefill GEMM (relaxed block order). sums != NULL writes the exact
 * per-block int32 sums, sums[(t*rows + r)*nb + b], instead of the outputs.
 * mfma_layout_ok: 4-byte aligned rows and activations, even nb for Q5. */
bool mfma_layout_ok(const MatArgs &a, bool q5);
hipError_t launch_matmul_mfma(const MatArgs &a, bool q5, int32_t *sums, hipStream_t s);
/* Activation producer rows (model.c:354-415): optional RMSNorm, optional
 * gated activation (act 1 = SwiGLU, 2 = GeGLU), optional f32 store, Q8. */
constexpr uint32_t MAX_ROW = 16384;
hipError_t launch_row_quantize(const float *src, const float *norm, float eps, const float *gate, int act,
                               uint32_t rows, uint32_t n, float *y, float *d, int8_t *q, int *flag, hipStream_t s);
hipError_t launch_dequantize_row(const unsigned char *w, uint32_t cols, float *out, bool q5, hipStream_t s);

}  // namespace smq

#endif
