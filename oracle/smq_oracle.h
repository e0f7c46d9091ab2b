/* CPU oracle for the quantized matrix-product path (test infrastructure only).
 * See smq_oracle.c for what each function restates and what pins it. */
#ifndef SMQ_ORACLE_H
#define SMQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORC_Q8_BLOCK 36u /* f32 scale + int8[32] */
#define ORC_Q5_BLOCK 22u /* f16 scale + u32 high plane + 16 nibble bytes */

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

int orc_quantize_q8(const float *x, uint32_t n, float *d, int8_t *q);
void orc_unpack_q5(const unsigned char *blk, int8_t out[32]);

float orc_dot_q8(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
float orc_dot_q5(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
float orc_dot_q8_fast(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
float orc_dot_q5_fast(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
void orc_dot_x4(int q5, int fast, const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb,
                uint32_t stride, float out[4]);
void orc_dot_r4(int q5, int fast, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                uint32_t nb, float out[4]);
void orc_gemm(int q5, int fast, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
              uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride);
void orc_block_sums(int q5, const unsigned char *w, size_t row_bytes, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, int32_t *sums);
void orc_gemm_blockwise(int q5, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                        uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride);

void orc_split_range(uint32_t total, uint32_t index, uint32_t count, uint32_t *begin, uint32_t *end);
int orc_mat_item(int q5, int fast, const unsigned char *w, size_t row_bytes, uint32_t rows, const float *bias,
                 const float *xd, const int8_t *xq, uint32_t ntok, uint32_t nb, float *y);
int orc_rmsnorm(const float *x, const float *w, float *y, uint32_t n, float eps);

const uint64_t *orc_exp2_table(void);
float orc_exp_det(float x);
void orc_silu_mul(float *up, const float *gate, size_t n);
void orc_gelu_mul(float *up, const float *gate, size_t n);
int orc_row_work(const float *src, const float *norm, float eps, const float *gate, int gelu, uint32_t rows,
                 uint32_t n, float *y, float *d, int8_t *q);

float orc_dot_f32(const float *a, const float *b, uint32_t n);
void orc_rope(float *x, uint32_t heads, uint32_t hd, uint32_t pairs, const float *cs, const float *sn);
void orc_attend_f32(const float *q, const float *keys, const float *values, uint32_t stride, uint32_t hd,
                    uint32_t start, uint32_t pos, float *scores, float *out);
uint32_t orc_argmax(const float *logits, uint32_t n, const unsigned char *banned);

void orc_q8_weight_rows(const float *x, uint32_t rows, uint32_t cols, unsigned char *out);
void orc_quantize_q5_row(const float *x, uint32_t cols, unsigned char *out);
void orc_dequantize_row(int q5, const unsigned char *w, uint32_t cols, float *out);

/* CPU baseline timing (cpu_timing.c): runs `gemm` (a GemmQ8-shaped function,
 * the reference's kernels.h:60-65 signature) over `nmats` weight matrices in
 * turn (blocks of `block_bytes`), rows split statically over `threads` threads with the caller as
 * worker 0, `reps` times; returns the best wall time of one pass in seconds
 * (and each pass's time in times[0, reps) when times is not NULL). */
typedef void (*orc_gemm_fn)(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                            uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride,
                            unsigned char *scratch);
double orc_time_gemm_pass(orc_gemm_fn gemm, const unsigned char *const *mats, const uint32_t *rows,
                          const uint32_t *nbs, const float *const *xds, const int8_t *const *xqs, uint32_t nmats,
                          uint32_t ntok, uint32_t block_bytes, float *out, uint32_t threads, uint32_t reps,
                          size_t scratch_bytes, double *times);
/* The oracle's own scalar gemm in the GemmQ8 shape (exact contract, Q8 / Q5). */
void orc_gemm_q8_fn(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);
void orc_gemm_q5_fn(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);

#endif
