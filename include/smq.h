/* smq.h - C ABI of the MI355X (gfx950) quantized matrix-product path.
 *
 * A drop-in for the reference's kernel seam (src/kernels.h in
 * ktfth/smolmoe-c99): activation quantization to Q8, Q8 and Q5 weight rows
 * against Q8 activations (dot, 4-token, 4-row and gemm variants), the fused
 * matmul of up to four matrices sharing one input with bias and a finiteness
 * check (src/model.c:236-310), and row dequantization for embeddings.
 *
 * Conventions
 *  - Every array argument is a DEVICE pointer (hipMalloc'd or from smq_malloc)
 *    unless its comment says "host".
 *  - Work is enqueued on the library stream (smq_stream / smq_set_stream) and
 *    is ordered like any other work on that stream. Functions that return a
 *    computed value (smq_quantize_q8, smq_dot_q8, smq_dot_q5) synchronize.
 *  - Block layouts are the reference's on-disk layouts (docs/FORMAT.md:124-150):
 *    Q8 block = f32 LE scale + int8[32] (36 B); Q5 block = f16 LE scale + u32 LE
 *    high-bit plane + 16 nibble bytes (22 B); value = scale * (q - 16).
 *  - Results follow the reference's arithmetic contract (docs/FORMAT.md:152-171):
 *    exact int32 lane sums of 4 products, per lane acc = acc + (ws*xs)*lane in
 *    increasing block order (a single fmaf per lane in fast mode), then
 *    ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). Every smq_gemm_* output is bit
 *    identical to the reference's scalar kernel, except smq_gemm_*_mfma, whose
 *    per-block int32 sums are exact but whose f32 block order differs.
 *  - Errors: functions return or record an smq_status (the reference's
 *    sm_status values, src/util.h:28-37); smq_last_status / smq_last_error give
 *    the calling thread's latest failure (src/util.h:44-47).
 */
#ifndef SMQ_H
#define SMQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMQ_QK 32u
#define SMQ_Q8_BLOCK_BYTES 36u /* kernels.h:46 */
#define SMQ_Q5_BLOCK_BYTES 22u /* kernels.h:47 */

/* src/util.h:28-37 */
typedef enum smq_status {
    SMQ_OK = 0,
    SMQ_ERR = 1,
    SMQ_ERR_IO = 2,
    SMQ_ERR_FORMAT = 3,
    SMQ_ERR_RANGE = 4,
    SMQ_ERR_NUMERIC = 5,
    SMQ_ERR_NOMEM = 6,
    SMQ_ERR_STATE = 7
} smq_status;

/* The calling thread's latest status and message (src/util.h:44-47). */
smq_status smq_last_status(void);
const char *smq_last_error(void);
void smq_clear_error(void);
/* Records a status and message for the calling thread, as sm_set does
 * (src/util.h:40-43), so host code layered on this library (the forward pass
 * in smq_model.h) reports through the same smq_last_error. Returns status. */
smq_status smq_set_error(smq_status status, const char *message);

/* ---- context ------------------------------------------------------------
 * One device per process (the reference's kernel table is process-global,
 * src/kernels.c:20-27). smq_init selects the device, checks it is gfx950 and
 * creates the library stream. */
smq_status smq_init(int device);
void smq_shutdown(void);
void *smq_stream(void);                      /* hipStream_t */
smq_status smq_set_stream(void *hip_stream); /* NULL restores the library stream */
smq_status smq_synchronize(void);
/* Device name of the selected GPU, e.g. "gfx950". */
const char *smq_device_arch(void);

/* ---- backend selection (src/kernels.h:72-87) -----------------------------
 * smq_kernels_select installs the GPU kernels behind the smq_* entry points
 * and returns the backend name: "gfx950" (exact mul+add contract) or
 * "gfx950-fast" (lane-wise FMA, kernels.h:9-11). force_exact ignores fast. */
const char *smq_kernels_select(int force_exact);
void smq_kernels_set_fast(int fast); /* kernels.h:77 */
int smq_kernels_fast(void);          /* kernels.h:78 */
/* kernels.h:72-73. The GPU kernels need no caller scratch: returns 0, and
 * every smq_gemm_* accepts scratch == NULL (a non-NULL scratch is ignored). */
size_t smq_gemm_scratch_bytes(uint32_t nb);
/* Host-side bounds checks of every operand range against its device
 * allocation before a launch (no reference counterpart). On by default, or
 * off when the environment sets SMQ_CHECKS=0. Ranges inside smq_malloc
 * allocations are checked against the library's own record; other device
 * memory through the runtime, except during a capture, where such ranges are
 * taken as given (no runtime call runs inside a capture). */
void smq_set_checks(int on);

/* ---- activation quantizer (src/kernels.h:183-187, kernels.c:912-935) ---- */
/* QuantizeQ8: n floats -> ceil(n/32) f32 scales d and 32*ceil(n/32) int8 q,
 * padding zero. Synchronous. Returns 0, or -1 if any input is inf or NaN (then
 * d and q are unspecified, as the reference's caller never reads them). */
int smq_quantize_q8(const float *x, uint32_t n, float *d, int8_t *q);
/* The caller's per-token loop (model.c:354-370): `rows` rows of n floats,
 * row r at x + r*n, into d + r*nb and q + r*nb*32. Asynchronous: a non-finite
 * input raises the sticky numeric flag read by smq_numeric_check. */
smq_status smq_quantize_q8_rows(const float *x, uint32_t rows, uint32_t n, float *d, int8_t *q);

/* ---- activation producers (src/model.c:347-415, src/vecmath.c:61-93) ----
 * The caller's per-token row work (row_work, model.c:354-362) for `rows` rows
 * of n floats (n <= 16384): optional RMSNorm with weight `norm` (NULL: none)
 * and eps (model.c:334-342, sequential f32 sum of squares); optional gated
 * activation with `gate` (act 0 = none, 1 = SwiGLU vecmath.c:78-81,
 * 2 = GeGLU vecmath.c:86-93, both with the deterministic binary64 exp of
 * vecmath.c:61-76); the f32 result stored to y when y != NULL (y may alias
 * src, as silu_quantize updates m->up in place); then quantize_q8 into
 * d + r*nb, q + r*nb*32. Bit-identical to the reference. A non-finite sum,
 * scale or value raises the sticky numeric flag. Asynchronous. */
smq_status smq_row_quantize(const float *src, const float *norm, float eps, const float *gate, int act, uint32_t rows,
                            uint32_t n, float *y, float *d, int8_t *q);
/* norm_quantize (model.c:393-400): RMSNorm then quantize. */
smq_status smq_norm_quantize(const float *src, const float *norm, float eps, uint32_t rows, uint32_t n, float *y,
                             float *d, int8_t *q);
/* silu_quantize (model.c:409-415): up *= act(gate) in place, then quantize;
 * gemma3 != 0 selects GeGLU. */
smq_status smq_silu_quantize(float *up, const float *gate, int gemma3, uint32_t rows, uint32_t n, float *d,
                             int8_t *q);

/* ---- dot products and gemm (src/kernels.h:49-70) -------------------------
 * Parameter lists are those of DotQ8, DotQ8x4, DotQ8R4 and GemmQ8. out is a
 * device array; smq_dot_q8/q5 return the value (synchronous). */
float smq_dot_q8(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
float smq_dot_q5(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb);
void smq_dot_q8_x4(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, uint32_t stride,
                   float *out);
void smq_dot_q5_x4(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, uint32_t stride,
                   float *out);
void smq_dot_q8_r4(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nb,
                   float *out);
void smq_dot_q5_r4(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nb,
                   float *out);
/* GemmQ8: out[t*stride + r] = dot(row r, activation t); activation t at
 * xd + t*nb, xq + t*nb*32. Decode (ntok == 1) runs the bandwidth GEMV;
 * ntok > 1 runs the exact LDS-tiled GEMM. Asynchronous. */
void smq_gemm_q8(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                 uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);
void smq_gemm_q5(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                 uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);
/* Prefill GEMM on int8 MFMA (no reference counterpart for its order: the
 * reference has one order). The per-block int32 sums are exact; each output is
 * acc = fma(wscale*xscale, float(blocksum), acc) over blocks in order, which
 * matches the exact contract within 1e-5 relative (|err| <= 1e-5 * max|out|
 * over a token's outputs). Same parameters as GemmQ8. Asynchronous. */
void smq_gemm_q8_mfma(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                      uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);
void smq_gemm_q5_mfma(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                      uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch);
/* The MFMA path's per-block int32 sums, sums[(t*nrows + r)*nb + b] (device),
 * for the bit-exact integer check (test entry point, no reference counterpart). */
void smq_block_sums(int q5, const unsigned char *w, size_t row_bytes, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, int32_t *sums);
/* Which kernel smq_matmul uses when ntok > 1: 0 = the exact GEMM (default,
 * bit-identical to the reference), 1 = the int8-MFMA GEMM. */
void smq_set_prefill_mfma(int on);
/* Tuning (no reference counterpart): rows per workgroup of the
 * one-launch decode GEMV, 1, 2, 4, 8 or 16 (every output unchanged), or 0 =
 * chosen per width and row count (the default). Any other value is refused
 * with SMQ_ERR_RANGE. */
smq_status smq_set_gemv_rows(int rows);
/* Tuning (no reference counterpart): which kernel the exact prefill GEMM
 * (smq_gemm_q8 / smq_gemm_q5 / smq_matmul with ntok > 1) takes: 0 = chosen by
 * shape (the default), 1 = the one whose lane sums run on the matrix cores,
 * 2 = the one whose lane sums run as v_dot4, 3 (4) = the matrix-core one with
 * each tile's eight lane sums split over two (four) waves. Every output is the
 * same, bit for bit. Any other value is refused with SMQ_ERR_RANGE. */
smq_status smq_set_exact_gemm(int mode);

/* ---- fused matmul with bias and finiteness (src/model.c:236-310) -------- */
/* QMat (model.h:15-19): a weight matrix in device memory. dtype 1 = Q8, 2 = Q5
 * (docs/FORMAT.md:101). */
typedef struct smq_qmat {
    const unsigned char *data;
    uint32_t rows, cols, nb, dtype;
    size_t row_bytes;
} smq_qmat;
/* MatItem (model.c:236-240): y[token*w->rows + row] = dot + bias[row].
 * accumulate != 0 adds the result into y instead (y = y + result: the
 * residual add_rows of model.c:452-455 fused into the store, model.c:540,
 * 643); the finiteness check still looks at the result before the add. */
typedef struct smq_mat_item {
    const smq_qmat *w; /* host pointer to the descriptor */
    const float *bias; /* device, may be NULL */
    float *y;          /* device */
    int accumulate;
} smq_mat_item;
#define SMQ_MAX_ITEMS 4
/* Up to SMQ_MAX_ITEMS matrices with the same nb sharing one quantized input,
 * in one launch. A non-finite output raises the sticky numeric flag.
 * Asynchronous; SMQ_ERR_STATE if the items differ in width (model.c:298). */
smq_status smq_matmul(const smq_mat_item *items, uint32_t n, const float *xd, const int8_t *xq, uint32_t ntok);
/* No reference counterpart (the reference runs such matrices one matmul
 * after another, e.g. its experts in routed_experts, model.c:587-606):
 * independent decode GEMVs (one token each) in one launch. Item i computes
 * y_i[r] = dot(w_i row r, x_i) (+ bias_i[r]; added into y_i when accumulate),
 * with its own quantized activation x_i = (xd_i, xq_i). All items share nb
 * and the weight format; every output is bit-identical to smq_matmul's.
 * Persistent workgroups stream all items' weights back to back. At most
 * SMQ_MAX_GROUP items; asynchronous; the numeric flag as smq_matmul. */
#define SMQ_MAX_GROUP 48
typedef struct smq_group_item {
    const smq_qmat *w;  /* host pointer to the descriptor */
    const float *bias;  /* device, may be NULL */
    float *y;           /* device */
    int accumulate;
    const float *xd;    /* device: nb scales */
    const int8_t *xq;   /* device: nb*32 values */
} smq_group_item;
smq_status smq_gemv_grouped(const smq_group_item *items, uint32_t n);
/* A plan of independent one-token Q8 GEMVs streamed by one launch (no
 * reference counterpart: the reference runs them one after another), for
 * more items than SMQ_MAX_GROUP and for 28- and 152-block rows together (the
 * 896- and 4864-wide projections of Qwen2.5-0.5B: a whole FFN step's 72
 * GEMVs in one launch). Every item: packed Q8 rows (row_bytes = nb*36) of
 * nb = 28 or 152 blocks, 16-byte aligned, 4-byte aligned activations; every
 * output bit-identical to smq_matmul's. smq_gemv_plan_create validates the
 * items, splits them over workgroups in proportion to their bytes and copies
 * the split to device memory the plan owns (synchronously; not under
 * capture). smq_gemv_plan_launch is one asynchronous launch that may be
 * captured; the numeric flag as smq_matmul. The items' buffers must outlive
 * the plan; destroy a plan after every graph that launches it. */
#define SMQ_MAX_PLAN_ITEMS 4096
typedef struct smq_gemv_plan smq_gemv_plan;
smq_status smq_gemv_plan_create(const smq_group_item *items, uint32_t n, smq_gemv_plan **plan);
smq_status smq_gemv_plan_launch(const smq_gemv_plan *plan);
void smq_gemv_plan_destroy(smq_gemv_plan *plan);
/* Synchronizes, then returns SMQ_ERR_NUMERIC (and clears the flag) if any
 * quantize or matmul since the last check saw a non-finite value. */
/* ---- fused decode matmuls (one token) --------------------------------------
 * The activation of a decode matmul formed inside the matmul's own launch:
 * norm_quantize + matmul (model.c:503-509, 636-638) and silu_quantize +
 * matmul (model.c:639-643) without the activation round trip. Outputs are
 * bit-identical to the two-call forms, which these calls fall back to where
 * a shape does not fit the fused kernel (then the Q8 blocks go to the
 * scratch buffers). */
#define SMQ_ACT_Q8 0   /* xd, xq: the quantized activation */
#define SMQ_ACT_NORM 1 /* RMSNorm of x with norm and eps (model.c:334-342), then Q8 */
#define SMQ_ACT_F32 2  /* Q8 of the f32 row x (kernels.c:912-935) */
typedef struct smq_act {
    int kind;
    uint32_t cols;          /* elements: the matrices' cols */
    const float *x;         /* NORM, F32: cols floats */
    const float *norm;      /* NORM: cols floats */
    float eps;              /* NORM */
    const float *xd;        /* Q8: ceil(cols/32) scales */
    const int8_t *xq;       /* Q8: ceil(cols/32)*32 values */
    float *xd_scratch;      /* NORM, F32: room for the Q8 blocks if the call falls back */
    int8_t *xq_scratch;
} smq_act;
/* smq_matmul of one token with the activation `act`. */
smq_status smq_matmul_act(const smq_mat_item *items, uint32_t n, const smq_act *act);
/* The gate/up pair of a dense FFN (model.c:636-640): h[r] = up[r] *
 * act(gate[r]) with act 1 SwiGLU, 2 GeGLU (vecmath.c:78-93), gate and up the
 * matmuls of `act` (same rows and cols, no bias); a non-finite gate or up
 * raises the numeric flag. gate_scratch (gate->rows floats) holds the gate
 * row if the call falls back. */
smq_status smq_matmul_glu(const smq_qmat *gate, const smq_qmat *up, const smq_act *act, int glu, float *h,
                          float *gate_scratch);
/* smq_matmul_glu followed by silu_quantize's quantization (model.c:409-415:
 * quantize_q8 of h): hd (ceil(rows/32) scales) and hq (32 per block) receive
 * h's Q8 blocks, h (may be NULL where the shape allows) the f32 values. On
 * packed 896-wide Q8 rows the whole step is one launch; other shapes take the
 * two-call form, which needs h. The numeric flag as smq_matmul_glu, plus a
 * non-finite h. */
smq_status smq_matmul_glu_q8(const smq_qmat *gate, const smq_qmat *up, const smq_act *act, int glu, float *h,
                             float *hd, int8_t *hq, float *gate_scratch);
smq_status smq_numeric_check(void);

/* ---- decoder pieces around the matmuls ----------------------------------
 * Device-resident steps of the reference's forward pass (src/model.c:425-542,
 * 669-677) and its greedy choice (src/sampler.c:57-63). `pos_dev`, when not
 * NULL, is a device int32 read by the kernel in place of pos0, so a captured
 * decode step replays at successive positions. */
typedef struct smq_attn_shape {
    uint32_t heads, kv_heads, head_dim; /* query heads, KV heads (heads % kv_heads == 0) */
    uint32_t rotary_pairs;              /* rotary_dim / 2 (config.c:25-47) */
    uint32_t window;                    /* sliding window, 0 = full causal (model.c:466-470) */
    uint32_t context;                   /* positions the caches hold */
} smq_attn_shape;
/* model.c:511-526: for each of ntok tokens at position p = pos0 + t, rotate
 * q[t] (heads*head_dim) and k[t] (kv_heads*head_dim) in place by the table
 * rows cos_table[p], sin_table[p] (rotary_pairs floats each, model.c:425-450),
 * then store k[t] and v[t] into keys[p] and values[p] (kv_heads*head_dim f32
 * each). A position at or past context raises the numeric flag instead. */
smq_status smq_rope_kv(float *q, float *k, const float *v, uint32_t ntok, const smq_attn_shape *shape,
                       const float *cos_table, const float *sin_table, float *keys, float *values, uint32_t pos0,
                       const int32_t *pos_dev);
/* model.c:459-491 with attend_f32 (kernels.c:1154-1176): causal attention of
 * each query head of ntok tokens over keys/values[start .. p], p = pos0 + t,
 * in the reference's order (8-lane dot, exp_det softmax, sums in position
 * order), writing att[t] (heads*head_dim). Bit identical to the reference. */
smq_status smq_attention(const float *q, const float *keys, const float *values, float *att, uint32_t ntok,
                         const smq_attn_shape *shape, uint32_t pos0, const int32_t *pos_dev);
/* smq_attention followed by quantize_attention (model.c:402-406): att rows
 * also quantized to Q8 into xd (ntok*nb f32) and xq (ntok*nb*32), nb =
 * ceil(heads*head_dim / 32); one launch when head_dim % 32 == 0. */
smq_status smq_attention_q8(const float *q, const float *keys, const float *values, float *att, uint32_t ntok,
                            const smq_attn_shape *shape, uint32_t pos0, const int32_t *pos_dev, float *xd,
                            int8_t *xq);
/* One decoding token (model.c:511-542 for ntok = 1): smq_rope_kv, then
 * smq_attention_q8, as one launch where the shape allows (head_dim 64,
 * 16-byte aligned q, k, v and caches; otherwise the two calls). q and k are the unrotated QKV outputs; afterwards their contents
 * are unspecified (rotated or not). keys/values[p] receive the rotated k and
 * v of this position, att the attention row, xd/xq its Q8 blocks. */
smq_status smq_attention_rope_q8(float *q, float *k, const float *v, const smq_attn_shape *shape,
                                 const float *cos_table, const float *sin_table, float *keys, float *values,
                                 float *att, uint32_t pos0, const int32_t *pos_dev, float *xd, int8_t *xq);
/* The q, k, v matmuls of one decoding token (items[0..2], rows q_dim, kv_dim,
 * kv_dim, no accumulate) with the activation `act`, followed by RoPE and the
 * cache store (model.c:496-526): the same results as smq_matmul_act then
 * smq_rope_kv(items[0].y, items[1].y, items[2].y, 1, ...), i.e. q and k rotated
 * by the position's table rows (model.c:442-450) in their outputs, and the
 * rotated k and the v row written into keys/values at the position (pos_dev if
 * not NULL, else pos0). Q8 rows of 28 blocks with an RMSNorm activation do it in
 * one launch. No reference counterpart of its own: it fuses the two calls above,
 * each of which has one. */
smq_status smq_matmul_act_rope(const smq_mat_item *items, const smq_act *act, const smq_attn_shape *shape,
                               const float *cos_table, const float *sin_table, float *keys, float *values,
                               uint32_t pos0, const int32_t *pos_dev);
/* sampler.c:57-63: *token = first non-banned id, replaced by any later
 * non-banned id with a strictly greater logit (NaN never wins unless it is
 * the first candidate). banned may be NULL. UINT32_MAX if every id is banned. */
smq_status smq_argmax(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): smq_argmax with its partial results in a static device
 * array of the library (12 KiB per GPU, bound at smq_init) instead of the
 * library's allocated workspace; it calls no allocation routine. Same result
 * as smq_argmax. vocab is limited to 1,048,576 ids (SMQ_ERR_RANGE beyond).
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (different streams, or concurrent host threads) race. Asynchronous. */
smq_status smq_argmax_noalloc(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token);
/* model.c:669-677: x[t] = dequantized row tokens[t] of the embedding matrix
 * (embed->cols floats). Ids must be < embed->rows (checked by the caller, as
 * model.c:671-672 does; an id out of range raises the numeric flag). */
smq_status smq_embed(const smq_qmat *embed, const uint32_t *tokens, uint32_t ntok, float *x);
/* Decode-loop bookkeeping on the device: history[*count] = *token when
 * *count < capacity, then ++*count and ++*pos (lets a captured step advance). */
smq_status smq_decode_advance(int32_t *pos, uint32_t *count, const uint32_t *token, uint32_t *history,
                              uint32_t capacity);
/* smq_argmax then smq_decode_advance in one call (the greedy step of the
 * reference's generation loop, main.c:580-600, on device state). Calls on one
 * stream share the library's argmax workspace; concurrent calls on different
 * streams race. */
smq_status smq_argmax_advance(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token,
                              int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity);
/* smq_argmax_advance, then the chosen token's embedding row into x
 * (embed->cols floats): the next decode step's input (model.c:669-677), so a
 * captured step needs no embedding launch of its own. No reference
 * counterpart: it fuses the greedy pick (sampler.c:57-63) with the next
 * step's smq_embed. An id past the vocabulary (every id banned) raises the
 * numeric flag instead of writing x, as smq_embed does. */
smq_status smq_argmax_advance_embed(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token,
                                    int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity,
                                    const smq_qmat *embed, float *x);

/* ---- Q5 weight conversion (src/kernels.h:205, kernels.c:1064-1117) -------
 * quantize_q5_row: cols floats x -> ceil(cols/32) Q5 blocks (22 B each) at
 * out, byte for byte the reference's: signed extreme, the first minimum of 21
 * f16-rounded candidate scales by binary64 squared error, codes packed as in
 * docs/FORMAT.md:124-134. Device pointers, asynchronous. */
void smq_quantize_q5_row(const float *x, uint32_t cols, unsigned char *out);
/* The converter's loop over a tensor (src/quantize_main.c:107-121): `rows`
 * rows of cols floats (row r at x + r*cols) into rows of ceil(cols/32)*22
 * bytes (row r at out + r*ceil(cols/32)*22), one launch. */
smq_status smq_quantize_q5_rows(const float *x, uint32_t rows, uint32_t cols, unsigned char *out);

/* ---- dequantization (src/kernels.h:193-196, kernels.c:1044-1062) -------- */
void smq_dequantize_q8_row(const unsigned char *w, uint32_t cols, float *out);
void smq_dequantize_q5_row(const unsigned char *w, uint32_t cols, float *out);

/* ---- graph capture (no reference counterpart: amortizes launches) -------
 * Work enqueued on the library stream between smq_capture_begin and
 * smq_capture_end is recorded, not run, and replayed by smq_graph_launch
 * (a HIP graph). Only asynchronous entry points may be captured: smq_gemm_*,
 * smq_dot_*_x4/_r4, smq_matmul, smq_quantize_q8_rows, smq_dequantize_*. */
smq_status smq_capture_begin(void);
void *smq_capture_end(void);
smq_status smq_graph_launch(void *graph);
void smq_graph_destroy(void *graph);

/* ---- device memory and timing helpers (plumbing for C hosts and tests) -- */
void *smq_malloc(size_t bytes);
void smq_free(void *p);
smq_status smq_memcpy_htod(void *dst, const void *host_src, size_t bytes);
smq_status smq_memcpy_dtoh(void *host_dst, const void *src, size_t bytes);
smq_status smq_memcpy_dtod(void *dst, const void *src, size_t bytes);
smq_status smq_memset(void *dst, int value, size_t bytes);
/* Records a start event on the library stream. */
smq_status smq_timer_start(void);
/* Records a stop event, waits for it, returns milliseconds since start (<0 on error). */
double smq_timer_stop(void);

/* ---- cross-workgroup hand-off anchor (no reference counterpart: measurement)
 * One launch of `workgroups` workgroups (1..the device's CU count; each holds
 * 96 KB of LDS, so one per CU and all resident) passing `episodes` (<= 100000)
 * grid barriers, timed on the library stream into *ms (host). kind 0: one
 * counter, every workgroup adds 1 and waits for the generation's total; kind
 * 1: eight counters by workgroup index % 8 (the XCD the workgroup is dealt
 * to), the last arriver of each adds 1 to one release counter; kind 2: no
 * atomics, every workgroup stores the generation into a word of its own,
 * workgroup 0 waits for all of them and publishes it. Agent-scope release and
 * acquire. Every wait is bounded (2^20 polls), a workgroup that gives up ends
 * every other wait, and the call then returns SMQ_ERR_STATE. Synchronizes;
 * not for use under capture; allocates a 2.5 KB counter buffer once. */
smq_status smq_grid_barrier_probe(uint32_t workgroups, uint32_t episodes, uint32_t kind, double *ms);

/* ---- HBM bandwidth anchors (no reference counterpart: measurement) ------
 * Plain kernels that read (smq_stream_read) or copy (smq_stream_copy) `bytes`
 * (a multiple of 16, 16-byte aligned) with coalesced 16-byte loads, so a
 * GEMV's GB/s can be read against what the device's HBM delivers. A grid of
 * `workgroups` x `threads` (64..1024, a multiple of 64) threads; nontemporal
 * selects non-temporal loads and stores. The read writes nothing (`sink`, a
 * device word, is written only for one improbable data pattern).
 * Asynchronous, capturable. */
smq_status smq_stream_read(const void *p, size_t bytes, uint32_t workgroups, uint32_t threads, int nontemporal,
                           uint32_t *sink);
smq_status smq_stream_copy(void *dst, const void *src, size_t bytes, uint32_t workgroups, uint32_t threads,
                           int nontemporal);

#ifdef __cplusplus
}
#endif

#endif
