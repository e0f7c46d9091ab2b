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
    int accumulate;      /* y += result (the residual add of model.c:540, 643) */
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

/* Grouped decode GEMV (ntok == 1): independent matrices with the same nb,
 * each with its own activation, streamed by persistent workgroups. */
constexpr uint32_t MAX_GROUP_ITEMS = 48;
struct GroupItem {
    const unsigned char *w;
    size_t row_bytes;
    const float *bias;
    float *y;
    const float *xd;
    const int8_t *xq;
    uint32_t rows;
    uint32_t tile_begin;
    int accumulate;
    uint32_t wg_begin, nwg; /* pinned launch: this item's workgroups */
};
template <uint32_t N>
struct GroupArgsN {
    GroupItem item[N];
    uint32_t nitems, nb, total_tiles;
    int *flag;
    uint32_t cpr, nch, rt; /* pinned launch: tasks per chunk, chunks per row, rows per tile */
};
using GroupArgs = GroupArgsN<MAX_GROUP_ITEMS>;
/* A launch of at most FEW_GROUP_ITEMS items (a single matmul, the decode LM head) passes this
 * copy by value: about 0.3 KB of kernel arguments instead of 3.5 KB. */
constexpr uint32_t FEW_GROUP_ITEMS = 4;
using GroupArgsFew = GroupArgsN<FEW_GROUP_ITEMS>;
inline GroupArgsFew group_args_few(const GroupArgs &g) {
    GroupArgsFew f;
    for (uint32_t i = 0; i < FEW_GROUP_ITEMS; ++i) f.item[i] = g.item[i];
    f.nitems = g.nitems;
    f.nb = g.nb;
    f.total_tiles = g.total_tiles;
    f.flag = g.flag;
    f.cpr = g.cpr;
    f.nch = g.nch;
    f.rt = g.rt;
    return f;
}
/* Coalesced-tile Q8 GEMV (csrc/smq_gemv.hip): rows of nb = 28 or 152 blocks
 * packed at 36*nb bytes, 16-byte aligned, 4-byte aligned activations. */
bool gemv_ct_ok(const GroupArgs &g, bool q5);
hipError_t launch_gemv_ct(GroupArgs &g, bool fast, hipStream_t s);
/* A planned grouped launch (csrc/smq_gemv.hip): one descriptor per workgroup, a contiguous tile range
 * [t0, t1), t1 > t0, of one item; kind 0 = Q8 rows of 28 blocks (tiles of plan_rows_per_tile(false)
 * rows), 1 = Q8 rows of 152 blocks (plan_rows_per_tile(true) rows); both as gemv_ct_ok requires. */
struct PlanWg {
    GroupItem item;
    uint32_t t0, t1, kind, pad;
};
uint32_t plan_rows_per_tile(bool wide);
hipError_t plan_resident(int &per_cu);
hipError_t launch_gemv_plan(const PlanWg *wgs, uint32_t n, bool fast, bool bp, int *flag, hipStream_t s);
/* Layout the streaming kernel needs: 4-byte aligned rows, Q5 nb even. */
bool group_layout_ok(const GroupArgs &g, bool q5);
hipError_t launch_gemv_grouped(GroupArgs &g, bool q5, bool fast, hipStream_t s);

/* Fused decode GEMV (ntok == 1): the activation formed in the launch
 * (pro 0: Q8 given in xd/xq; 1: RMSNorm of src with norm/eps, then Q8; 2: Q8
 * of the f32 row src; n columns), and optionally the gated product of a
 * gate/up pair (glu: items 0 and 1, `rows` each, h = up * act(gate); act 1
 * SwiGLU, 2 GeGLU). fused_layout_ok: 4-byte aligned rows, nb <= MAX_FAST_NB,
 * even nb for Q5, n <= MAX_NORM_K for RMSNorm. The exact contract only (the
 * fast one takes the unfused calls). */
constexpr uint32_t MAX_NORM_K = 8192;
/* Decode QKV store with RoPE (items q, k, v of one token): q and k rows rotated by the position's
 * table row, q, k and v stored to their items and k and v also into the caches at the position. */
struct RopeStore {
    const float *cs, *sn;   /* [context][pairs] */
    float *kcache, *vcache; /* [context][kv_dim] */
    const int32_t *pos_dev; /* the position, else pos0 */
    uint32_t pos0, head_dim, pairs, kv_dim, context;
};
struct FusedArgs {
    Item item[MAX_ITEMS];
    uint32_t nitems, nb, n;
    const float *src, *norm;
    float eps;
    const float *xd;
    const int8_t *xq;
    float *h;
    float *hd;  /* GLU: Q8 blocks of h (rows/32 scales, rows int8), or NULL */
    int8_t *hq;
    uint32_t rows;
    int act;
    int *flag;
    RopeStore rope; /* rope.kcache set: the decode QKV store with RoPE */
};
bool fused_layout_ok(const FusedArgs &a, bool q5, int pro);
/* Decode matmuls on packed 28-block Q8 rows with the activation formed in the launch and,
 * for glu, h and its Q8 blocks formed in the store (csrc/smq_decode.hip). decode_ct_ok: Q8,
 * nb 28, 16-byte aligned packed rows, pro 1 (RMSNorm) or 2 (f32 row), glu with hd/hq. */
bool decode_ct_ok(const FusedArgs &a, bool q5, int pro, bool glu);
hipError_t launch_decode_ct(const FusedArgs &a, int pro, bool glu, hipStream_t s);
/* Rows per decode-GEMV workgroup for nb blocks (smq_kernels.hip). */
int gemv_rows_per_tile(uint32_t nb, bool q5, uint32_t total_rows);
/* Tuning, set from the host thread that launches: rows per tile of the
 * one-tile-per-workgroup decode GEMV (0 = chosen per width, else 1, 2, 4, 8
 * or 16; false for any other value), and whether prefill attention takes the
 * grouped kernel. */
bool set_gemv_rows(int rt);
void set_att_grouped(bool on);
/* Which kernel the exact prefill GEMM (ntok > 1) takes: 0 = chosen by shape, 1 = the MFMA lane-sum
 * kernel, 2 = the VALU kernel, 3 (4) = the MFMA lane-sum kernel with each tile's lane sums split over two
 * (four) waves (false for any other value); every output is the same. */
bool set_exact_gemm(int mode);
/* The exact prefill GEMM with its lane sums on f16 MFMA (csrc/smq_mfma.hip): fast_layout shapes; split 1:
 * 32 x 32 tiles of rows and tokens; 2: 16 x 32 tiles whose lane sums 0-3 and 4-7 run in two waves; 4: 16 x 16
 * tiles, two lane sums per wave. */
hipError_t launch_gemm_xm(MatArgs a, bool q5, bool fast, int split, hipStream_t s);
hipError_t launch_matmul_fused(const FusedArgs &a, bool q5, int pro, bool glu, hipStream_t s);
/* h = h * act(gate) elementwise (act 1 SwiGLU, 2 GeGLU). */
hipError_t launch_glu(float *h, const float *gate, uint32_t n, int act, hipStream_t s);

/* Launchers; each returns the hipError_t of its launch. */
hipError_t launch_quantize_q8(const float *x, uint32_t rows, uint32_t n, float *d, int8_t *q, int *flag,
                              hipStream_t s);
hipError_t launch_matmul(const MatArgs &a, bool q5, bool fast, hipStream_t s);
/* Int8-MFMA prefill GEMM (relaxed block order). sums != NULL writes the exact
 * per-block int32 sums, sums[(t*rows + r)*nb + b], instead of the outputs.
 * ws (ws_bytes of device workspace, may be NULL) holds the partial tiles when
 * K is split over slices (few tiles); launches that overlap in time must not
 * share it. mfma_layout_ok: 4-byte aligned rows and activations, even nb for Q5. */
bool mfma_layout_ok(const MatArgs &a, bool q5);
hipError_t launch_matmul_mfma(const MatArgs &a, bool q5, int32_t *sums, float *ws, size_t ws_bytes, hipStream_t s);
/* Q8 prefill GEMM on int8 MFMA with 64 x 64 tiles and K split over slices when the tiles are few
 * (csrc/smq_mfma.hip); ws: MQ_WORKSPACE_BYTES of device workspace for the slices' partial sums.
 * mq8_ok: 4-byte aligned rows and activations, ntok >= 2. */
constexpr size_t MQ_WORKSPACE_BYTES = (size_t)16 << 20;
bool mq8_ok(const MatArgs &a);
/* mq8_ok and few enough tiles (with a K long enough) that splitting K pays: the shapes
 * launch_mq8 serves (the others take launch_matmul_mfma). */
bool mq8_wanted(const MatArgs &a);
hipError_t launch_mq8(MatArgs a, float *ws, size_t ws_bytes, hipStream_t s);
hipError_t prepare_mq8_attributes();
/* The f16-MFMA prefill GEMM with the activation in registers (csrc/smq_mfma.hip): Q8 rows of 28
 * blocks, at least two tokens, 8-byte aligned quants, 16-byte aligned activation scale rows. Same results as the int8 kernels bit for
 * bit. set_mh_enabled(false) (SMQ_MFMA_MH=0 at init) sends those shapes back to the int8 kernels. */
bool mh_wanted(const MatArgs &a);
hipError_t launch_mh(MatArgs a, hipStream_t s);
void set_mh_enabled(bool on);
bool mh_enabled();
/* Activation producer rows (model.c:354-415): optional RMSNorm, optional
 * gated activation (act 1 = SwiGLU, 2 = GeGLU), optional f32 store, Q8. */
constexpr uint32_t MAX_ROW = 16384;
hipError_t launch_row_quantize(const float *src, const float *norm, float eps, const float *gate, int act,
                               uint32_t rows, uint32_t n, float *y, float *d, int8_t *q, int *flag, hipStream_t s);
/* Decoder pieces (model.c:425-542, 673-676; sampler.c:57-63). pos_dev, when
 * not NULL, supplies the first position from device memory (graph replay).
 * RoPE tables hold `pairs` floats per absolute position; caches hold kv_dim
 * floats per position, `context` positions. */
constexpr uint32_t MAX_HEAD_DIM = 256;
constexpr uint32_t MAX_ATT_POSITIONS = 16384; /* one f32 score per position in LDS */
struct AttnShape {
    uint32_t heads, kv_heads, head_dim, q_dim, kv_dim, pairs, window, context;
};
hipError_t launch_rope_kv(float *q, float *k, const float *v, uint32_t ntok, const AttnShape &sh, const float *cs,
                          const float *sn, float *kcache, float *vcache, uint32_t pos0, const int32_t *pos_dev,
                          int *flag, hipStream_t s);
hipError_t launch_attention(const float *q, const float *kcache, const float *vcache, float *att, uint32_t ntok,
                            const AttnShape &sh, uint32_t pos0, const int32_t *pos_dev, int *flag, float *xd,
                            int8_t *xq, hipStream_t s,
                            float *scores = nullptr);
/* One decoding token: RoPE of q and k, the cache store of k and v, and
 * attention (+ Q8 of the row) in one launch; q/k/v are the unrotated QKV
 * outputs. Needs attention_rows_ok (head_dim 64, 16-byte aligned q and
 * caches) and 16-byte aligned k, v. */
bool attention_rows_ok(const AttnShape &sh, const void *q, const void *kcache, const void *vcache);
/* scores: SCORE_WORKSPACE_BYTES of device workspace (heads x context f32) for
 * the two-launch form; NULL (or a shape past it) takes the one-launch form. */
constexpr size_t SCORE_WORKSPACE_BYTES = (size_t)4 << 22;
hipError_t launch_attention_rope(const float *q, const float *k, const float *v, const float *cs, const float *sn,
                                 float *kcache, float *vcache, float *att, const AttnShape &sh, uint32_t pos0,
                                 const int32_t *pos_dev, int *flag, float *xd, int8_t *xq, float *scores,
                                 hipStream_t s);
hipError_t launch_decode_advance(int32_t *pos, uint32_t *count, const uint32_t *token, uint32_t *history,
                                 uint32_t capacity, hipStream_t s);
/* Greedy argmax in two launches through `parts` (ARGMAX_PART_BYTES *
 * MAX_ARGMAX_PARTS bytes of device workspace); with count != NULL also the
 * bookkeeping of one decode step (as launch_decode_advance); with embed also
 * the chosen token's embedding row into embed->out (as launch_embed). */
constexpr uint32_t MAX_ARGMAX_PARTS = 1024;
constexpr uint32_t ARGMAX_PART_BYTES = 12;
struct EmbedArgs {
    const unsigned char *w;
    size_t row_bytes;
    uint32_t vocab, cols;
    bool q5;
    float *out;
    int *flag;
};
hipError_t launch_argmax(const float *logits, uint32_t n, const unsigned char *banned, uint32_t *out, void *parts,
                         int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity, hipStream_t s,
                         const EmbedArgs *embed = nullptr);
/* The allocation-free argmax's partials: a static device array of
 * MAX_ARGMAX_PARTS partials. bind_noalloc_scratch (with `device` current)
 * records its device address; noalloc_scratch returns it (NULL if unbound).
 * With one span of AM_SPAN ids per partial it serves vocabularies up to
 * NOALLOC_MAX_VOCAB ids. */
constexpr uint32_t NOALLOC_MAX_VOCAB = MAX_ARGMAX_PARTS * 1024u;
hipError_t bind_noalloc_scratch(int device);

/* Raise the dynamic-LDS limits of the attention and fused-GEMV kernels once,
 * at smq_init (no kernel attribute changes later, inside or after a capture). */
hipError_t prepare_attention_attributes();
hipError_t prepare_fused_attributes();
void *noalloc_scratch(int device);
hipError_t launch_embed(const unsigned char *w, size_t row_bytes, bool q5, uint32_t vocab, const uint32_t *tokens,
                        uint32_t ntok, uint32_t cols, float *out, int *flag, hipStream_t s);
/* Q5 conversion (kernels.c:1064-1117): rows of cols floats to rows of
 * ceil(cols/32) 22-byte blocks, row r at out + r*nb*22. */
hipError_t launch_quantize_q5(const float *x, uint32_t rows, uint32_t cols, unsigned char *out, hipStream_t s);
hipError_t launch_dequantize_row(const unsigned char *w, uint32_t cols, float *out, bool q5, hipStream_t s);

/* Grid barrier probe (csrc/smq_anchor.hip): clears `words` (GRID_BARRIER_WORDS of them), then one launch
 * of wgs workgroups (one per CU, wgs <= the CU count) passing `episodes` barriers of the given kind;
 * words[GRID_BARRIER_TIMEOUTS] counts the workgroups that gave up a wait. */
constexpr uint32_t GRID_BARRIER_WORDS = 10 * 64;
constexpr uint32_t GRID_BARRIER_TIMEOUTS = 9 * 64 + 16;
hipError_t launch_grid_barrier(uint32_t *words, uint32_t wgs, uint32_t episodes, uint32_t kind, hipStream_t s);

/* HBM bandwidth anchors (csrc/smq_anchor.hip): bytes / 16 pieces of 16 bytes over wgs x threads. */
hipError_t launch_stream_read(const void *p, size_t bytes, uint32_t wgs, uint32_t threads, bool nt, uint32_t *sink,
                              hipStream_t s);
hipError_t launch_stream_copy(void *dst, const void *src, size_t bytes, uint32_t wgs, uint32_t threads, bool nt,
                              hipStream_t s);

}  // namespace smq

#endif
