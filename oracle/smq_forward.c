/* CPU oracle of the dense decoder forward pass (test infrastructure only:
 * imported by tests/ and bench.py's CPU baseline, never by the product).
 *
 * Restates src/model.c:425-686 for one-expert checkpoints with the f32 KV
 * cache, composed from the restated pieces in smq_oracle.c:
 *   embedding rows            model.c:669-677   orc_dequantize_row
 *   RoPE tables (double)      model.c:425-437   inline below
 *   RMSNorm -> Q8             model.c:393-400   orc_row_work
 *   Q/K/V (+bias), O, FFN     model.c:252-310   orc_mat_item
 *   RoPE, KV store            model.c:511-526   orc_rope + copies
 *   attention                 model.c:459-491   orc_attend_f32
 *   attention-out quantize    model.c:402-406   orc_quantize_q8
 *   residual adds             model.c:452-455   x = x + out
 *   SwiGLU -> Q8              model.c:409-415   orc_row_work
 *   final norm + LM head      model.c:650-658
 * Pinned against the reference's own model_forward (oracle/_ref) on
 * synthetic checkpoints: logits, KV caches and greedy tokens bit-identical.
 */
#include "smq_forward.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static size_t row_bytes_of(uint32_t dtype, uint32_t cols) {
    return (size_t)((cols + 31u) / 32u) * (dtype == 2 ? ORC_Q5_BLOCK : ORC_Q8_BLOCK);
}

static int matmul(const unsigned char *w, uint32_t dtype, uint32_t rows, uint32_t cols, const float *bias,
                  const float *xd, const int8_t *xq, uint32_t ntok, float *y) {
    return orc_mat_item(dtype == 2, 0, w, row_bytes_of(dtype, cols), rows, bias, xd, xq, ntok, (cols + 31u) / 32u,
                        y);
}

/* model.c:95-107 */
static double llama3_scale(const OrcModel *m, double freq) {
    double wavelen, smooth;
    if (!m->llama3_rope) return freq;
    wavelen = 2.0 * 3.14159265358979323846 / freq;
    if (wavelen < (double)m->llama3_original / m->llama3_high) return freq;
    if (wavelen > (double)m->llama3_original / m->llama3_low) return freq / m->llama3_factor;
    smooth = ((double)m->llama3_original / wavelen - m->llama3_low) / (m->llama3_high - m->llama3_low);
    return (1.0 - smooth) * freq / m->llama3_factor + smooth * freq;
}

int orc_forward(const OrcModel *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int mode, float *logits) {
    const uint32_t dim = m->dim, hd = m->head_dim, qd = m->heads * hd, kd = m->kv_heads * hd, H = m->hidden;
    const uint32_t half = m->rotary_dim / 2, nbd = (dim + 31) / 32, nbq = (qd + 31) / 32, nbh = (H + 31) / 32;
    const uint32_t nbmax = nbd > nbq ? nbd : nbq;
    float *x = calloc((size_t)n * dim, 4), *xn = calloc((size_t)n * (dim > qd ? dim : qd), 4);
    float *q = calloc((size_t)n * qd, 4), *k = calloc((size_t)n * kd, 4), *v = calloc((size_t)n * kd, 4);
    float *att = calloc((size_t)n * qd, 4), *out = calloc((size_t)n * dim, 4);
    float *gate = calloc((size_t)n * H, 4), *up = calloc((size_t)n * H, 4);
    float *xd = calloc((size_t)n * nbmax, 4), *hdv = calloc((size_t)n * nbh, 4);
    int8_t *xq = calloc((size_t)n * nbmax * 32, 1), *hq = calloc((size_t)n * nbh * 32, 1);
    float *scores = calloc((size_t)m->context + 1, 4);
    float *cs = calloc((size_t)n * (half ? half : 1), 4), *sn = calloc((size_t)n * (half ? half : 1), 4);
    double *inv_freq = calloc(half ? half : 1, sizeof(double));
    uint32_t t, l, i, h;
    size_t j;
    int ok = 1;
    if (!x || !xn || !q || !k || !v || !att || !out || !gate || !up || !xd || !hdv || !xq || !hq || !scores || !cs ||
        !sn || !inv_freq) {
        ok = -1;
        goto done;
    }
    for (t = 0; t < n; ++t)
        orc_dequantize_row(m->embed_dtype == 2, m->embed + (size_t)tokens[t] * row_bytes_of(m->embed_dtype, dim),
                           dim, x + (size_t)t * dim);
    /* A sliding window makes every layer of a non-Gemma model local
     * (model.c:463-466): local layers use the rope_local_theta tables, which
     * carry no Llama 3 scaling (model.c:166-169, 502-504). */
    for (i = 0; i < half; ++i)
        inv_freq[i] = m->window ? pow((double)m->local_theta, -(double)(2 * i) / (double)m->rotary_dim)
                                : llama3_scale(m, pow((double)m->theta, -(double)(2 * i) / (double)m->rotary_dim));
    for (t = 0; t < n; ++t)
        for (i = 0; i < half; ++i) {
            double angle = (double)(pos0 + t) * inv_freq[i];
            cs[t * half + i] = (float)(m->rope_factor * cos(angle));
            sn[t * half + i] = (float)(m->rope_factor * sin(angle));
        }
    for (l = 0; l < m->layers; ++l) {
        const OrcLayer *L = &m->layer[l];
        float *keys = m->keys + (size_t)l * m->context * kd, *values = m->values + (size_t)l * m->context * kd;
        ok &= orc_row_work(x, L->attn_norm, m->eps, NULL, 0, n, dim, xn, xd, xq);
        ok &= matmul(L->q, L->q_dtype, qd, dim, L->q_bias, xd, xq, n, q);
        ok &= matmul(L->k, L->k_dtype, kd, dim, L->k_bias, xd, xq, n, k);
        ok &= matmul(L->v, L->v_dtype, kd, dim, L->v_bias, xd, xq, n, v);
        for (t = 0; t < n; ++t) {
            orc_rope(q + (size_t)t * qd, m->heads, hd, half, cs + t * half, sn + t * half);
            orc_rope(k + (size_t)t * kd, m->kv_heads, hd, half, cs + t * half, sn + t * half);
            memcpy(keys + (size_t)(pos0 + t) * kd, k + (size_t)t * kd, (size_t)kd * 4);
            memcpy(values + (size_t)(pos0 + t) * kd, v + (size_t)t * kd, (size_t)kd * 4);
        }
        for (t = 0; t < n; ++t)
            for (h = 0; h < m->heads; ++h) {
                const uint32_t pos = pos0 + t, kh = h / (m->heads / m->kv_heads);
                const uint32_t start = m->window && pos >= m->window ? pos - m->window + 1 : 0;
                orc_attend_f32(q + (size_t)t * qd + (size_t)h * hd, keys + (size_t)kh * hd, values + (size_t)kh * hd,
                               kd, hd, start, pos, scores, att + (size_t)t * qd + (size_t)h * hd);
            }
        for (t = 0; t < n; ++t)
            ok &= orc_quantize_q8(att + (size_t)t * qd, qd, xd + (size_t)t * nbq, xq + (size_t)t * nbq * 32) == 0;
        ok &= matmul(L->o, L->o_dtype, dim, qd, NULL, xd, xq, n, out);
        for (j = 0; j < (size_t)n * dim; ++j) x[j] = x[j] + out[j];
        ok &= orc_row_work(x, L->ffn_norm, m->eps, NULL, 0, n, dim, xn, xd, xq);
        ok &= matmul(L->gate, L->gate_dtype, H, dim, NULL, xd, xq, n, gate);
        ok &= matmul(L->up, L->up_dtype, H, dim, NULL, xd, xq, n, up);
        ok &= orc_row_work(up, NULL, 0.0f, gate, 0, n, H, up, hdv, hq);
        ok &= matmul(L->down, L->down_dtype, dim, H, NULL, hdv, hq, n, out);
        for (j = 0; j < (size_t)n * dim; ++j) x[j] = x[j] + out[j];
    }
    if (mode) {
        const uint32_t first = mode == 2 ? 0 : n - 1, rows = n - first;
        ok &= orc_row_work(x + (size_t)first * dim, m->final_norm, m->eps, NULL, 0, rows, dim, xn, xd, xq);
        ok &= matmul(m->head, m->head_dtype, m->vocab, dim, NULL, xd, xq, rows, logits);
    }
done:
    free(x); free(xn); free(q); free(k); free(v); free(att); free(out); free(gate); free(up);
    free(xd); free(hdv); free(xq); free(hq); free(scores); free(cs); free(sn); free(inv_freq);
    return ok;
}
