/* CPU oracle of the dense decoder forward (test infrastructure only). */
#ifndef SMQ_FORWARD_H
#define SMQ_FORWARD_H

#include "smq_oracle.h"

/* One layer's tensors as they sit in the checkpoint (host memory). dtype
 * 1 = Q8, 2 = Q5; biases may be NULL (smolmoe_v1). */
typedef struct OrcLayer {
    const float *attn_norm, *ffn_norm, *q_bias, *k_bias, *v_bias;
    const unsigned char *q, *k, *v, *o, *gate, *up, *down;
    uint32_t q_dtype, k_dtype, v_dtype, o_dtype, gate_dtype, up_dtype, down_dtype;
} OrcLayer;

typedef struct OrcModel {
    uint32_t dim, hidden, layers, heads, kv_heads, head_dim, vocab, rotary_dim, window, context;
    uint32_t llama3_rope, llama3_original;
    float eps, theta, local_theta;
    double rope_factor, llama3_factor, llama3_low, llama3_high;
    const unsigned char *embed, *head;
    uint32_t embed_dtype, head_dtype;
    const float *final_norm;
    const OrcLayer *layer;
    float *keys, *values; /* caller-owned [layers][context][kv_heads*head_dim] */
} OrcModel;

/* model_forward (src/model.c:660-686): tokens at pos0..pos0+n-1; mode 0 no
 * logits, 1 the last token's row, 2 every row. Returns 1, 0 if the
 * reference would fail with SM_ERR_NUMERIC, -1 on allocation failure. */
int orc_forward(const OrcModel *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int mode, float *logits);

#endif
