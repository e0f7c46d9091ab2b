/* smq_model.h - C host forward pass on the gfx950 path.
 *
 * The reference's model layer (src/config.c, src/modelfile.c, src/model.c,
 * src/sampler.c:57-63) rebuilt over the C ABI of smq.h: a SMOEQ8 checkpoint
 * is parsed and validated on the host exactly as the reference does, its
 * tensors are uploaded once to device memory, and every step of the forward
 * pass (embedding, RMSNorm+quantize, QKV/O/FFN/LM-head matmuls with bias and
 * fused residual add, RoPE, KV cache, attention, SwiGLU+quantize, greedy
 * choice) runs on the GPU with activations device-resident. Logits are bit
 * identical to the reference's model_forward with the f32 KV cache.
 *
 * Greedy decoding replays one captured HIP graph per token: the graph reads
 * the token and position from device memory and advances them itself, so a
 * run of decode steps needs no host round trip.
 *
 * Supported: architectures smolmoe_v1 and smolmoe_qwen2 with one expert and
 * no shared experts (every dense Llama/Qwen2 checkpoint the reference
 * converts), Q8 or Q5 matrices, partial rotary, RoPE attention factor,
 * Llama 3 RoPE scaling, sliding window. Refused with SMQ_ERR_FORMAT: routed
 * MoE layers (experts > 1), shared experts, smolmoe_gemma3, and (at the API)
 * the f16 KV cache. Every call returns an smq_status with the message in
 * smq_last_error (smq.h).
 */
#ifndef SMQ_MODEL_H
#define SMQ_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "smq.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SMQ_BOS_ID 256u /* config.h:11 */
#define SMQ_EOS_ID 257u /* config.h:12 */

/* Config (src/config.h:13-28): the key=value architecture description. */
typedef struct smq_config {
    uint32_t dim, hidden, layers, heads, kv_heads, experts, top_k, vocab;
    uint32_t max_context, shared, bos, eos, qkv_bias, gemma3;
    uint32_t head_dim, rotary_dim, sliding_window;
    float eps, theta, local_theta;
    double rope_factor;
    uint32_t llama3_rope, llama3_original;
    double llama3_factor, llama3_low, llama3_high;
} smq_config;

/* config_parse / config_read (src/config.c:56-161): same keys, defaults,
 * limits and SMQ_ERR_FORMAT messages. */
smq_status smq_config_parse(const unsigned char *text, size_t size, smq_config *out);
smq_status smq_config_read(const char *path, smq_config *out);

/* Tensor / ModelFile (src/modelfile.h:21-33). data points into the caller's
 * bytes (host memory). */
#define SMQ_TENSOR_NAME_SIZE 40u
#define SMQ_DTYPE_F32 0u
#define SMQ_DTYPE_Q8 1u
#define SMQ_DTYPE_Q5 2u
#define SMQ_DTYPE_BLOB 3u
#define SMQ_DTYPE_QUANTIZED 0xffffffffu
typedef struct smq_tensor {
    char name[SMQ_TENSOR_NAME_SIZE];
    uint32_t rows, cols, dtype, alias;
    uint64_t offset, bytes;
    const unsigned char *data;
} smq_tensor;
typedef struct smq_modelfile {
    const unsigned char *base;
    uint64_t size;
    uint32_t version, count, blobs;
    smq_tensor *tensors; /* malloc'd; smq_modelfile_release frees it */
} smq_modelfile;

/* modelfile_parse (src/modelfile.c:47-100): header, sorted directory,
 * extents and the one permitted alias (lm_head = embed, version >= 2). */
smq_status smq_modelfile_parse(smq_modelfile *mf, const unsigned char *data, uint64_t size);
/* modelfile_verify_payload (src/modelfile.c:142-201): every Q8 scale finite
 * and >= 0, every Q5 scale finite, every F32 value finite. */
smq_status smq_modelfile_verify_payload(const smq_modelfile *mf);
/* modelfile_find / modelfile_blob (src/modelfile.c:109-140). */
const smq_tensor *smq_modelfile_find(const smq_modelfile *mf, const char *name, uint32_t rows, uint32_t cols,
                                     uint32_t dtype);
const smq_tensor *smq_modelfile_blob(const smq_modelfile *mf, const char *name);
void smq_modelfile_release(smq_modelfile *mf);

typedef struct smq_model smq_model;

/* Logit modes (src/model.h:39). */
#define SMQ_LOGITS_NONE 0
#define SMQ_LOGITS_LAST 1
#define SMQ_LOGITS_ALL 2

/* Opens `path` (mapped read-only), takes the configuration from config_path,
 * or else from the embedded "__config__" blob (main.c:494-513), parses and
 * verifies the container, checks the tensor set against the configuration
 * (model.c:109-131), uploads every tensor to the GPU once and allocates the
 * device activations for `batch` tokens, `logit_rows` logit rows and a KV
 * cache of `context` positions (model.c:132-188). smq_init must have been
 * called. NULL on failure (reason in smq_last_error). */
smq_model *smq_model_open(const char *path, const char *config_path, uint32_t context, uint32_t batch,
                          uint32_t logit_rows);
/* The same from checkpoint bytes already in host memory (not kept). */
smq_model *smq_model_open_bytes(const unsigned char *data, uint64_t size, const smq_config *config,
                                uint32_t context, uint32_t batch, uint32_t logit_rows);
void smq_model_close(smq_model *m);
const smq_config *smq_model_config(const smq_model *m);
/* Device bytes held by weights, activations and the KV cache. */
size_t smq_model_device_bytes(const smq_model *m);

/* model_forward (model.c:660-724): tokens[0..n) (host) at positions
 * pos0..pos0+n-1; LOGITS_LAST leaves the last token's logits in row 0,
 * LOGITS_ALL n rows. Synchronizes; SMQ_ERR_NUMERIC on a non-finite
 * activation, SMQ_ERR_RANGE on an id outside the vocabulary or a batch
 * past the context. A batch (n > 1) drops the captured decode step, so no
 * decode graph is replayed after launches made since its capture; the next
 * smq_model_generate (or smq_model_prepare_decode) captures it again. */
smq_status smq_model_forward(smq_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int mode);
/* model_prefill (model.c:703-714): n tokens in batch-sized chunks. */
smq_status smq_model_prefill(smq_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int last_logits);
/* Copies `rows` logit rows (vocab floats each) to host memory. */
smq_status smq_model_logits(const smq_model *m, float *out, uint32_t rows);
/* Device pointer to the logits (row-major, vocab floats per row). */
const float *smq_model_logits_device(const smq_model *m);
/* model_kv_layer (model.h:96-98): device pointer to position 0 of one
 * layer's keys (values = 0) or values (values = 1), kv_dim f32 per position. */
const float *smq_model_kv_layer(const smq_model *m, uint32_t layer, int values);

/* Ids the greedy choice skips (sampler.c:57-63): vocab bytes (host), nonzero
 * = banned; NULL bans nothing (the default). */
smq_status smq_model_set_banned(smq_model *m, const unsigned char *banned);
/* Greedy generation as main.c:571-600 runs it with temperature 0: out[0] =
 * argmax of logits row 0 (left by a LOGITS_LAST forward of the prompt), then
 * for i = 1..ntokens-1 one decode forward of out[i-1] at position pos+i-1
 * and out[i] = its argmax. Decode steps replay a captured graph; the host
 * waits once at the end. It does not stop at EOS: a caller stops where the
 * reference would (the tokens up to EOS are the same). */
smq_status smq_model_generate(smq_model *m, uint32_t pos, uint32_t ntokens, uint32_t *out);
/* No reference counterpart: captures the decode step now if none is held
 * (smq_model_generate otherwise does it on its first call after a batch
 * forward), so a timed generate holds replays only. Synchronizes. */
smq_status smq_model_prepare_decode(smq_model *m);

/* No reference counterpart (the reference's fixtures are built the same way by
 * tests/support/fixture.ts and its Q8 writer tools/q8pack.c:38-44): writes a
 * synthetic one-expert checkpoint for config_text (SMOEQ8 v3, the config
 * embedded): matrices N(0, sigma) packed to Q8, norm weights 1, Qwen2
 * biases N(0, sigma), seeded per tensor name; tied stores lm_head as an
 * alias of embed. Host only (no GPU); `threads` worker threads. */
smq_status smq_synth_checkpoint(const char *path, const char *config_text, uint64_t seed, float sigma, int tied,
                                uint32_t threads);

#ifdef __cplusplus
}
#endif

#endif
