/* Driver over the reference's own model layer (test infrastructure only).
 *
 * Compiled by oracle/Makefile together with the reference's unmodified
 * sources (model.c, kernels*.c, vecmath.c, threadpool.c, util.c, modelfile.c,
 * config.c, platform.c, sampler.c) into oracle/_ref/libsmref_model.so. It
 * opens a checkpoint the way src/main.c:494-513, 798-808 does and exposes
 * model_forward, the logits, the KV cache and main.c:571-600's greedy loop
 * (temperature 0) to the tests, which compare them with the restated forward
 * (smq_forward.c) and the GPU path. */
#include "config.h"
#include "kernels.h"
#include "model.h"
#include "modelfile.h"
#include "platform.h"
#include "sampler.h"
#include "threadpool.h"
#include "util.h"

#include <stdlib.h>
#include <string.h>

typedef struct RefModel {
    MappedFile file;
    ModelFile mf;
    Config c;
    Memory mem;
    Pool *pool;
    Model model;
    unsigned char *banned;
    Sampler sampler;
} RefModel;

const char *ref_last_error(void) { return sm_last_error(); }
const char *ref_backend(int scalar, int fast) {
    kernels_set_fast(fast);
    return kernels_select(scalar);
}

/* kernels_select (kernels.c:721-800) on a host with AVX2+F16C but no AVX-VNNI
 * or AVX512-VNNI: the same selection, then the integer dot kernels set to the
 * AVX2 ones that kernels.c:796-806 picks there (exact contract). Returns
 * "avx2", or NULL when this CPU has no AVX2+F16C. */
const char *ref_backend_avx2(void) {
#if defined(SM_HAVE_AVX2)
    const char *picked;
    kernels_set_fast(0);
    picked = kernels_select(0);
    if (!strncmp(picked, "scalar", 6)) return NULL;
    dot_q8 = dot_q8_avx2;
    dot_q8_x4 = dot_q8_avx2_x4;
    dot_q8_r4 = dot_q8_avx2_r4;
    dot_q5 = dot_q5_avx2;
    dot_q5_x4 = dot_q5_avx2_x4;
    dot_q5_r4 = dot_q5_avx2_r4;
    gemm_q8 = gemm_q8_avx2;
    gemm_q5 = gemm_q5_avx2;
    return "avx2";
#else
    return NULL;
#endif
}

void ref_model_close(RefModel *r) {
    if (!r) return;
    if (r->pool) pool_destroy(r->pool);
    if (r->file.data) unmap_file(&r->file);
    mem_release(&r->mem);
    free(r);
}

/* config_path NULL: the embedded "__config__" blob. */
RefModel *ref_model_open(const char *path, const char *config_path, uint32_t context, uint32_t batch,
                         uint32_t logit_rows, uint32_t threads) {
    char err[512];
    const Tensor *blob;
    RefModel *r = (RefModel *)calloc(1, sizeof(RefModel));
    if (!r) return NULL;
    r->mem.limit = (size_t)-1;
    if (!try_map_file(path, &r->file, err, sizeof(err))) {
        sm_set(SM_ERR_IO, "%s", err);
        free(r);
        return NULL;
    }
    if (modelfile_parse(&r->mf, r->file.data, r->file.size, &r->mem) != SM_OK) goto fail;
    if (config_path) {
        if (config_read(config_path, &r->c) != SM_OK) goto fail;
    } else {
        blob = modelfile_blob(&r->mf, BLOB_CONFIG);
        if (!blob) {
            sm_set(SM_ERR_FORMAT, "no embedded config");
            goto fail;
        }
        if (config_parse(blob->data, (size_t)blob->bytes, &r->c) != SM_OK) goto fail;
    }
    r->pool = pool_create(threads ? threads : 1, &r->mem);
    if (!r->pool) goto fail;
    if (modelfile_verify_payload(&r->mf, r->pool) != SM_OK) goto fail;
    if (model_init(&r->model, &r->c, &r->mf, context, batch < context ? batch : context, logit_rows, r->pool, &r->mem,
                   0) != SM_OK)
        goto fail;
    r->banned = (unsigned char *)mem_alloc(&r->mem, r->c.vocab, 1);
    if (!r->banned) goto fail;
    if (sampler_init(&r->sampler, r->c.vocab, r->banned, 0.0f, 0, 1.0f, 1, &r->mem) != SM_OK) goto fail;
    return r;
fail:
    ref_model_close(r);
    return NULL;
}

int ref_model_forward(RefModel *r, const uint32_t *tokens, uint32_t n, uint32_t pos0, int mode) {
    return (int)model_forward(&r->model, tokens, n, pos0, (LogitsMode)mode);
}

int ref_model_prefill(RefModel *r, const uint32_t *tokens, uint32_t n, uint32_t pos0, int last_logits) {
    return (int)model_prefill(&r->model, tokens, n, pos0, last_logits);
}

const float *ref_model_logits(RefModel *r) { return r->model.logits; }
const void *ref_model_kv(RefModel *r, uint32_t layer, int values) { return model_kv_layer(&r->model, layer, values); }
uint32_t ref_model_vocab(RefModel *r) { return r->c.vocab; }

/* banned: vocab bytes, or NULL for none. */
void ref_model_set_banned(RefModel *r, const unsigned char *banned) {
    if (banned) memcpy(r->banned, banned, r->c.vocab);
    else memset(r->banned, 0, r->c.vocab);
}

/* main.c:580-597 with temperature 0 and no EOS stop: out[0] from the current
 * logits, then one decode forward per further token. */
int ref_model_generate(RefModel *r, uint32_t pos, uint32_t ntokens, uint32_t *out) {
    uint32_t i;
    for (i = 0; i < ntokens; ++i) {
        sm_status st = sampler_next(&r->sampler, r->model.logits, &out[i]);
        if (st != SM_OK) return (int)st;
        if (i + 1 < ntokens) {
            st = model_forward(&r->model, &out[i], 1, pos + i, LOGITS_LAST);
            if (st != SM_OK) return (int)st;
        }
    }
    return 0;
}

/* modelfile_parse, then modelfile_verify_payload on `threads` workers, as
 * ref_model_open runs them (src/main.c:494-513), over a checkpoint already in
 * memory. Returns the status; the message is ref_last_error's. */
int ref_modelfile_check(const unsigned char *data, uint64_t size, uint32_t threads) {
    Memory mem;
    ModelFile mf;
    Pool *pool;
    sm_status st;
    memset(&mem, 0, sizeof(mem));
    mem.limit = (size_t)-1;
    st = modelfile_parse(&mf, data, size, &mem);
    if (st == SM_OK) {
        pool = pool_create(threads ? threads : 1, &mem);
        if (!pool) {
            st = sm_last_status();
        } else {
            st = modelfile_verify_payload(&mf, pool);
            pool_destroy(pool);
        }
    }
    mem_release(&mem);
    return (int)st;
}
