/* Host forward pass over the gfx950 C ABI (include/smq_model.h).
 *
 * Mirrors the reference's model layer: config.c (key=value parsing),
 * modelfile.c (SMOEQ8 container), model.c (weights, buffers, forward) and
 * sampler.c:57-63 (greedy choice). All arithmetic runs in libsmq_gfx950.so;
 * this file validates inputs, lays out device memory and enqueues launches.
 *
 * Device layout (one process, one GPU):
 *   weights  one arena; each Q8/Q5 matrix at a 256-byte aligned offset, rows
 *            packed at the checkpoint's row_bytes (tied lm_head shares embed)
 *   vectors  one f32 arena for norms and biases
 *   acts     x, q, k, v, att, gate, up (batch rows each), the quantized
 *            activations xd/xq (dim or q_dim wide) and hd/hq (hidden wide)
 *   kv       keys and values, [layers][context][kv_dim] f32 each
 *   rope     cos and sin tables, [context][rotary_dim/2] f32, computed once in
 *            double on the host exactly as model.c:425-437 does per call
 *   decode   token, position, step counter and token history in device
 *            memory, advanced by the captured decode step itself
 */
#define _POSIX_C_SOURCE 200809L

#include "smq_model.h"

#include <errno.h>
#include <fcntl.h>
#include <float.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define QK 32u
#define Q8_BLOCK 36u
#define Q5_BLOCK 22u
#define MAX_CONTEXT 1048576u /* config.h:6 */
#define MAX_DIM 65536u       /* config.h:7 */
#define MAX_MERGES 262144u   /* config.h:8 */

/* ---- status ----------------------------------------------------------- */

static smq_status fail(smq_status st, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return smq_set_error(st, buf);
}

static int finite_f(double v) { return v == v && v <= DBL_MAX && v >= -DBL_MAX; }

static uint32_t rd_u32(const unsigned char *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t rd_u64(const unsigned char *p) { return (uint64_t)rd_u32(p) | (uint64_t)rd_u32(p + 4) << 32; }
static float rd_f32(const unsigned char *p) {
    uint32_t u = rd_u32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* f16 bits -> f32, exact (f16.h:10-27 semantics, written from the format). */
static float f16_value(uint16_t h) {
    const int sign = h >> 15, exp = (h >> 10) & 31, man = h & 1023;
    double v;
    if (exp == 31) return man ? NAN : (sign ? -INFINITY : INFINITY);
    v = exp ? ldexp(1024 + man, exp - 25) : ldexp(man, -24);
    return (float)(sign ? -v : v);
}

/* ---- config (config.c) -------------------------------------------------- */

enum {
    K_ARCH, K_DIM, K_HIDDEN, K_LAYERS, K_HEADS, K_KV_HEADS, K_EXPERTS, K_TOP_K, K_VOCAB, K_MAX_CONTEXT, K_SHARED,
    K_BOS, K_EOS, K_EPS, K_THETA, /* the 15 required keys */
    K_ROTARY_DIM, K_ROPE_FACTOR, K_HEAD_DIM, K_SLIDING_WINDOW, K_LOCAL_THETA, K_L3_FACTOR, K_L3_LOW, K_L3_HIGH,
    K_L3_ORIGINAL, K_COUNT
};
static const char *const CONFIG_KEYS[K_COUNT] = {
    "architecture", "dim", "hidden_dim", "layers", "heads", "kv_heads", "experts", "top_k", "vocab_size",
    "max_context", "shared_experts", "bos_id", "eos_id", "rms_eps", "rope_theta", "rotary_dim",
    "rope_attention_factor", "head_dim", "sliding_window", "rope_local_theta", "rope_llama3_factor",
    "rope_llama3_low_freq_factor", "rope_llama3_high_freq_factor", "rope_llama3_original_context"};
#define REQUIRED_MASK ((1u << 15) - 1u)
#define LLAMA3_MASK (0xfu << K_L3_FACTOR)

static char *trim_ws(char *s) {
    char *end;
    while (*s == ' ' || *s == '\t' || *s == '\r' || *s == '\n') ++s;
    end = s + strlen(s);
    while (end > s && (end[-1] == ' ' || end[-1] == '\t' || end[-1] == '\r' || end[-1] == '\n')) --end;
    *end = 0;
    return s;
}

/* util.c:161-187: decimal u32 <= max, no sign; finite real. 0 on error. */
static int parse_u32v(const char *s, uint32_t max, const char *what, uint32_t *out) {
    char *end;
    unsigned long long n;
    if (!*s || *s == '-' || *s == '+') return fail(SMQ_ERR_FORMAT, "invalid %s: %s", what, s), 0;
    errno = 0;
    n = strtoull(s, &end, 10);
    if (errno || *end || n > max) return fail(SMQ_ERR_FORMAT, "invalid %s: %s", what, s), 0;
    *out = (uint32_t)n;
    return 1;
}
static int parse_realv(const char *s, const char *what, double *out) {
    char *end;
    double n;
    errno = 0;
    n = strtod(s, &end);
    if (!*s || errno || *end || !finite_f(n)) return fail(SMQ_ERR_FORMAT, "invalid %s: %s", what, s), 0;
    *out = n;
    return 1;
}

smq_status smq_config_parse(const unsigned char *text, size_t size, smq_config *out) {
    smq_config c;
    uint32_t *u32_keys[K_COUNT];
    unsigned seen = 0;
    size_t pos = 0;
    char line[512];
    memset(&c, 0, sizeof(c));
    memset(u32_keys, 0, sizeof(u32_keys));
    u32_keys[K_DIM] = &c.dim; u32_keys[K_HIDDEN] = &c.hidden; u32_keys[K_LAYERS] = &c.layers;
    u32_keys[K_HEADS] = &c.heads; u32_keys[K_KV_HEADS] = &c.kv_heads; u32_keys[K_EXPERTS] = &c.experts;
    u32_keys[K_TOP_K] = &c.top_k; u32_keys[K_VOCAB] = &c.vocab; u32_keys[K_MAX_CONTEXT] = &c.max_context;
    u32_keys[K_SHARED] = &c.shared; u32_keys[K_BOS] = &c.bos; u32_keys[K_EOS] = &c.eos;
    if (!out) return fail(SMQ_ERR_RANGE, "config: output is NULL");
    while (pos < size) {
        size_t n = 0;
        char *s, *eq, *value, *hash;
        unsigned k;
        double real;
        uint32_t u;
        /* one line with its newline (util.c:198-216) */
        while (pos < size) {
            char ch = (char)text[pos++];
            if (!ch) return fail(SMQ_ERR_FORMAT, "config contains a NUL byte");
            if (n + 1 >= sizeof(line)) return fail(SMQ_ERR_FORMAT, "config line too long");
            line[n++] = ch;
            if (ch == '\n') break;
        }
        line[n] = 0;
        hash = strchr(line, '#');
        if (hash) *hash = 0;
        s = trim_ws(line);
        if (!*s) continue;
        eq = strchr(s, '=');
        if (!eq) return fail(SMQ_ERR_FORMAT, "config requires key=value lines");
        *eq = 0;
        s = trim_ws(s);
        value = trim_ws(eq + 1);
        for (k = 0; k < K_COUNT && strcmp(s, CONFIG_KEYS[k]); ++k) {}
        if (k == K_COUNT) return fail(SMQ_ERR_FORMAT, "unknown config key: %s", s);
        if (seen & (1u << k)) return fail(SMQ_ERR_FORMAT, "duplicate config key: %s", s);
        seen |= 1u << k;
        if (k == K_ARCH) {
            if (!strcmp(value, "smolmoe_qwen2")) c.qkv_bias = 1;
            else if (!strcmp(value, "smolmoe_gemma3")) c.gemma3 = 1;
            else if (strcmp(value, "smolmoe_v1")) return fail(SMQ_ERR_FORMAT, "unsupported architecture: %s", value);
        } else if (u32_keys[k]) {
            if (!parse_u32v(value, MAX_CONTEXT, s, u32_keys[k])) return smq_last_status();
        } else if (k == K_EPS || k == K_THETA || k == K_LOCAL_THETA) {
            if (!parse_realv(value, s, &real)) return smq_last_status();
            if (k == K_EPS) c.eps = (float)real;
            else if (k == K_THETA) c.theta = (float)real;
            else c.local_theta = (float)real;
        } else if (k == K_ROPE_FACTOR || k == K_L3_FACTOR || k == K_L3_LOW || k == K_L3_HIGH) {
            if (!parse_realv(value, s, &real)) return smq_last_status();
            if (k == K_ROPE_FACTOR) c.rope_factor = real;
            else if (k == K_L3_FACTOR) c.llama3_factor = real;
            else if (k == K_L3_LOW) c.llama3_low = real;
            else c.llama3_high = real;
        } else if (k == K_ROTARY_DIM || k == K_HEAD_DIM) {
            if (!parse_u32v(value, MAX_DIM, s, &u)) return smq_last_status();
            if (k == K_ROTARY_DIM) c.rotary_dim = u;
            else c.head_dim = u;
        } else { /* sliding_window, rope_llama3_original_context */
            if (!parse_u32v(value, MAX_CONTEXT, s, &u)) return smq_last_status();
            if (k == K_SLIDING_WINDOW) c.sliding_window = u;
            else c.llama3_original = u;
        }
    }
    if ((seen & REQUIRED_MASK) != REQUIRED_MASK) return fail(SMQ_ERR_FORMAT, "config is missing required fields");
    if (!(seen & (1u << K_HEAD_DIM))) {
        if (!c.heads || c.heads > c.dim || c.dim % c.heads)
            return fail(SMQ_ERR_FORMAT, "invalid config dimensions or special token IDs");
        c.head_dim = c.dim / c.heads;
    }
    if (!c.dim || c.dim > MAX_DIM || !c.hidden || c.hidden > MAX_DIM || !c.layers || c.layers > 1024 || !c.heads ||
        c.heads > MAX_DIM || !c.head_dim || c.head_dim > MAX_DIM || c.head_dim % 2 ||
        (uint64_t)c.heads * c.head_dim > MAX_DIM || !c.kv_heads || c.heads % c.kv_heads || !c.experts ||
        c.experts > 4096 || !c.top_k || c.top_k > c.experts || c.shared > 16 || c.vocab < 258 ||
        c.vocab > 258 + MAX_MERGES || !c.max_context || c.max_context > MAX_CONTEXT || c.bos != SMQ_BOS_ID ||
        c.eos != SMQ_EOS_ID || !(c.eps > 0 && c.eps < 1) || !(c.theta > 1) || !finite_f(c.theta))
        return fail(SMQ_ERR_FORMAT, "invalid config dimensions or special token IDs");
    /* config.c:25-54: RoPE defaults and limits */
    if (!(seen & (1u << K_ROTARY_DIM))) c.rotary_dim = c.head_dim;
    if (!(seen & (1u << K_ROPE_FACTOR))) c.rope_factor = 1.0;
    if (!(seen & (1u << K_LOCAL_THETA))) c.local_theta = c.theta;
    if (!c.rotary_dim || c.rotary_dim % 2 || c.rotary_dim > c.head_dim)
        return fail(SMQ_ERR_FORMAT, "invalid rotary_dim %u: must be even and at most the head size %u", c.rotary_dim,
                    c.head_dim);
    if (!(c.rope_factor > 0 && c.rope_factor <= 1000.0))
        return fail(SMQ_ERR_FORMAT, "invalid rope_attention_factor: must be in (0, %g]", 1000.0);
    if ((seen & (1u << K_SLIDING_WINDOW)) && (!c.sliding_window || c.sliding_window > c.max_context))
        return fail(SMQ_ERR_FORMAT, "invalid sliding_window %u: must be in 1..%u", c.sliding_window, c.max_context);
    if (!(c.local_theta > 1) || !finite_f(c.local_theta))
        return fail(SMQ_ERR_FORMAT, "invalid rope_local_theta: must be finite and > 1");
    if ((seen & LLAMA3_MASK) && (seen & LLAMA3_MASK) != LLAMA3_MASK)
        return fail(SMQ_ERR_FORMAT, "llama3 RoPE scaling needs all of rope_llama3_factor, rope_llama3_low_freq_factor, "
                    "rope_llama3_high_freq_factor and rope_llama3_original_context");
    c.llama3_rope = (seen & LLAMA3_MASK) != 0;
    if (c.llama3_rope && (!(c.llama3_factor >= 1 && c.llama3_factor <= 1000.0) || !(c.llama3_low > 0) ||
                          !(c.llama3_high > c.llama3_low) || !finite_f(c.llama3_high) || !c.llama3_original))
        return fail(SMQ_ERR_FORMAT, "invalid llama3 RoPE scaling: needs factor in [1, %g], 0 < low_freq_factor < "
                    "high_freq_factor and original_context > 0", 1000.0);
    *out = c;
    smq_clear_error();
    return SMQ_OK;
}

typedef struct Mapping {
    unsigned char *data;
    uint64_t size;
} Mapping;

static smq_status map_file(const char *path, Mapping *m) {
    struct stat st;
    int fd;
    m->data = NULL;
    m->size = 0;
    if (!path) return fail(SMQ_ERR_IO, "path is NULL");
    fd = open(path, O_RDONLY);
    if (fd < 0) return fail(SMQ_ERR_IO, "%s: %s", path, strerror(errno));
    if (fstat(fd, &st) != 0) {
        int e = errno;
        close(fd);
        return fail(SMQ_ERR_IO, "%s: %s", path, strerror(e));
    }
    m->size = (uint64_t)st.st_size;
    if (m->size) {
        void *p = mmap(NULL, (size_t)m->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            int e = errno;
            close(fd);
            return fail(SMQ_ERR_IO, "%s: mmap: %s", path, strerror(e));
        }
        m->data = (unsigned char *)p;
    }
    close(fd);
    return SMQ_OK;
}

static void unmap(Mapping *m) {
    if (m->data) munmap(m->data, (size_t)m->size);
    m->data = NULL;
    m->size = 0;
}

smq_status smq_config_read(const char *path, smq_config *out) {
    Mapping f;
    smq_status st = map_file(path, &f);
    if (st != SMQ_OK) return st;
    st = smq_config_parse(f.data, (size_t)f.size, out);
    unmap(&f);
    return st;
}

/* ---- container (modelfile.c) -------------------------------------------- */

#define HEADER_BYTES 16u
#define RECORD_BYTES 72u
#define MAX_TENSORS 2000000u
#define MAX_TENSOR_COLS 65536u

static uint64_t block_size(uint32_t dtype) { return dtype == SMQ_DTYPE_Q8 ? Q8_BLOCK : Q5_BLOCK; }

static uint64_t payload_bytes(const smq_tensor *t) {
    if (t->dtype == SMQ_DTYPE_BLOB) return t->bytes;
    if (t->dtype != SMQ_DTYPE_F32) return (uint64_t)t->rows * ((t->cols + QK - 1) / QK) * block_size(t->dtype);
    return (uint64_t)t->rows * t->cols * 4;
}

void smq_modelfile_release(smq_modelfile *mf) {
    if (!mf) return;
    free(mf->tensors);
    memset(mf, 0, sizeof(*mf));
}

smq_status smq_modelfile_parse(smq_modelfile *mf, const unsigned char *data, uint64_t size) {
    uint64_t previous;
    uint32_t i;
    if (!mf) return fail(SMQ_ERR_RANGE, "modelfile is NULL");
    memset(mf, 0, sizeof(*mf));
    if (size < HEADER_BYTES || !data) return fail(SMQ_ERR_FORMAT, "invalid checkpoint size");
    mf->base = data;
    mf->size = size;
    mf->version = data[7];
    if (memcmp(data, "SMOEQ8\0", 7) || mf->version < 1 || mf->version > 3 || rd_u32(data + 12))
        return fail(SMQ_ERR_FORMAT, "unsupported checkpoint format (expected SMOEQ8 v1-v3)");
    mf->count = rd_u32(data + 8);
    if (!mf->count || mf->count > MAX_TENSORS) return fail(SMQ_ERR_FORMAT, "invalid tensor count");
    previous = HEADER_BYTES + (uint64_t)mf->count * RECORD_BYTES;
    if (previous > size) return fail(SMQ_ERR_FORMAT, "truncated checkpoint directory");
    mf->tensors = (smq_tensor *)calloc(mf->count, sizeof(smq_tensor));
    if (!mf->tensors) return fail(SMQ_ERR_NOMEM, "allocation of %u tensor records failed", mf->count);
    for (i = 0; i < mf->count; ++i) {
        const unsigned char *rec = data + HEADER_BYTES + (uint64_t)i * RECORD_BYTES;
        smq_tensor *t = &mf->tensors[i];
        memcpy(t->name, rec, SMQ_TENSOR_NAME_SIZE);
        if (!memchr(t->name, 0, SMQ_TENSOR_NAME_SIZE) || !t->name[0]) goto bad_name;
        t->rows = rd_u32(rec + 40);
        t->cols = rd_u32(rec + 44);
        t->dtype = rd_u32(rec + 48);
        t->alias = rd_u32(rec + 52);
        t->offset = rd_u64(rec + 56);
        t->bytes = rd_u64(rec + 64);
        if (t->dtype == SMQ_DTYPE_BLOB) { /* v3 embedded blobs, "__" names */
            if (mf->version < 3 || t->rows != 1 || t->cols != 1 || t->alias || strncmp(t->name, "__", 2)) {
                fail(SMQ_ERR_FORMAT, "invalid blob record: %s", t->name);
                goto out;
            }
        } else if (t->alias > 1 || (t->alias && mf->version < 2) || !t->rows || !t->cols ||
                   t->cols > MAX_TENSOR_COLS || t->dtype > SMQ_DTYPE_Q5 || !strncmp(t->name, "__", 2)) {
            fail(SMQ_ERR_FORMAT, "invalid tensor metadata: %s", t->name);
            goto out;
        }
        if (t->bytes != payload_bytes(t) || (!t->alias && t->offset < previous) || t->offset > size ||
            t->bytes > size - t->offset) {
            fail(SMQ_ERR_FORMAT, "invalid tensor extent: %s", t->name);
            goto out;
        }
        if (t->alias) { /* the only alias: lm_head sharing embed's extent */
            const smq_tensor *e = NULL;
            uint32_t j;
            for (j = 0; j < i; ++j)
                if (!strcmp(mf->tensors[j].name, "embed")) e = &mf->tensors[j];
            if (!e || strcmp(t->name, "lm_head") || t->offset != e->offset || t->bytes != e->bytes ||
                t->rows != e->rows || t->cols != e->cols || t->dtype != e->dtype) {
                fail(SMQ_ERR_FORMAT, "invalid tied embedding alias");
                goto out;
            }
        }
        previous = t->offset + t->bytes;
        if (i && strcmp(mf->tensors[i - 1].name, t->name) >= 0) {
            fail(SMQ_ERR_FORMAT, "tensor directory must have unique sorted names");
            goto out;
        }
        if (t->dtype == SMQ_DTYPE_BLOB) ++mf->blobs;
        t->data = data + t->offset;
    }
    smq_clear_error();
    return SMQ_OK;
bad_name:
    fail(SMQ_ERR_FORMAT, "invalid tensor name");
out:
    smq_modelfile_release(mf);
    return smq_last_status();
}

const smq_tensor *smq_modelfile_blob(const smq_modelfile *mf, const char *name) {
    uint32_t i;
    for (i = 0; mf && i < mf->count; ++i)
        if (mf->tensors[i].dtype == SMQ_DTYPE_BLOB && !strcmp(mf->tensors[i].name, name)) return &mf->tensors[i];
    return NULL;
}

const smq_tensor *smq_modelfile_find(const smq_modelfile *mf, const char *name, uint32_t rows, uint32_t cols,
                                     uint32_t dtype) {
    uint32_t lo = 0, hi = mf ? mf->count : 0;
    const smq_tensor *t;
    while (lo < hi) { /* names are sorted */
        uint32_t mid = lo + (hi - lo) / 2;
        if (strcmp(mf->tensors[mid].name, name) < 0) lo = mid + 1;
        else hi = mid;
    }
    if (!mf || lo == mf->count || strcmp(mf->tensors[lo].name, name)) {
        fail(SMQ_ERR_FORMAT, "missing tensor: %s", name);
        return NULL;
    }
    t = &mf->tensors[lo];
    if (t->rows != rows || t->cols != cols ||
        (dtype == SMQ_DTYPE_QUANTIZED ? t->dtype == SMQ_DTYPE_F32 : t->dtype != dtype)) {
        fail(SMQ_ERR_FORMAT, "wrong tensor shape/type: %s", name);
        return NULL;
    }
    return t;
}

smq_status smq_modelfile_verify_payload(const smq_modelfile *mf) {
    uint32_t i;
    for (i = 0; mf && i < mf->count; ++i) {
        const smq_tensor *t = &mf->tensors[i];
        uint64_t u, units;
        int ok = 1;
        if (t->alias || t->dtype == SMQ_DTYPE_BLOB) continue;
        units = t->dtype == SMQ_DTYPE_F32 ? t->bytes / 4 : t->bytes / block_size(t->dtype);
        for (u = 0; u < units && ok; ++u) {
            if (t->dtype == SMQ_DTYPE_Q8) {
                float s = rd_f32(t->data + u * Q8_BLOCK);
                ok = finite_f(s) && s >= 0;
            } else if (t->dtype == SMQ_DTYPE_Q5) {
                const unsigned char *p = t->data + u * Q5_BLOCK;
                ok = finite_f(f16_value((uint16_t)(p[0] | p[1] << 8)));
            } else {
                ok = finite_f(rd_f32(t->data + u * 4));
            }
        }
        if (!ok) return fail(SMQ_ERR_NUMERIC, "non-finite value or invalid scale in tensor %s", t->name);
    }
    return SMQ_OK;
}

/* ---- model ------------------------------------------------------------- */

typedef struct Layer {
    const float *attn_norm, *ffn_norm, *q_bias, *k_bias, *v_bias;
    smq_qmat q, k, v, o, gate, up, down;
} Layer;

struct smq_model {
    smq_config c;
    uint32_t context, batch, logit_rows, head_dim, q_dim, kv_dim, nb_dim, nb_q, nb_hidden, pairs;
    smq_attn_shape shape;
    smq_qmat embed, head;
    const float *final_norm;
    Layer *layers;
    /* device memory */
    unsigned char *weights;
    float *vectors;
    float *x, *q, *k, *v, *att, *gate, *up, *xd, *hd, *logits, *keys, *values, *rope_cos, *rope_sin;
    int8_t *xq, *hq;
    uint32_t *tokens, *token, *count, *history;
    int32_t *pos;
    unsigned char *banned;
    size_t device_bytes;
    void *step; /* captured decode step */
};

static void *dev_alloc(smq_model *m, size_t bytes) {
    void *p = smq_malloc(bytes);
    if (p) m->device_bytes += bytes;
    return p;
}

void smq_model_close(smq_model *m) {
    if (!m) return;
    if (m->step) smq_graph_destroy(m->step);
    smq_free(m->weights);
    smq_free(m->vectors);
    smq_free(m->x);
    smq_free(m->q);
    smq_free(m->k);
    smq_free(m->v);
    smq_free(m->att);
    smq_free(m->gate);
    smq_free(m->up);
    smq_free(m->xd);
    smq_free(m->xq);
    smq_free(m->hd);
    smq_free(m->hq);
    smq_free(m->logits);
    smq_free(m->keys);
    smq_free(m->values);
    smq_free(m->rope_cos);
    smq_free(m->rope_sin);
    smq_free(m->tokens);
    smq_free(m->token);
    smq_free(m->count);
    smq_free(m->history);
    smq_free(m->pos);
    smq_free(m->banned);
    free(m->layers);
    free(m);
}

const smq_config *smq_model_config(const smq_model *m) { return m ? &m->c : NULL; }
size_t smq_model_device_bytes(const smq_model *m) { return m ? m->device_bytes : 0; }

/* Llama 3 RoPE frequency scaling (model.c:95-107). */
static double llama3_scale(const smq_config *c, double freq) {
    double wavelen, smooth;
    if (!c->llama3_rope) return freq;
    wavelen = 2.0 * 3.14159265358979323846 / freq;
    if (wavelen < (double)c->llama3_original / c->llama3_high) return freq;
    if (wavelen > (double)c->llama3_original / c->llama3_low) return freq / c->llama3_factor;
    smooth = ((double)c->llama3_original / wavelen - c->llama3_low) / (c->llama3_high - c->llama3_low);
    return (1.0 - smooth) * freq / c->llama3_factor + smooth * freq;
}

/* A tensor to upload: where it is in the checkpoint and where it goes. */
typedef struct Upload {
    const smq_tensor *t;
    size_t at;
} Upload;

typedef struct Loader {
    const smq_modelfile *mf;
    Upload *q;      /* quantized matrices */
    uint32_t nq, capq;
    size_t qbytes;  /* weight arena size */
    Upload *f;      /* f32 vectors */
    uint32_t nf, capf;
    size_t fcount;  /* f32 arena length in floats */
} Loader;

static int push(Upload **list, uint32_t *n, uint32_t *cap, const smq_tensor *t, size_t at) {
    if (*n == *cap) {
        uint32_t nc = *cap ? 2 * *cap : 64;
        Upload *p = (Upload *)realloc(*list, nc * sizeof(Upload));
        if (!p) return fail(SMQ_ERR_NOMEM, "allocation failed"), 0;
        *list = p;
        *cap = nc;
    }
    (*list)[*n].t = t;
    (*list)[*n].at = at;
    ++*n;
    return 1;
}

/* qmat (model.c:15-29): finds the matrix and reserves its device slot; the
 * data pointer is an arena offset until the arena exists. A tied lm_head
 * reuses embed's slot. */
static int plan_qmat(Loader *ld, const char *name, uint32_t rows, uint32_t cols, smq_qmat *q) {
    const smq_tensor *t = smq_modelfile_find(ld->mf, name, rows, cols, SMQ_DTYPE_QUANTIZED);
    uint32_t i;
    size_t at;
    if (!t) return 0;
    q->rows = rows;
    q->cols = cols;
    q->nb = (cols + QK - 1) / QK;
    q->dtype = t->dtype;
    q->row_bytes = (size_t)q->nb * block_size(t->dtype);
    for (i = 0; i < ld->nq; ++i)
        if (ld->q[i].t->offset == t->offset && ld->q[i].t->bytes == t->bytes && t->alias) {
            q->data = (const unsigned char *)(uintptr_t)ld->q[i].at;
            return 1;
        }
    at = (ld->qbytes + 255) & ~(size_t)255;
    if (!push(&ld->q, &ld->nq, &ld->capq, t, at)) return 0;
    ld->qbytes = at + (size_t)t->bytes;
    q->data = (const unsigned char *)(uintptr_t)at;
    return 1;
}

/* fvec (model.c:32-42): an F32 1 x n vector, slot in the f32 arena. */
static int plan_fvec(Loader *ld, const char *name, uint32_t n, const float **v) {
    const smq_tensor *t = smq_modelfile_find(ld->mf, name, 1, n, SMQ_DTYPE_F32);
    size_t at;
    if (!t) return 0;
    at = (ld->fcount + 63) & ~(size_t)63;
    if (!push(&ld->f, &ld->nf, &ld->capf, t, at)) return 0;
    ld->fcount = at + n;
    *v = (const float *)(uintptr_t)at;
    return 1;
}

static const char *lname(char *buf, uint32_t layer, const char *suffix) {
    snprintf(buf, SMQ_TENSOR_NAME_SIZE, "l.%u.%s", layer, suffix);
    return buf;
}

static void rebase_q(smq_qmat *q, unsigned char *base) { q->data = base + (uintptr_t)q->data; }
static const float *rebase_f(const float *v, float *base) { return v ? base + (uintptr_t)v : NULL; }

static int plan_model(smq_model *m, Loader *ld) {
    const smq_config *c = &m->c;
    char name[SMQ_TENSOR_NAME_SIZE];
    smq_qmat unused;
    uint32_t l;
    if (!plan_qmat(ld, "embed", c->vocab, c->dim, &m->embed) || !plan_qmat(ld, "lm_head", c->vocab, c->dim, &m->head) ||
        !plan_fvec(ld, "final_norm", c->dim, &m->final_norm))
        return 0;
    for (l = 0; l < c->layers; ++l) {
        Layer *L = &m->layers[l];
        if (!plan_fvec(ld, lname(name, l, "attn_norm"), c->dim, &L->attn_norm) ||
            !plan_fvec(ld, lname(name, l, "ffn_norm"), c->dim, &L->ffn_norm) ||
            !plan_qmat(ld, lname(name, l, "q"), m->q_dim, c->dim, &L->q) ||
            !plan_qmat(ld, lname(name, l, "k"), m->kv_dim, c->dim, &L->k) ||
            !plan_qmat(ld, lname(name, l, "v"), m->kv_dim, c->dim, &L->v) ||
            !plan_qmat(ld, lname(name, l, "o"), c->dim, m->q_dim, &L->o))
            return 0;
        /* the router of a one-expert layer is loaded but never applied (model.c:631-633) */
        if (!smq_modelfile_find(ld->mf, lname(name, l, "router"), c->experts, c->dim, SMQ_DTYPE_QUANTIZED)) return 0;
        if (c->qkv_bias && (!plan_fvec(ld, lname(name, l, "q_bias"), m->q_dim, &L->q_bias) ||
                            !plan_fvec(ld, lname(name, l, "k_bias"), m->kv_dim, &L->k_bias) ||
                            !plan_fvec(ld, lname(name, l, "v_bias"), m->kv_dim, &L->v_bias)))
            return 0;
        if (!plan_qmat(ld, lname(name, l, "e.0.gate"), c->hidden, c->dim, &L->gate) ||
            !plan_qmat(ld, lname(name, l, "e.0.up"), c->hidden, c->dim, &L->up) ||
            !plan_qmat(ld, lname(name, l, "e.0.down"), c->dim, c->hidden, &L->down))
            return 0;
    }
    (void)unused;
    return 1;
}

/* Copies the planned tensors into the arenas. */
static int upload(smq_model *m, Loader *ld) {
    uint32_t i, l;
    float *staging;
    m->weights = (unsigned char *)dev_alloc(m, ld->qbytes ? ld->qbytes : 1);
    m->vectors = (float *)dev_alloc(m, (ld->fcount ? ld->fcount : 1) * sizeof(float));
    if (!m->weights || !m->vectors) return 0;
    for (i = 0; i < ld->nq; ++i)
        if (smq_memcpy_htod(m->weights + ld->q[i].at, ld->q[i].t->data, (size_t)ld->q[i].t->bytes) != SMQ_OK)
            return 0;
    staging = (float *)calloc(ld->fcount ? ld->fcount : 1, sizeof(float));
    if (!staging) return fail(SMQ_ERR_NOMEM, "allocation failed"), 0;
    for (i = 0; i < ld->nf; ++i) {
        const smq_tensor *t = ld->f[i].t;
        uint32_t j;
        for (j = 0; j < t->cols; ++j) staging[ld->f[i].at + j] = rd_f32(t->data + (size_t)j * 4);
    }
    i = smq_memcpy_htod(m->vectors, staging, ld->fcount * sizeof(float)) == SMQ_OK;
    free(staging);
    if (!i) return 0;
    rebase_q(&m->embed, m->weights);
    rebase_q(&m->head, m->weights);
    m->final_norm = rebase_f(m->final_norm, m->vectors);
    for (l = 0; l < m->c.layers; ++l) {
        Layer *L = &m->layers[l];
        rebase_q(&L->q, m->weights);
        rebase_q(&L->k, m->weights);
        rebase_q(&L->v, m->weights);
        rebase_q(&L->o, m->weights);
        rebase_q(&L->gate, m->weights);
        rebase_q(&L->up, m->weights);
        rebase_q(&L->down, m->weights);
        L->attn_norm = rebase_f(L->attn_norm, m->vectors);
        L->ffn_norm = rebase_f(L->ffn_norm, m->vectors);
        L->q_bias = rebase_f(L->q_bias, m->vectors);
        L->k_bias = rebase_f(L->k_bias, m->vectors);
        L->v_bias = rebase_f(L->v_bias, m->vectors);
    }
    return 1;
}

/* cos/sin tables for every position (model.c:425-437, host double). */
static int rope_tables(smq_model *m) {
    const smq_config *c = &m->c;
    const uint32_t half = m->pairs;
    const size_t n = (size_t)m->context * half;
    double *inv_freq = (double *)calloc(half ? half : 1, sizeof(double));
    float *cs = (float *)calloc(n ? n : 1, sizeof(float)), *sn = (float *)calloc(n ? n : 1, sizeof(float));
    uint32_t i, p;
    int ok = 0;
    if (!inv_freq || !cs || !sn) {
        fail(SMQ_ERR_NOMEM, "allocation failed");
        goto done;
    }
    /* With a sliding window every layer of a non-Gemma model is local
     * (model.c:463-466) and rotates by the rope_local_theta tables, which
     * carry no Llama 3 scaling (model.c:166-169, 502-504). */
    for (i = 0; i < half; ++i)
        inv_freq[i] = c->sliding_window
                          ? pow((double)c->local_theta, -(double)(2 * i) / (double)c->rotary_dim)
                          : llama3_scale(c, pow((double)c->theta, -(double)(2 * i) / (double)c->rotary_dim));
    for (p = 0; p < m->context; ++p)
        for (i = 0; i < half; ++i) {
            double angle = (double)p * inv_freq[i];
            cs[(size_t)p * half + i] = (float)(c->rope_factor * cos(angle));
            sn[(size_t)p * half + i] = (float)(c->rope_factor * sin(angle));
        }
    m->rope_cos = (float *)dev_alloc(m, (n ? n : 1) * sizeof(float));
    m->rope_sin = (float *)dev_alloc(m, (n ? n : 1) * sizeof(float));
    ok = m->rope_cos && m->rope_sin && smq_memcpy_htod(m->rope_cos, cs, n * sizeof(float)) == SMQ_OK &&
         smq_memcpy_htod(m->rope_sin, sn, n * sizeof(float)) == SMQ_OK;
done:
    free(inv_freq);
    free(cs);
    free(sn);
    return ok;
}

static int buffers(smq_model *m) {
    const smq_config *c = &m->c;
    const size_t b = m->batch, nb_max = m->nb_dim > m->nb_q ? m->nb_dim : m->nb_q;
    const size_t kv = (size_t)c->layers * m->context * m->kv_dim * sizeof(float);
    m->x = (float *)dev_alloc(m, b * c->dim * 4);
    m->q = (float *)dev_alloc(m, b * m->q_dim * 4);
    m->k = (float *)dev_alloc(m, b * m->kv_dim * 4);
    m->v = (float *)dev_alloc(m, b * m->kv_dim * 4);
    m->att = (float *)dev_alloc(m, b * m->q_dim * 4);
    m->gate = (float *)dev_alloc(m, b * c->hidden * 4);
    m->up = (float *)dev_alloc(m, b * c->hidden * 4);
    m->xd = (float *)dev_alloc(m, b * nb_max * 4);
    m->xq = (int8_t *)dev_alloc(m, b * nb_max * QK);
    m->hd = (float *)dev_alloc(m, b * m->nb_hidden * 4);
    m->hq = (int8_t *)dev_alloc(m, b * m->nb_hidden * QK);
    m->logits = (float *)dev_alloc(m, (size_t)m->logit_rows * c->vocab * 4);
    m->keys = (float *)dev_alloc(m, kv);
    m->values = (float *)dev_alloc(m, kv);
    m->tokens = (uint32_t *)dev_alloc(m, b * 4);
    m->token = (uint32_t *)dev_alloc(m, 4);
    m->count = (uint32_t *)dev_alloc(m, 4);
    m->pos = (int32_t *)dev_alloc(m, 4);
    m->history = (uint32_t *)dev_alloc(m, (size_t)m->context * 4);
    m->banned = (unsigned char *)dev_alloc(m, c->vocab);
    if (!m->x || !m->q || !m->k || !m->v || !m->att || !m->gate || !m->up || !m->xd || !m->xq || !m->hd || !m->hq ||
        !m->logits || !m->keys || !m->values || !m->tokens || !m->token || !m->count || !m->pos || !m->history ||
        !m->banned)
        return 0;
    /* zeroed once: the reference's calloc'd cache (util.c:116) */
    return smq_memset(m->keys, 0, kv) == SMQ_OK && smq_memset(m->values, 0, kv) == SMQ_OK &&
           smq_memset(m->banned, 0, c->vocab) == SMQ_OK && smq_synchronize() == SMQ_OK;
}

smq_model *smq_model_open_bytes(const unsigned char *data, uint64_t size, const smq_config *config,
                                uint32_t context, uint32_t batch, uint32_t logit_rows) {
    smq_modelfile mf;
    Loader ld;
    smq_model *m;
    uint64_t expected;
    int ok = 0;
    memset(&ld, 0, sizeof(ld));
    if (!config) return fail(SMQ_ERR_RANGE, "config is NULL"), NULL;
    if (smq_modelfile_parse(&mf, data, size) != SMQ_OK) return NULL;
    m = (smq_model *)calloc(1, sizeof(smq_model));
    if (!m) {
        smq_modelfile_release(&mf);
        return fail(SMQ_ERR_NOMEM, "allocation failed"), NULL;
    }
    m->c = *config;
    if (smq_modelfile_verify_payload(&mf) != SMQ_OK) goto done;
    if (m->c.gemma3 || m->c.experts != 1 || m->c.shared) {
        fail(SMQ_ERR_FORMAT, "the gfx950 forward runs dense smolmoe_v1/smolmoe_qwen2 checkpoints (experts = 1, no "
             "shared experts); this one has %s, %u experts, %u shared", m->c.gemma3 ? "gemma3" : "no gemma3",
             m->c.experts, m->c.shared);
        goto done;
    }
    if (!context || context > m->c.max_context || !batch || !logit_rows || logit_rows > batch) {
        fail(SMQ_ERR_RANGE, "invalid context %u (max %u), batch %u or logit rows %u", context, m->c.max_context,
             batch, logit_rows);
        goto done;
    }
    m->context = context;
    m->batch = batch < context ? batch : context; /* main.c:804 */
    m->logit_rows = logit_rows < m->batch ? logit_rows : m->batch;
    m->head_dim = m->c.head_dim;
    m->q_dim = m->c.heads * m->head_dim;
    m->kv_dim = m->c.kv_heads * m->head_dim;
    m->nb_dim = (m->c.dim + QK - 1) / QK;
    m->nb_q = (m->q_dim + QK - 1) / QK;
    m->nb_hidden = (m->c.hidden + QK - 1) / QK;
    m->pairs = m->c.rotary_dim / 2;
    m->shape.heads = m->c.heads;
    m->shape.kv_heads = m->c.kv_heads;
    m->shape.head_dim = m->head_dim;
    m->shape.rotary_pairs = m->pairs;
    m->shape.window = m->c.sliding_window; /* every layer is local when set (model.c:464-466) */
    m->shape.context = context;
    expected = 3 + (uint64_t)m->c.layers * (7 + 3 * m->c.qkv_bias + 3 * (uint64_t)(m->c.experts + m->c.shared));
    if (expected != mf.count - mf.blobs) {
        fail(SMQ_ERR_FORMAT, "tensor count does not match config");
        goto done;
    }
    m->layers = (Layer *)calloc(m->c.layers, sizeof(Layer));
    if (!m->layers) {
        fail(SMQ_ERR_NOMEM, "allocation failed");
        goto done;
    }
    ld.mf = &mf;
    ld.fcount = 64; /* no vector at offset 0: a zero offset stands for "absent" */
    ok = plan_model(m, &ld) && upload(m, &ld) && buffers(m) && rope_tables(m);
done:
    free(ld.q);
    free(ld.f);
    smq_modelfile_release(&mf);
    if (!ok) {
        smq_status st = smq_last_status();
        char msg[1024];
        snprintf(msg, sizeof(msg), "%s", smq_last_error());
        smq_model_close(m);
        smq_set_error(st == SMQ_OK ? SMQ_ERR : st, msg);
        return NULL;
    }
    smq_clear_error();
    return m;
}

smq_model *smq_model_open(const char *path, const char *config_path, uint32_t context, uint32_t batch,
                          uint32_t logit_rows) {
    Mapping f;
    smq_config c;
    smq_model *m = NULL;
    if (map_file(path, &f) != SMQ_OK) return NULL;
    if (config_path) {
        if (smq_config_read(config_path, &c) != SMQ_OK) goto done;
    } else {
        smq_modelfile mf;
        const smq_tensor *blob;
        if (smq_modelfile_parse(&mf, f.data, f.size) != SMQ_OK) goto done;
        blob = smq_modelfile_blob(&mf, "__config__");
        if (!blob) {
            smq_modelfile_release(&mf);
            fail(SMQ_ERR_FORMAT, "no config: pass a config path, or embed it in the checkpoint");
            goto done;
        }
        if (smq_config_parse(blob->data, (size_t)blob->bytes, &c) != SMQ_OK) {
            smq_modelfile_release(&mf);
            goto done;
        }
        smq_modelfile_release(&mf);
    }
    m = smq_model_open_bytes(f.data, f.size, &c, context, batch, logit_rows);
done:
    unmap(&f);
    return m;
}

/* ---- forward ------------------------------------------------------------ */

#define TRY(call)                             \
    do {                                      \
        if ((call) != SMQ_OK) return smq_last_status(); \
    } while (0)

static smq_mat_item mat(const smq_qmat *w, const float *bias, float *y, int accumulate) {
    smq_mat_item it;
    it.w = w;
    it.bias = bias;
    it.y = y;
    it.accumulate = accumulate;
    return it;
}

/* The RMSNorm activation of one token's row x (model.c:334-342), formed by
 * the consuming matmul itself; xd/xq are the fallback's scratch. */
static smq_act norm_act(smq_model *m, const float *x, const float *weight) {
    smq_act a;
    memset(&a, 0, sizeof(a));
    a.kind = SMQ_ACT_NORM;
    a.cols = m->c.dim;
    a.x = x;
    a.norm = weight;
    a.eps = m->c.eps;
    a.xd_scratch = m->xd;
    a.xq_scratch = m->xq;
    return a;
}

/* attention_block (model.c:496-542) for one layer. */
static smq_status attention_block(smq_model *m, uint32_t l, uint32_t n, uint32_t pos0, const int32_t *pos_dev) {
    const Layer *L = &m->layers[l];
    const size_t base = (size_t)l * m->context * m->kv_dim;
    smq_mat_item qkv[3];
    qkv[0] = mat(&L->q, L->q_bias, m->q, 0);
    qkv[1] = mat(&L->k, L->k_bias, m->k, 0);
    qkv[2] = mat(&L->v, L->v_bias, m->v, 0);
    if (n == 1) { /* decode: the RMSNorm and its Q8 blocks inside the QKV launch, RoPE and the cache store in
                   * its store, then attention over the caches */
        smq_act act = norm_act(m, m->x, L->attn_norm);
        TRY(smq_matmul_act_rope(qkv, &act, &m->shape, m->rope_cos, m->rope_sin, m->keys + base, m->values + base,
                                pos0, pos_dev));
        TRY(smq_attention_q8(m->q, m->keys + base, m->values + base, m->att, 1, &m->shape, pos0, pos_dev, m->xd,
                             m->xq));
    } else {
        TRY(smq_norm_quantize(m->x, L->attn_norm, m->c.eps, n, m->c.dim, NULL, m->xd, m->xq));
        TRY(smq_matmul(qkv, 3, m->xd, m->xq, n));
        TRY(smq_rope_kv(m->q, m->k, m->v, n, &m->shape, m->rope_cos, m->rope_sin, m->keys + base, m->values + base,
                        pos0, pos_dev));
        TRY(smq_attention_q8(m->q, m->keys + base, m->values + base, m->att, n, &m->shape, pos0, pos_dev, m->xd,
                             m->xq));
    }
    qkv[0] = mat(&L->o, NULL, m->x, 1); /* x += o(att) */
    return smq_matmul(qkv, 1, m->xd, m->xq, n);
}

/* ffn_block with one expert (model.c:622-650). */
static smq_status ffn_block(smq_model *m, uint32_t l, uint32_t n) {
    const Layer *L = &m->layers[l];
    smq_mat_item it[2];
    if (n == 1) { /* decode: RMSNorm in the gate/up launch, SwiGLU and the Q8 of h in its store */
        smq_act act = norm_act(m, m->x, L->ffn_norm);
        TRY(smq_matmul_glu_q8(&L->gate, &L->up, &act, 1, m->up, m->hd, m->hq, m->gate));
        it[0] = mat(&L->down, NULL, m->x, 1); /* x += down(act) */
        return smq_matmul(it, 1, m->hd, m->hq, 1);
    }
    TRY(smq_norm_quantize(m->x, L->ffn_norm, m->c.eps, n, m->c.dim, NULL, m->xd, m->xq));
    it[0] = mat(&L->gate, NULL, m->gate, 0);
    it[1] = mat(&L->up, NULL, m->up, 0);
    TRY(smq_matmul(it, 2, m->xd, m->xq, n));
    TRY(smq_row_quantize(m->up, NULL, 0.0f, m->gate, 1, n, m->c.hidden, NULL, m->hd, m->hq));
    it[0] = mat(&L->down, NULL, m->x, 1); /* x += down(act) */
    return smq_matmul(it, 1, m->hd, m->hq, n);
}

/* model_forward_body (model.c:660-686) on device ids; asynchronous. With tokens_dev NULL, x already holds
 * the embedding of the one token (written by the previous decode step's argmax). */
static smq_status enqueue_forward(smq_model *m, const uint32_t *tokens_dev, uint32_t n, uint32_t pos0,
                                  const int32_t *pos_dev, int mode) {
    uint32_t l;
    if (tokens_dev) TRY(smq_embed(&m->embed, tokens_dev, n, m->x));
    for (l = 0; l < m->c.layers; ++l) {
        TRY(attention_block(m, l, n, pos0, pos_dev));
        TRY(ffn_block(m, l, n));
    }
    if (mode != SMQ_LOGITS_NONE) { /* output_logits (model.c:650-658) */
        const uint32_t first = mode == SMQ_LOGITS_ALL ? 0 : n - 1, rows = n - first;
        smq_mat_item head = mat(&m->head, NULL, m->logits, 0);
        if (rows > m->logit_rows) return fail(SMQ_ERR_STATE, "internal error: logits buffer too small");
        TRY(smq_norm_quantize(m->x + (size_t)first * m->c.dim, m->final_norm, m->c.eps, rows, m->c.dim, NULL, m->xd,
                              m->xq));
        TRY(smq_matmul(&head, 1, m->xd, m->xq, rows));
    }
    return SMQ_OK;
}

smq_status smq_model_forward(smq_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int mode) {
    uint32_t t;
    if (!m || !tokens) return fail(SMQ_ERR_RANGE, "forward: NULL argument");
    if (!n || n > m->batch || pos0 > m->context || n > m->context - pos0)
        return fail(SMQ_ERR_RANGE, "token batch exceeds context");
    if (mode < SMQ_LOGITS_NONE || mode > SMQ_LOGITS_ALL) return fail(SMQ_ERR_RANGE, "invalid logits mode %d", mode);
    for (t = 0; t < n; ++t)
        if (tokens[t] >= m->c.vocab) return fail(SMQ_ERR_RANGE, "token %u out of vocabulary", tokens[t]);
    /* A captured decode step is replayed only over launches made after its capture: a batch
     * forward (a prefill) drops it and the next smq_model_generate captures afresh. */
    if (n > 1 && m->step) {
        TRY(smq_synchronize());
        smq_graph_destroy(m->step);
        m->step = NULL;
    }
    TRY(smq_memcpy_htod(m->tokens, tokens, (size_t)n * 4));
    TRY(enqueue_forward(m, m->tokens, n, pos0, NULL, mode));
    return smq_numeric_check();
}

smq_status smq_model_prefill(smq_model *m, const uint32_t *tokens, uint32_t n, uint32_t pos0, int last_logits) {
    uint32_t done = 0;
    if (!m) return fail(SMQ_ERR_RANGE, "prefill: model is NULL");
    while (done < n) {
        const uint32_t chunk = n - done < m->batch ? n - done : m->batch;
        const int mode = last_logits && done + chunk == n ? SMQ_LOGITS_LAST : SMQ_LOGITS_NONE;
        TRY(smq_model_forward(m, tokens + done, chunk, pos0 + done, mode));
        done += chunk;
    }
    return SMQ_OK;
}

smq_status smq_model_logits(const smq_model *m, float *out, uint32_t rows) {
    if (!m || !out) return fail(SMQ_ERR_RANGE, "logits: NULL argument");
    if (rows > m->logit_rows) return fail(SMQ_ERR_RANGE, "logits: %u rows > %u", rows, m->logit_rows);
    return smq_memcpy_dtoh(out, m->logits, (size_t)rows * m->c.vocab * 4);
}

const float *smq_model_logits_device(const smq_model *m) { return m ? m->logits : NULL; }

const float *smq_model_kv_layer(const smq_model *m, uint32_t layer, int values) {
    if (!m || layer >= m->c.layers) return NULL;
    return (values ? m->values : m->keys) + (size_t)layer * m->context * m->kv_dim;
}

smq_status smq_model_set_banned(smq_model *m, const unsigned char *banned) {
    if (!m) return fail(SMQ_ERR_RANGE, "set_banned: model is NULL");
    if (!banned) {
        TRY(smq_memset(m->banned, 0, m->c.vocab));
        return smq_synchronize();
    }
    return smq_memcpy_htod(m->banned, banned, m->c.vocab);
}

/* One decode step on device state: the layers over x (the embedding of *token) at *pos, logits, argmax
 * into *token, history[*count++] = *token and ++*pos, and x = the embedding of the new *token, the next
 * step's input (one launch fewer per token than embedding at the step's start). */
static smq_status enqueue_step(smq_model *m) {
    TRY(enqueue_forward(m, NULL, 1, 0, m->pos, SMQ_LOGITS_LAST));
    return smq_argmax_advance_embed(m->logits, m->c.vocab, m->banned, m->token, m->pos, m->count, m->history,
                                    m->context, &m->embed, m->x);
}

smq_status smq_model_prepare_decode(smq_model *m) {
    smq_status st;
    if (!m) return fail(SMQ_ERR_RANGE, "prepare_decode: model is NULL");
    if (m->step) return SMQ_OK;
    /* capture once; replays read pos/token from device memory */
    TRY(smq_synchronize());
    TRY(smq_capture_begin());
    st = enqueue_step(m);
    m->step = smq_capture_end();
    if (st != SMQ_OK) return st;
    if (!m->step) return smq_last_status();
    return SMQ_OK;
}

smq_status smq_model_generate(smq_model *m, uint32_t pos, uint32_t ntokens, uint32_t *out) {
    const int32_t start = (int32_t)pos;
    const uint32_t one = 1;
    uint32_t i;
    if (!m || !out) return fail(SMQ_ERR_RANGE, "generate: NULL argument");
    if (!ntokens) return SMQ_OK;
    if (pos > m->context || ntokens - 1 > m->context - pos || ntokens > m->context)
        return fail(SMQ_ERR_RANGE, "prompt + tokens exceeds context");
    if (ntokens > 1) TRY(smq_model_prepare_decode(m));
    /* out[0] from the logits already there (main.c:580-582); its embedding is the first step's input */
    TRY(smq_argmax(m->logits, m->c.vocab, m->banned, m->token));
    if (ntokens > 1) TRY(smq_embed(&m->embed, m->token, 1, m->x));
    TRY(smq_memcpy_dtod(m->history, m->token, 4));
    TRY(smq_memcpy_htod(m->count, &one, 4));
    TRY(smq_memcpy_htod(m->pos, &start, 4));
    for (i = 1; i < ntokens; ++i) TRY(smq_graph_launch(m->step));
    TRY(smq_numeric_check());
    TRY(smq_memcpy_dtoh(out, m->history, (size_t)ntokens * 4));
    for (i = 0; i < ntokens; ++i)
        if (out[i] >= m->c.vocab) return fail(SMQ_ERR_STATE, "every token is banned"); /* sampler.c:62 */
    return SMQ_OK;
}
