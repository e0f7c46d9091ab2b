/* Synthetic checkpoints for benchmarks and tests (include/smq_model.h).
 *
 * Writes a SMOEQ8 version-3 file (docs/FORMAT.md "Checkpoint container") with
 * the embedded "__config__" blob and the one-expert tensor set of the config
 * (docs/FORMAT.md "Tensor names"): every quantized matrix drawn from
 * N(0, sigma) and packed with the Q8 writer's rule (tools/q8pack.c:38-44:
 * scale = f32(max|v| / 127), q = clamp(nearbyint(double(v)/double(scale)),
 * -127, 127), zero padding), norm weights 1, Qwen2 biases N(0, sigma). A tied
 * checkpoint stores lm_head as an alias of embed.
 *
 * Draws: per tensor, a splitmix64 stream seeded from (seed, tensor name);
 * consecutive outputs pair into Box-Muller normals in double, scaled by
 * sigma and rounded once to f32 -- the recipe of the package's synth.py, run
 * over rows in parallel threads so a 0.5B-parameter checkpoint takes seconds.
 */
#define _POSIX_C_SOURCE 200809L

#include "smq_model.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Output i (0-based) of the splitmix64 stream seeded with s. */
static uint64_t stream_at(uint64_t s, uint64_t i) { return mix(s + (i + 1) * GOLDEN); }

/* Element e of the N(0, 1) sequence of stream s (Box-Muller over pairs). */
static double normal_at(uint64_t s, uint64_t e) {
    const uint64_t p = e / 2;
    const double u1 = 1.0 - (double)(stream_at(s, 2 * p) >> 11) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(stream_at(s, 2 * p + 1) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1)), a = 2.0 * 3.14159265358979323846 * u2;
    return (e & 1) ? r * sin(a) : r * cos(a);
}

static uint64_t name_seed(uint64_t seed, const char *name) {
    uint64_t h = 1469598103934665603ull; /* FNV-1a */
    for (; *name; ++name) h = (h ^ (unsigned char)*name) * 1099511628211ull;
    return mix(seed ^ h);
}

typedef struct Tensor {
    char name[SMQ_TENSOR_NAME_SIZE];
    uint32_t rows, cols, dtype, alias;
    uint64_t offset, bytes;
    float fill; /* F32 vectors: constant value, or NAN for N(0, sigma) */
} Tensor;

typedef struct Job {
    const Tensor *t;
    uint64_t seed;
    double sigma;
    unsigned char *out;
    uint32_t r0, r1;
} Job;

/* Q8 rows [r0, r1) of one matrix (tools/q8pack.c:38-44). */
static void *q8_rows(void *arg) {
    const Job *j = (const Job *)arg;
    const uint32_t cols = j->t->cols, nb = (cols + 31) / 32;
    float v[32];
    uint32_t r, b, i;
    for (r = j->r0; r < j->r1; ++r)
        for (b = 0; b < nb; ++b) {
            unsigned char *blk = j->out + ((size_t)r * nb + b) * 36;
            float high = 0.0f, scale;
            for (i = 0; i < 32; ++i) {
                const uint32_t c = b * 32 + i;
                v[i] = c < cols ? (float)(normal_at(j->seed, (uint64_t)r * cols + c) * j->sigma) : 0.0f;
                if (fabsf(v[i]) > high) high = fabsf(v[i]);
            }
            scale = high / 127.0f;
            memcpy(blk, &scale, 4);
            for (i = 0; i < 32; ++i) {
                double q = scale != 0.0f ? nearbyint((double)v[i] / (double)scale) : 0.0;
                if (q > 127) q = 127;
                if (q < -127) q = -127;
                blk[4 + i] = (unsigned char)(int8_t)q;
            }
        }
    return NULL;
}

static int add(Tensor *list, uint32_t *n, uint32_t cap, const char *name, uint32_t rows, uint32_t cols,
               uint32_t dtype, float fill) {
    Tensor *t;
    if (*n == cap || strlen(name) >= SMQ_TENSOR_NAME_SIZE) return 0;
    t = &list[(*n)++];
    memset(t, 0, sizeof(*t));
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->rows = rows;
    t->cols = cols;
    t->dtype = dtype;
    t->fill = fill;
    t->bytes = dtype == SMQ_DTYPE_F32 ? (uint64_t)rows * cols * 4
             : dtype == SMQ_DTYPE_BLOB ? 0 : (uint64_t)rows * ((cols + 31) / 32) * 36;
    return 1;
}

static int by_name(const void *a, const void *b) { return strcmp(((const Tensor *)a)->name, ((const Tensor *)b)->name); }

static void put_u32(unsigned char *p, uint32_t v) {
    p[0] = (unsigned char)v;
    p[1] = (unsigned char)(v >> 8);
    p[2] = (unsigned char)(v >> 16);
    p[3] = (unsigned char)(v >> 24);
}
static void put_u64(unsigned char *p, uint64_t v) {
    put_u32(p, (uint32_t)v);
    put_u32(p + 4, (uint32_t)(v >> 32));
}

static int write_all(int fd, const void *buf, size_t n, uint64_t at) {
    const unsigned char *p = (const unsigned char *)buf;
    while (n) {
        ssize_t w = pwrite(fd, p, n, (off_t)at);
        if (w <= 0) return 0;
        p += w;
        n -= (size_t)w;
        at += (uint64_t)w;
    }
    return 1;
}

smq_status smq_synth_checkpoint(const char *path, const char *config_text, uint64_t seed, float sigma, int tied,
                                uint32_t threads) {
    smq_config c;
    Tensor *list = NULL;
    uint32_t n = 0, cap, l, i;
    uint64_t at;
    unsigned char *dir = NULL;
    int fd = -1;
    smq_status st;
    char name[64];
    if (!path || !config_text) return smq_set_error(SMQ_ERR_RANGE, "synth_checkpoint: NULL argument");
    st = smq_config_parse((const unsigned char *)config_text, strlen(config_text), &c);
    if (st != SMQ_OK) return st;
    if (c.experts != 1 || c.shared || c.gemma3)
        return smq_set_error(SMQ_ERR_FORMAT, "synth_checkpoint: only one-expert smolmoe_v1/qwen2 configs");
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    cap = 4 + c.layers * 13;
    list = (Tensor *)calloc(cap, sizeof(Tensor));
    if (!list) return smq_set_error(SMQ_ERR_NOMEM, "allocation failed");
    {
        const uint32_t qd = c.heads * c.head_dim, kd = c.kv_heads * c.head_dim;
        int ok = add(list, &n, cap, "__config__", 1, 1, SMQ_DTYPE_BLOB, 0) &&
                 add(list, &n, cap, "embed", c.vocab, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, "lm_head", c.vocab, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, "final_norm", 1, c.dim, SMQ_DTYPE_F32, 1.0f);
        list[0].bytes = strlen(config_text);
        for (l = 0; ok && l < c.layers; ++l) {
#define LN(s) (snprintf(name, sizeof(name), "l.%u.%s", l, s), name)
            ok = add(list, &n, cap, LN("attn_norm"), 1, c.dim, SMQ_DTYPE_F32, 1.0f) &&
                 add(list, &n, cap, LN("ffn_norm"), 1, c.dim, SMQ_DTYPE_F32, 1.0f) &&
                 add(list, &n, cap, LN("q"), qd, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("k"), kd, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("v"), kd, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("o"), c.dim, qd, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("router"), 1, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("e.0.gate"), c.hidden, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("e.0.up"), c.hidden, c.dim, SMQ_DTYPE_Q8, 0) &&
                 add(list, &n, cap, LN("e.0.down"), c.dim, c.hidden, SMQ_DTYPE_Q8, 0);
            if (ok && c.qkv_bias)
                ok = add(list, &n, cap, LN("q_bias"), 1, qd, SMQ_DTYPE_F32, NAN) &&
                     add(list, &n, cap, LN("k_bias"), 1, kd, SMQ_DTYPE_F32, NAN) &&
                     add(list, &n, cap, LN("v_bias"), 1, kd, SMQ_DTYPE_F32, NAN);
#undef LN
        }
        if (!ok) {
            free(list);
            return smq_set_error(SMQ_ERR_RANGE, "synth_checkpoint: tensor table overflow");
        }
    }
    qsort(list, n, sizeof(Tensor), by_name);
    at = 16 + (uint64_t)n * 72;
    for (i = 0; i < n; ++i) { /* payloads in directory order, 64-byte aligned */
        if (tied && !strcmp(list[i].name, "lm_head")) continue;
        at = (at + 63) & ~(uint64_t)63;
        list[i].offset = at;
        at += list[i].bytes;
    }
    if (tied) { /* the alias is placed after embed (embed < lm_head) */
        for (i = 0; i < n; ++i)
            if (!strcmp(list[i].name, "lm_head")) {
                uint32_t e;
                for (e = 0; e < n; ++e)
                    if (!strcmp(list[e].name, "embed")) {
                        list[i].offset = list[e].offset;
                        list[i].bytes = list[e].bytes;
                        list[i].alias = 1;
                    }
            }
    }
    dir = (unsigned char *)calloc(16 + (size_t)n * 72, 1);
    if (!dir) {
        free(list);
        return smq_set_error(SMQ_ERR_NOMEM, "allocation failed");
    }
    memcpy(dir, "SMOEQ8\0\3", 8);
    put_u32(dir + 8, n);
    for (i = 0; i < n; ++i) {
        unsigned char *rec = dir + 16 + (size_t)i * 72;
        memcpy(rec, list[i].name, strlen(list[i].name));
        put_u32(rec + 40, list[i].rows);
        put_u32(rec + 44, list[i].cols);
        put_u32(rec + 48, list[i].dtype);
        put_u32(rec + 52, list[i].alias);
        put_u64(rec + 56, list[i].offset);
        put_u64(rec + 64, list[i].bytes);
    }
    fd = open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) {
        st = smq_set_error(SMQ_ERR_IO, strerror(errno));
        goto done;
    }
    if (ftruncate(fd, (off_t)at) != 0 || !write_all(fd, dir, 16 + (size_t)n * 72, 0)) {
        st = smq_set_error(SMQ_ERR_IO, "write failed");
        goto done;
    }
    for (i = 0; i < n; ++i) {
        const Tensor *t = &list[i];
        const uint64_t s = name_seed(seed, t->name);
        unsigned char *buf;
        if (t->alias) continue;
        if (t->dtype == SMQ_DTYPE_BLOB) {
            if (!write_all(fd, config_text, (size_t)t->bytes, t->offset)) goto io;
            continue;
        }
        buf = (unsigned char *)malloc(t->bytes ? (size_t)t->bytes : 1);
        if (!buf) {
            st = smq_set_error(SMQ_ERR_NOMEM, "allocation failed");
            goto done;
        }
        if (t->dtype == SMQ_DTYPE_F32) {
            uint32_t e;
            for (e = 0; e < t->cols; ++e) {
                float v = t->fill == t->fill ? t->fill : (float)(normal_at(s, e) * (double)sigma);
                memcpy(buf + (size_t)e * 4, &v, 4);
            }
        } else {
            pthread_t tid[256];
            Job jobs[256];
            uint32_t w, used = 0;
            for (w = 0; w < threads; ++w) {
                jobs[w].t = t;
                jobs[w].seed = s;
                jobs[w].sigma = (double)sigma;
                jobs[w].out = buf;
                jobs[w].r0 = (uint32_t)((uint64_t)t->rows * w / threads);
                jobs[w].r1 = (uint32_t)((uint64_t)t->rows * (w + 1) / threads);
                if (w == 0) continue;
                if (pthread_create(&tid[w], NULL, q8_rows, &jobs[w]) != 0) break;
                used = w;
            }
            q8_rows(&jobs[0]);
            for (w = 1; w <= used; ++w) pthread_join(tid[w], NULL);
            if (used + 1 < threads) /* a thread failed to start: do its share here */
                for (w = used + 1; w < threads; ++w) q8_rows(&jobs[w]);
        }
        if (!write_all(fd, buf, (size_t)t->bytes, t->offset)) {
            free(buf);
            goto io;
        }
        free(buf);
    }
    st = SMQ_OK;
    goto done;
io:
    st = smq_set_error(SMQ_ERR_IO, "write failed");
done:
    if (fd >= 0 && close(fd) != 0 && st == SMQ_OK) st = smq_set_error(SMQ_ERR_IO, "close failed");
    free(dir);
    free(list);
    return st;
}
