/* C ABI of the gfx950 quantized matrix-product path (include/smq.h).
 *
 * Host side of the drop-in: validates shapes and buffer extents before any
 * launch (a kernel must never be handed a grid or a pointer range it does not
 * fit), maps the reference's entry points (src/kernels.h:49-87, 183-196;
 * src/model.c:236-310) to launches on one stream, and keeps the reference's
 * error model: a status code plus a thread-local message (src/util.c:24-61).
 */
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <vector>
#include <mutex>

#include "smq.h"
#include "smq_internal.h"

namespace {

struct Context {
    bool ready = false;
    int device = -1;
    hipStream_t own = nullptr;
    hipStream_t cur = nullptr;
    int *flag = nullptr;    /* sticky numeric fault (quantize rows, matmul) */
    int *qflag = nullptr;   /* per-call fault of the synchronous quantizer */
    float *scalar = nullptr;
    void *argmax_parts = nullptr; /* smq::MAX_ARGMAX_PARTS partials of the two-stage argmax */
    float *scores = nullptr;      /* decode attention scores (heads x context), smq::SCORE_WORKSPACE_BYTES */
    float *mq_ws = nullptr;       /* split-K partial sums of the MFMA prefill GEMM, smq::MQ_WORKSPACE_BYTES */
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int fast = 0;
    int prefill_mfma = 0;
    int checks = 1;
    char arch[64] = {0};
    char backend[80] = {0};
};

Context g;
thread_local smq_status t_status = SMQ_OK;
thread_local char t_message[1024];
/* set between smq_capture_begin and smq_capture_end on the capturing thread */
thread_local bool t_capturing = false;

/* The library's own allocations (smq_malloc), base -> size: extent checks look here first, so a
 * check needs no runtime call for them, and none at all runs inside a stream capture. */
std::mutex g_alloc_mu;
std::map<uintptr_t, size_t> g_allocs;

/* 1: inside a registered allocation, 0: outside it, -1: not a registered allocation. */
int registry_extent(uintptr_t q, size_t bytes, uintptr_t &base, size_t &size) {
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_allocs.upper_bound(q);
    if (it == g_allocs.begin()) return -1;
    --it;
    base = it->first;
    size = it->second;
    if (q - base >= size) return -1;
    return bytes <= size - (q - base) ? 1 : 0;
}

smq_status set_status(smq_status s, const char *fmt, ...) {
    t_status = s;
    if (s == SMQ_OK) {
        t_message[0] = 0;
        return s;
    }
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_message, sizeof(t_message), fmt, ap);
    va_end(ap);
    return s;
}

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_status(e == hipErrorOutOfMemory ? SMQ_ERR_NOMEM : SMQ_ERR_STATE, "%s: %s", what, hipGetErrorString(e));
    return false;
}

bool ready() {
    if (g.ready) return true;
    set_status(SMQ_ERR_STATE, "smq_init has not been called");
    return false;
}

/* The byte range [p, p + bytes) must lie inside one device allocation. */
bool extent_ok(const void *p, size_t bytes, const char *what) {
    if (!bytes) return true;
    if (!p) {
        set_status(SMQ_ERR_RANGE, "%s is NULL", what);
        return false;
    }
    if (!g.checks) return true;
    const uintptr_t q = (uintptr_t)p;
    uintptr_t rb = 0;
    size_t rsize = 0;
    const int known = registry_extent(q, bytes, rb, rsize);
    if (known == 1) return true;
    if (known == 0) {
        set_status(SMQ_ERR_RANGE, "%s: %zu bytes at offset %zu exceed its allocation of %zu bytes", what, bytes,
                   (size_t)(q - rb), rsize);
        return false;
    }
    /* memory from another allocator: the runtime's lookup, never while this thread captures (the
     * captured launches then rest on the caller's own extents) */
    if (t_capturing) return true;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        (void)hipGetLastError();
        set_status(SMQ_ERR_RANGE, "%s is not a device allocation", what);
        return false;
    }
    const uintptr_t b = (uintptr_t)base;
    if (q < b || q - b > size || bytes > size - (q - b)) {
        set_status(SMQ_ERR_RANGE, "%s: %zu bytes at offset %zu exceed its allocation of %zu bytes", what, bytes,
                   (size_t)(q - b), size);
        return false;
    }
    return true;
}

uint32_t block_bytes(bool q5) { return q5 ? smq::Q5_BYTES : smq::Q8_BYTES; }

/* Validates one weight matrix and the activations of a launch. */
bool check_operands(const unsigned char *w, size_t row_bytes, uint32_t nrows, uint32_t nb, bool q5, const float *xd,
                    const int8_t *xq, uint32_t ntok, uint32_t xstride, const float *y, size_t y_stride,
                    const char *who) {
    if (!nrows || !ntok) return true;
    if (!nb) {
        set_status(SMQ_ERR_RANGE, "%s: nb is 0", who);
        return false;
    }
    const size_t row_need = (size_t)nb * block_bytes(q5);
    if (row_bytes < row_need) {
        set_status(SMQ_ERR_RANGE, "%s: row_bytes %zu < nb*%u", who, row_bytes, block_bytes(q5));
        return false;
    }
    if (xstride < nb && ntok > 1) {
        set_status(SMQ_ERR_RANGE, "%s: activation stride %u < nb %u", who, xstride, nb);
        return false;
    }
    if (y_stride < nrows && ntok > 1) {
        set_status(SMQ_ERR_RANGE, "%s: output stride %zu < rows %u", who, y_stride, nrows);
        return false;
    }
    const size_t acts = (size_t)(ntok - 1) * xstride + nb;
    return extent_ok(w, (size_t)(nrows - 1) * row_bytes + row_need, "weights") &&
           extent_ok(xd, acts * sizeof(float), "activation scales") && extent_ok(xq, acts * smq::QK, "activations") &&
           extent_ok(y, ((size_t)(ntok - 1) * y_stride + nrows) * sizeof(float), "output");
}

smq::MatArgs one_item(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                      uint32_t ntok, uint32_t nb, uint32_t xstride, float *out, size_t stride) {
    smq::MatArgs a;
    memset(&a, 0, sizeof(a));
    a.item[0].w = w;
    a.item[0].row_bytes = row_bytes;
    a.item[0].y = out;
    a.item[0].y_stride = stride;
    a.item[0].rows = nrows;
    a.nitems = 1;
    a.xd = xd;
    a.xq = xq;
    a.nb = nb;
    a.ntok = ntok;
    a.xstride = xstride;
    return a;
}

void gemm_impl(bool q5, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
               uint32_t ntok, uint32_t nb, uint32_t xstride, float *out, size_t stride, const char *who) {
    if (!ready()) return;
    if (!nrows || !ntok) return;
    if (!check_operands(w, row_bytes, nrows, nb, q5, xd, xq, ntok, xstride, out, stride, who)) return;
    hip_ok(smq::launch_matmul(one_item(w, row_bytes, xd, xq, nrows, ntok, nb, xstride, out, stride), q5, g.fast != 0,
                              g.cur),
           who);
}

/* The int8-MFMA prefill GEMM (relaxed block order) for a, if its layout allows: few-tile Q8 shapes on
 * the 64 x 64 tile kernel, the others and every Q5 shape on the block-pair kernel (K split over the
 * library workspace where the tiles are few). Returns false when
 * the layout does not allow it (nothing launched); a launch error sets the status. */
bool mfma_launch(const smq::MatArgs &a, bool q5) {
    if (!q5 && smq::mh_wanted(a)) {
        hip_ok(smq::launch_mh(a, g.cur), "mfma gemm");
        return true;
    }
    if (!q5 && smq::mq8_wanted(a)) {
        hip_ok(smq::launch_mq8(a, g.mq_ws, smq::MQ_WORKSPACE_BYTES, g.cur), "mfma gemm");
        return true;
    }
    if (!smq::mfma_layout_ok(a, q5)) return false;
    hip_ok(smq::launch_matmul_mfma(a, q5, nullptr, g.mq_ws, smq::MQ_WORKSPACE_BYTES, g.cur), "mfma gemm");
    return true;
}

void gemm_mfma_impl(bool q5, const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq,
                    uint32_t nrows, uint32_t ntok, uint32_t nb, float *out, size_t stride, const char *who) {
    if (!ready()) return;
    if (!nrows || !ntok) return;
    if (!check_operands(w, row_bytes, nrows, nb, q5, xd, xq, ntok, nb, out, stride, who)) return;
    const smq::MatArgs a = one_item(w, row_bytes, xd, xq, nrows, ntok, nb, nb, out, stride);
    /* rows or activations the MFMA staging cannot load take the exact GEMM */
    if (mfma_launch(a, q5)) return; /* a launch error has set the status */
    hip_ok(smq::launch_matmul(a, q5, g.fast != 0, g.cur), who);
}

float dot_impl(bool q5, const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    if (!ready()) return 0.0f;
    gemm_impl(q5, w, (size_t)nb * block_bytes(q5), xd, xq, 1, 1, nb, nb, g.scalar, 1, q5 ? "dot_q5" : "dot_q8");
    if (t_status != SMQ_OK) return 0.0f;
    float v = 0.0f;
    if (!hip_ok(hipMemcpyAsync(&v, g.scalar, sizeof(v), hipMemcpyDeviceToHost, g.cur), "dot") ||
        !hip_ok(hipStreamSynchronize(g.cur), "dot"))
        return 0.0f;
    return v;
}

}  // namespace

extern "C" {

smq_status smq_last_status(void) { return t_status; }
const char *smq_last_error(void) { return t_message; }
void smq_clear_error(void) { set_status(SMQ_OK, ""); }
smq_status smq_set_error(smq_status status, const char *message) {
    return set_status(status, "%s", message ? message : "");
}

smq_status smq_init(int device) {
    if (g.ready) {
        if (device == g.device) return SMQ_OK;
        return set_status(SMQ_ERR_STATE, "already initialised on device %d", g.device);
    }
    int count = 0;
    if (!hip_ok(hipGetDeviceCount(&count), "hipGetDeviceCount")) return t_status;
    if (device < 0 || device >= count) return set_status(SMQ_ERR_RANGE, "device %d of %d", device, count);
    if (!hip_ok(hipSetDevice(device), "hipSetDevice")) return t_status;
    hipDeviceProp_t prop;
    if (!hip_ok(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) return t_status;
    snprintf(g.arch, sizeof(g.arch), "%s", prop.gcnArchName);
    char *colon = strchr(g.arch, ':');
    if (colon) *colon = 0;
    if (strcmp(g.arch, "gfx950") != 0)
        return set_status(SMQ_ERR_STATE, "device %d is %s; this library is built for gfx950", device, g.arch);
    /* Default priority only: streams of other priorities are not used here. */
    if (!hip_ok(hipStreamCreateWithFlags(&g.own, hipStreamNonBlocking), "hipStreamCreate")) return t_status;
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, 256), "hipMalloc")) return t_status;
    g.flag = (int *)p;
    g.qflag = (int *)p + 16;
    g.scalar = (float *)p + 32;
    if (!hip_ok(hipMemset(p, 0, 256), "hipMemset")) return t_status;
    if (!hip_ok(hipMalloc(&g.argmax_parts, (size_t)smq::MAX_ARGMAX_PARTS * smq::ARGMAX_PART_BYTES), "hipMalloc"))
        return t_status;
    if (!hip_ok(hipMalloc((void **)&g.scores, smq::SCORE_WORKSPACE_BYTES), "hipMalloc")) return t_status;
    if (!hip_ok(hipMalloc((void **)&g.mq_ws, smq::MQ_WORKSPACE_BYTES), "hipMalloc")) return t_status;
    if (!hip_ok(hipEventCreate(&g.t0), "hipEventCreate") || !hip_ok(hipEventCreate(&g.t1), "hipEventCreate"))
        return t_status;
    /* the allocation-free argmax's static partials: their device address, once, with the device current */
    if (!hip_ok(smq::bind_noalloc_scratch(device), "hipGetSymbolAddress(scratch)")) return t_status;
    if (!hip_ok(smq::prepare_attention_attributes(), "hipFuncSetAttribute(attention)") ||
        !hip_ok(smq::prepare_fused_attributes(), "hipFuncSetAttribute(fused GEMV)") ||
        !hip_ok(smq::prepare_mq8_attributes(), "hipFuncSetAttribute(MFMA GEMM)"))
        return t_status;
    g.cur = g.own;
    g.device = device;
    const char *env = getenv("SMQ_CHECKS");
    g.checks = !(env && !strcmp(env, "0"));
    env = getenv("SMQ_ATT_GROUP"); /* read once: 0 sends prefill attention to the per-head kernel */
    smq::set_att_grouped(!(env && !strcmp(env, "0")));
    env = getenv("SMQ_MFMA_MH"); /* read once: 0 sends 28-block Q8 prefill GEMMs to the int8 MFMA kernels */
    smq::set_mh_enabled(!(env && !strcmp(env, "0")));
    g.ready = true;
    return set_status(SMQ_OK, "");
}

void smq_shutdown(void) {
    if (!g.ready) return;
    (void)hipStreamSynchronize(g.cur);
    (void)hipEventDestroy(g.t0);
    (void)hipEventDestroy(g.t1);
    (void)hipFree(g.flag);
    (void)hipFree(g.argmax_parts);
    (void)hipFree(g.scores);
    (void)hipFree(g.mq_ws);
    (void)hipStreamDestroy(g.own);
    g = Context();
}

void *smq_stream(void) { return g.cur; }

smq_status smq_set_stream(void *s) {
    if (!ready()) return t_status;
    g.cur = s ? (hipStream_t)s : g.own;
    return SMQ_OK;
}

smq_status smq_synchronize(void) {
    if (!ready()) return t_status;
    return hip_ok(hipStreamSynchronize(g.cur), "hipStreamSynchronize") ? SMQ_OK : t_status;
}

const char *smq_device_arch(void) { return g.ready ? g.arch : ""; }

const char *smq_kernels_select(int force_exact) {
    if (!g.ready && smq_init(0) != SMQ_OK) return "none";
    if (force_exact) g.fast = 0;
    snprintf(g.backend, sizeof(g.backend), "%s%s", g.arch, g.fast ? "-fast" : "");
    return g.backend;
}

void smq_kernels_set_fast(int fast) { g.fast = fast ? 1 : 0; }
int smq_kernels_fast(void) { return g.fast; }
size_t smq_gemm_scratch_bytes(uint32_t nb) {
    (void)nb;
    return 0;
}

/* Bounds checking of every operand range against its allocation (on by
 * default; SMQ_CHECKS=0 or smq_set_checks(0) turns it off for timing). */
void smq_set_checks(int on) { g.checks = on ? 1 : 0; }

int smq_quantize_q8(const float *x, uint32_t n, float *d, int8_t *q) {
    if (!ready()) return -1;
    const uint32_t nb = (n + smq::QK - 1) / smq::QK;
    if (!n) return 0;
    if (!extent_ok(x, (size_t)n * 4, "x") || !extent_ok(d, (size_t)nb * 4, "d") ||
        !extent_ok(q, (size_t)nb * smq::QK, "q"))
        return -1;
    int bad = 0;
    if (!hip_ok(hipMemsetAsync(g.qflag, 0, sizeof(int), g.cur), "quantize_q8") ||
        !hip_ok(smq::launch_quantize_q8(x, 1, n, d, q, g.qflag, g.cur), "quantize_q8") ||
        !hip_ok(hipMemcpyAsync(&bad, g.qflag, sizeof(int), hipMemcpyDeviceToHost, g.cur), "quantize_q8") ||
        !hip_ok(hipStreamSynchronize(g.cur), "quantize_q8"))
        return -1;
    return bad ? -1 : 0;
}

smq_status smq_quantize_q8_rows(const float *x, uint32_t rows, uint32_t n, float *d, int8_t *q) {
    if (!ready()) return t_status;
    const uint32_t nb = (n + smq::QK - 1) / smq::QK;
    if (!rows || !n) return SMQ_OK;
    if (!extent_ok(x, (size_t)rows * n * 4, "x") || !extent_ok(d, (size_t)rows * nb * 4, "d") ||
        !extent_ok(q, (size_t)rows * nb * smq::QK, "q"))
        return t_status;
    return hip_ok(smq::launch_quantize_q8(x, rows, n, d, q, g.flag, g.cur), "quantize_q8_rows") ? SMQ_OK : t_status;
}

smq_status smq_row_quantize(const float *src, const float *norm, float eps, const float *gate, int act, uint32_t rows,
                            uint32_t n, float *y, float *d, int8_t *q) {
    if (!ready()) return t_status;
    if (!rows || !n) return SMQ_OK;
    if (n > smq::MAX_ROW) return set_status(SMQ_ERR_RANGE, "row_quantize: %u columns exceed %u", n, smq::MAX_ROW);
    if (act < 0 || act > 2) return set_status(SMQ_ERR_RANGE, "row_quantize: activation %d", act);
    if (act && !gate) return set_status(SMQ_ERR_RANGE, "row_quantize: activation without gate");
    const uint32_t nb = (n + smq::QK - 1) / smq::QK;
    const size_t cells = (size_t)rows * n;
    if (!extent_ok(src, cells * 4, "src") || !extent_ok(norm, norm ? (size_t)n * 4 : 0, "norm") ||
        !extent_ok(gate, act ? cells * 4 : 0, "gate") || !extent_ok(y, y ? cells * 4 : 0, "y") ||
        !extent_ok(d, (size_t)rows * nb * 4, "d") || !extent_ok(q, (size_t)rows * nb * smq::QK, "q"))
        return t_status;
    return hip_ok(smq::launch_row_quantize(src, norm, eps, act ? gate : nullptr, act, rows, n, y, d, q, g.flag, g.cur),
                  "row_quantize")
               ? SMQ_OK
               : t_status;
}

smq_status smq_norm_quantize(const float *src, const float *norm, float eps, uint32_t rows, uint32_t n, float *y,
                             float *d, int8_t *q) {
    if (!norm) return set_status(SMQ_ERR_RANGE, "norm_quantize: norm is NULL");
    return smq_row_quantize(src, norm, eps, nullptr, 0, rows, n, y, d, q);
}

smq_status smq_silu_quantize(float *up, const float *gate, int gemma3, uint32_t rows, uint32_t n, float *d,
                             int8_t *q) {
    return smq_row_quantize(up, nullptr, 0.0f, gate, gemma3 ? 2 : 1, rows, n, up, d, q);
}

float smq_dot_q8(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_impl(false, w, xd, xq, nb);
}
float smq_dot_q5(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb) {
    return dot_impl(true, w, xd, xq, nb);
}

void smq_dot_q8_x4(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, uint32_t stride,
                   float *out) {
    gemm_impl(false, w, (size_t)nb * smq::Q8_BYTES, xd, xq, 1, 4, nb, stride, out, 1, "dot_q8_x4");
}
void smq_dot_q5_x4(const unsigned char *w, const float *xd, const int8_t *xq, uint32_t nb, uint32_t stride,
                   float *out) {
    gemm_impl(true, w, (size_t)nb * smq::Q5_BYTES, xd, xq, 1, 4, nb, stride, out, 1, "dot_q5_x4");
}
void smq_dot_q8_r4(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nb,
                   float *out) {
    gemm_impl(false, w, row_bytes, xd, xq, 4, 1, nb, nb, out, 4, "dot_q8_r4");
}
void smq_dot_q5_r4(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nb,
                   float *out) {
    gemm_impl(true, w, row_bytes, xd, xq, 4, 1, nb, nb, out, 4, "dot_q5_r4");
}

void smq_gemm_q8(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                 uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    gemm_impl(false, w, row_bytes, xd, xq, nrows, ntok, nb, nb, out, stride, "gemm_q8");
}
void smq_gemm_q5(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                 uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    gemm_impl(true, w, row_bytes, xd, xq, nrows, ntok, nb, nb, out, stride, "gemm_q5");
}

void smq_gemm_q8_mfma(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                      uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    gemm_mfma_impl(false, w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, "gemm_q8_mfma");
}
void smq_gemm_q5_mfma(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                      uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    gemm_mfma_impl(true, w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, "gemm_q5_mfma");
}

void smq_block_sums(int q5, const unsigned char *w, size_t row_bytes, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, int32_t *sums) {
    if (!ready()) return;
    if (!nrows || !ntok) return;
    if (!nb) {
        set_status(SMQ_ERR_RANGE, "block_sums: nb is 0");
        return;
    }
    const size_t row_need = (size_t)nb * block_bytes(q5 != 0);
    if (row_bytes < row_need) {
        set_status(SMQ_ERR_RANGE, "block_sums: row_bytes %zu < nb*%u", row_bytes, block_bytes(q5 != 0));
        return;
    }
    if (!extent_ok(w, (size_t)(nrows - 1) * row_bytes + row_need, "weights") ||
        !extent_ok(xq, (size_t)ntok * nb * smq::QK, "activations") ||
        !extent_ok(sums, (size_t)ntok * nrows * nb * sizeof(int32_t), "sums"))
        return;
    /* scales are not read in this mode: xq stands in for the scale pointer */
    smq::MatArgs a = one_item(w, row_bytes, (const float *)(const void *)xq, xq, nrows, ntok, nb, nb, nullptr, nrows);
    if (!smq::mfma_layout_ok(a, q5 != 0)) {
        set_status(SMQ_ERR_RANGE, "block_sums: rows and activations must be 4-byte aligned (and nb even for Q5)");
        return;
    }
    hip_ok(smq::launch_matmul_mfma(a, q5 != 0, sums, nullptr, 0, g.cur), "block_sums");
}

void smq_set_prefill_mfma(int on) { g.prefill_mfma = on ? 1 : 0; }

smq_status smq_set_gemv_rows(int rows) {
    if (!smq::set_gemv_rows(rows))
        return set_status(SMQ_ERR_RANGE, "set_gemv_rows: %d is not 0, 1, 2, 4, 8 or 16", rows);
    return SMQ_OK;
}

smq_status smq_set_exact_gemm(int mode) {
    if (!smq::set_exact_gemm(mode)) return set_status(SMQ_ERR_RANGE, "set_exact_gemm: %d is not 0, 1, 2, 3 or 4", mode);
    return SMQ_OK;
}

smq_status smq_matmul(const smq_mat_item *items, uint32_t n, const float *xd, const int8_t *xq, uint32_t ntok) {
    if (!ready()) return t_status;
    if (!items || n < 1 || n > SMQ_MAX_ITEMS) return set_status(SMQ_ERR_RANGE, "matmul: %u items", n);
    const uint32_t nb = items[0].w ? items[0].w->nb : 0;
    for (uint32_t i = 0; i < n; ++i) {
        const smq_qmat *w = items[i].w;
        if (!w) return set_status(SMQ_ERR_RANGE, "matmul: item %u has no matrix", i);
        if (w->nb != nb) return set_status(SMQ_ERR_STATE, "internal error: matmul inputs differ in width");
        if (w->dtype != 1 && w->dtype != 2) return set_status(SMQ_ERR_FORMAT, "matmul: dtype %u", w->dtype);
        if (w->nb != (w->cols + smq::QK - 1) / smq::QK)
            return set_status(SMQ_ERR_RANGE, "matmul: nb %u does not match %u columns", w->nb, w->cols);
        if (!check_operands(w->data, w->row_bytes, w->rows, w->nb, w->dtype == 2, xd, xq, ntok, nb, items[i].y,
                            w->rows, "matmul") ||
            !extent_ok(items[i].bias, items[i].bias ? (size_t)w->rows * 4 : 0, "bias"))
            return t_status;
    }
    if (!ntok) return SMQ_OK;
    /* One launch per weight format present (items keep their relative order). */
    for (int q5 = 0; q5 < 2; ++q5) {
        smq::MatArgs a;
        memset(&a, 0, sizeof(a));
        a.xd = xd;
        a.xq = xq;
        a.nb = nb;
        a.ntok = ntok;
        a.xstride = nb;
        a.flag = g.flag;
        for (uint32_t i = 0; i < n; ++i) {
            const smq_qmat *w = items[i].w;
            if ((w->dtype == 2) != (q5 == 1) || !w->rows) continue;
            smq::Item &it = a.item[a.nitems++];
            it.w = w->data;
            it.row_bytes = w->row_bytes;
            it.bias = items[i].bias;
            it.y = items[i].y;
            it.y_stride = w->rows;
            it.rows = w->rows;
            it.accumulate = items[i].accumulate != 0;
        }
        if (!a.nitems) continue;
        if (ntok > 1 && g.prefill_mfma && mfma_launch(a, q5 == 1)) {
            if (t_status != SMQ_OK) return t_status;
            continue;
        }
        if (!hip_ok(smq::launch_matmul(a, q5 == 1, g.fast != 0, g.cur), "matmul")) return t_status;
    }
    return SMQ_OK;
}

smq_status smq_gemv_grouped(const smq_group_item *items, uint32_t n) {
    if (!ready()) return t_status;
    if (!items || n < 1 || n > SMQ_MAX_GROUP) return set_status(SMQ_ERR_RANGE, "gemv_grouped: %u items", n);
    const smq_qmat *w0 = items[0].w;
    if (!w0) return set_status(SMQ_ERR_RANGE, "gemv_grouped: item 0 has no matrix");
    smq::GroupArgs ga;
    memset(&ga, 0, sizeof(ga));
    ga.nb = w0->nb;
    ga.flag = g.flag;
    for (uint32_t i = 0; i < n; ++i) {
        const smq_qmat *w = items[i].w;
        if (!w) return set_status(SMQ_ERR_RANGE, "gemv_grouped: item %u has no matrix", i);
        if (w->nb != ga.nb || w->dtype != w0->dtype)
            return set_status(SMQ_ERR_STATE, "gemv_grouped: items differ in width or format");
        if (w->dtype != 1 && w->dtype != 2) return set_status(SMQ_ERR_FORMAT, "gemv_grouped: dtype %u", w->dtype);
        if (w->nb != (w->cols + smq::QK - 1) / smq::QK)
            return set_status(SMQ_ERR_RANGE, "gemv_grouped: nb %u does not match %u columns", w->nb, w->cols);
        if (!check_operands(w->data, w->row_bytes, w->rows, w->nb, w->dtype == 2, items[i].xd, items[i].xq, 1, w->nb,
                            items[i].y, w->rows, "gemv_grouped") ||
            !extent_ok(items[i].bias, items[i].bias ? (size_t)w->rows * 4 : 0, "bias"))
            return t_status;
        smq::GroupItem &it = ga.item[ga.nitems++];
        it.w = w->data;
        it.row_bytes = w->row_bytes;
        it.bias = items[i].bias;
        it.y = items[i].y;
        it.xd = items[i].xd;
        it.xq = items[i].xq;
        it.rows = w->rows;
        it.accumulate = items[i].accumulate != 0;
    }
    const bool q5 = w0->dtype == 2;
    if (!smq::group_layout_ok(ga, q5)) {
        /* unaligned rows or activations, or very wide rows: one matmul per item */
        for (uint32_t i = 0; i < n; ++i) {
            smq_mat_item mi;
            mi.w = items[i].w;
            mi.bias = items[i].bias;
            mi.y = items[i].y;
            mi.accumulate = items[i].accumulate;
            const smq_status st = smq_matmul(&mi, 1, items[i].xd, items[i].xq, 1);
            if (st != SMQ_OK) return st;
        }
        return SMQ_OK;
    }
    return hip_ok(smq::launch_gemv_grouped(ga, q5, g.fast != 0, g.cur), "gemv_grouped") ? SMQ_OK : t_status;
}

struct smq_gemv_plan {
    smq::PlanWg *dev; /* one descriptor per workgroup, device memory owned by the plan */
    uint32_t wgs;
    int bp, device;
};

smq_status smq_gemv_plan_create(const smq_group_item *items, uint32_t n, smq_gemv_plan **plan) {
    if (!ready()) return t_status;
    if (!plan) return set_status(SMQ_ERR_RANGE, "gemv_plan_create: plan is NULL");
    *plan = nullptr;
    if (t_capturing) return set_status(SMQ_ERR_STATE, "gemv_plan_create: not under capture");
    if (!items || n < 1 || n > SMQ_MAX_PLAN_ITEMS)
        return set_status(SMQ_ERR_RANGE, "gemv_plan_create: %u items (1..%u)", n, (unsigned)SMQ_MAX_PLAN_ITEMS);
    std::vector<smq::GroupItem> its(n);
    std::vector<uint32_t> kind(n), tiles(n);
    std::vector<double> bytes(n);
    double total = 0.0;
    int bp = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const smq_qmat *w = items[i].w;
        if (!w) return set_status(SMQ_ERR_RANGE, "gemv_plan_create: item %u has no matrix", i);
        if (w->dtype != 1 || (w->nb != 28 && w->nb != 152) || w->nb != (w->cols + smq::QK - 1) / smq::QK ||
            w->row_bytes != (size_t)w->nb * smq::Q8_BYTES || ((uintptr_t)w->data & 15u) || !w->rows ||
            (((uintptr_t)items[i].xd | (uintptr_t)items[i].xq) & 3u))
            return set_status(SMQ_ERR_RANGE,
                              "gemv_plan_create: item %u: a plan takes packed, 16-byte aligned Q8 rows of 28 or 152 "
                              "blocks with 4-byte aligned activations",
                              i);
        if (!check_operands(w->data, w->row_bytes, w->rows, w->nb, false, items[i].xd, items[i].xq, 1, w->nb,
                            items[i].y, w->rows, "gemv_plan_create") ||
            !extent_ok(items[i].bias, items[i].bias ? (size_t)w->rows * 4 : 0, "bias"))
            return t_status;
        smq::GroupItem &it = its[i];
        memset(&it, 0, sizeof(it));
        it.w = w->data;
        it.row_bytes = w->row_bytes;
        it.bias = items[i].bias;
        it.y = items[i].y;
        it.xd = items[i].xd;
        it.xq = items[i].xq;
        it.rows = w->rows;
        it.accumulate = items[i].accumulate != 0;
        bp |= items[i].bias || items[i].accumulate;
        kind[i] = w->nb == 152;
        const uint32_t rt = smq::plan_rows_per_tile(kind[i] != 0);
        tiles[i] = (w->rows + rt - 1) / rt;
        bytes[i] = (double)w->rows * (double)w->row_bytes;
        total += bytes[i];
    }
    int per_cu = 0, cus = 0;
    if (!hip_ok(smq::plan_resident(per_cu), "gemv_plan_create") ||
        !hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g.device), "gemv_plan_create"))
        return t_status;
    /* every item a share of the resident workgroups in proportion to its bytes (at least one, at most
     * one per tile; largest remainders first, so the shares add up to the resident workgroups and
     * none waits for a second wave), each workgroup a contiguous tile range */
    const uint32_t resident = (uint32_t)per_cu * (uint32_t)(cus > 0 ? cus : 1);
    std::vector<uint32_t> share(n);
    std::vector<double> frac(n);
    uint64_t given = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const double q = (double)resident * bytes[i] / total;
        uint32_t k = (uint32_t)q;
        k = k < 1 ? 1 : (k > tiles[i] ? tiles[i] : k);
        share[i] = k;
        frac[i] = q - (double)(uint32_t)q;
        given += k;
    }
    while (given < resident) {
        uint32_t best = n;
        for (uint32_t i = 0; i < n; ++i)
            if (share[i] < tiles[i] && (best == n || frac[i] > frac[best])) best = i;
        if (best == n) break; /* every tile has its own workgroup */
        ++share[best];
        frac[best] = -1.0;
        ++given;
    }
    std::vector<smq::PlanWg> host;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t k = share[i];
        for (uint32_t j = 0; j < k; ++j) {
            smq::PlanWg d;
            memset(&d, 0, sizeof(d));
            d.item = its[i];
            d.t0 = (uint32_t)((uint64_t)tiles[i] * j / k);
            d.t1 = (uint32_t)((uint64_t)tiles[i] * (j + 1) / k);
            d.kind = kind[i];
            host.push_back(d);
        }
    }
    smq_gemv_plan *p = new (std::nothrow) smq_gemv_plan;
    if (!p) return set_status(SMQ_ERR_NOMEM, "gemv_plan_create: out of host memory");
    p->wgs = (uint32_t)host.size();
    p->bp = bp;
    p->device = g.device;
    p->dev = nullptr;
    const size_t nbytes = host.size() * sizeof(smq::PlanWg);
    if (!hip_ok(hipMalloc((void **)&p->dev, nbytes), "gemv_plan_create") ||
        !hip_ok(hipMemcpy(p->dev, host.data(), nbytes, hipMemcpyHostToDevice), "gemv_plan_create")) {
        if (p->dev) (void)hipFree(p->dev);
        delete p;
        return t_status;
    }
    *plan = p;
    return SMQ_OK;
}

smq_status smq_gemv_plan_launch(const smq_gemv_plan *plan) {
    if (!ready()) return t_status;
    if (!plan || !plan->dev) return set_status(SMQ_ERR_RANGE, "gemv_plan_launch: plan is NULL");
    if (plan->device != g.device)
        return set_status(SMQ_ERR_STATE, "gemv_plan_launch: plan made on device %d", plan->device);
    return hip_ok(smq::launch_gemv_plan(plan->dev, plan->wgs, g.fast != 0, plan->bp != 0, g.flag, g.cur),
                  "gemv_plan_launch")
               ? SMQ_OK
               : t_status;
}

void smq_gemv_plan_destroy(smq_gemv_plan *plan) {
    if (!plan) return;
    if (plan->dev) (void)hipFree(plan->dev);
    delete plan;
}

/* Validates a fused-call activation for matrices of `cols` columns. */
static bool act_ok(const smq_act *act, uint32_t cols, const char *who) {
    if (!act) {
        set_status(SMQ_ERR_RANGE, "%s: activation is NULL", who);
        return false;
    }
    if (act->cols != cols) {
        set_status(SMQ_ERR_RANGE, "%s: activation has %u columns, the matrices %u", who, act->cols, cols);
        return false;
    }
    const size_t nb = (cols + smq::QK - 1) / smq::QK;
    switch (act->kind) {
    case SMQ_ACT_Q8:
        return extent_ok(act->xd, nb * 4, "activation scales") && extent_ok(act->xq, nb * smq::QK, "activations");
    case SMQ_ACT_NORM:
        if (!extent_ok(act->norm, (size_t)cols * 4, "norm weights")) return false;
        /* fall through */
    case SMQ_ACT_F32:
        return extent_ok(act->x, (size_t)cols * 4, "x") &&
               extent_ok(act->xd_scratch, act->xd_scratch ? nb * 4 : 0, "scale scratch") &&
               extent_ok(act->xq_scratch, act->xq_scratch ? nb * smq::QK : 0, "value scratch");
    default:
        set_status(SMQ_ERR_RANGE, "%s: activation kind %d", who, act->kind);
        return false;
    }
}

/* The unfused form: the activation's Q8 blocks into (xd, xq). */
static bool act_materialize(const smq_act *act, const float **xd, const int8_t **xq, const char *who) {
    if (act->kind == SMQ_ACT_Q8) {
        *xd = act->xd;
        *xq = act->xq;
        return true;
    }
    if (!act->xd_scratch || !act->xq_scratch) {
        set_status(SMQ_ERR_RANGE, "%s: this shape needs the scratch buffers", who);
        return false;
    }
    const hipError_t e = act->kind == SMQ_ACT_NORM
                             ? smq::launch_row_quantize(act->x, act->norm, act->eps, nullptr, 0, 1, act->cols, nullptr,
                                                        act->xd_scratch, act->xq_scratch, g.flag, g.cur)
                             : smq::launch_quantize_q8(act->x, 1, act->cols, act->xd_scratch, act->xq_scratch, g.flag,
                                                       g.cur);
    if (!hip_ok(e, who)) return false;
    *xd = act->xd_scratch;
    *xq = act->xq_scratch;
    return true;
}

static void fused_act(smq::FusedArgs &f, const smq_act *act) {
    f.n = act->cols;
    f.src = act->x;
    f.norm = act->norm;
    f.eps = act->eps;
    f.xd = act->xd;
    f.xq = act->xq;
    f.flag = g.flag;
}

/* One launch of the fused kernel covers at most this many workgroup tiles
 * (about one resident wave): every workgroup repeats the prologue. */
static const uint32_t FUSED_MAX_TILES = 4096;
/* Rows x padded columns up to which an f32 activation is quantized in the matmul's own launch. */
static const uint64_t FUSED_F32_WORK = (uint64_t)1 << 20;

smq_status smq_matmul_act(const smq_mat_item *items, uint32_t n, const smq_act *act) {
    if (!ready()) return t_status;
    if (!items || n < 1 || n > SMQ_MAX_ITEMS) return set_status(SMQ_ERR_RANGE, "matmul_act: %u items", n);
    const uint32_t nb = items[0].w ? items[0].w->nb : 0, cols = items[0].w ? items[0].w->cols : 0;
    uint32_t total_rows = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const smq_qmat *w = items[i].w;
        if (!w) return set_status(SMQ_ERR_RANGE, "matmul_act: item %u has no matrix", i);
        if (w->nb != nb || w->cols != cols)
            return set_status(SMQ_ERR_STATE, "internal error: matmul inputs differ in width");
        if (w->dtype != 1 && w->dtype != 2) return set_status(SMQ_ERR_FORMAT, "matmul_act: dtype %u", w->dtype);
        if (w->nb != (w->cols + smq::QK - 1) / smq::QK)
            return set_status(SMQ_ERR_RANGE, "matmul_act: nb %u does not match %u columns", w->nb, w->cols);
        if (w->row_bytes < (size_t)w->nb * block_bytes(w->dtype == 2))
            return set_status(SMQ_ERR_RANGE, "matmul_act: row_bytes %zu < nb*%u", w->row_bytes,
                              block_bytes(w->dtype == 2));
        if (!extent_ok(w->data, w->rows ? (size_t)(w->rows - 1) * w->row_bytes + (size_t)w->nb * block_bytes(w->dtype == 2) : 0,
                       "weights") ||
            !extent_ok(items[i].y, (size_t)w->rows * 4, "output") ||
            !extent_ok(items[i].bias, items[i].bias ? (size_t)w->rows * 4 : 0, "bias"))
            return t_status;
        total_rows += w->rows;
    }
    if (!nb) return set_status(SMQ_ERR_RANGE, "matmul_act: nb is 0");
    if (!act_ok(act, cols, "matmul_act")) return t_status;
    if (!total_rows) return SMQ_OK;
    if (act->kind == SMQ_ACT_Q8) return smq_matmul(items, n, act->xd, act->xq, 1);
    /* fused: one launch per weight format present, each forming the activation itself */
    bool fused = true;
    smq::FusedArgs fa[2];
    for (int q5 = 0; q5 < 2; ++q5) {
        smq::FusedArgs &f = fa[q5];
        memset(&f, 0, sizeof(f));
        f.nb = nb;
        fused_act(f, act);
        uint32_t tiles = 0;
        for (uint32_t i = 0; i < n; ++i) {
            const smq_qmat *w = items[i].w;
            if ((w->dtype == 2) != (q5 == 1) || !w->rows) continue;
            smq::Item &it = f.item[f.nitems++];
            it.w = w->data;
            it.row_bytes = w->row_bytes;
            it.bias = items[i].bias;
            it.y = items[i].y;
            it.y_stride = w->rows;
            it.rows = w->rows;
            it.accumulate = items[i].accumulate != 0;
            tiles += w->rows; /* rows: an upper bound of the tiles */
        }
        /* every workgroup forms the activation: an f32 row is quantized once, apart, when the
         * repeated work would outweigh a launch (the down projection's 896 workgroups x 4864) */
        const uint64_t np = (uint64_t)nb * smq::QK;
        if (f.nitems && (g.fast || !smq::fused_layout_ok(f, q5 == 1, act->kind) || tiles / 8 > FUSED_MAX_TILES ||
                         (act->kind == SMQ_ACT_F32 && (uint64_t)tiles * np > FUSED_F32_WORK)))
            fused = false;
    }
    if (fused) {
        for (int q5 = 0; q5 < 2; ++q5) {
            if (!fa[q5].nitems) continue;
            const hipError_t e = smq::decode_ct_ok(fa[q5], q5 == 1, act->kind, false)
                                     ? smq::launch_decode_ct(fa[q5], act->kind, false, g.cur)
                                     : smq::launch_matmul_fused(fa[q5], q5 == 1, act->kind, false, g.cur);
            if (!hip_ok(e, "matmul_act")) return t_status;
        }
        return SMQ_OK;
    }
    const float *xd = nullptr;
    const int8_t *xq = nullptr;
    if (!act_materialize(act, &xd, &xq, "matmul_act")) return t_status;
    return smq_matmul(items, n, xd, xq, 1);
}

smq_status smq_matmul_glu_q8(const smq_qmat *gate, const smq_qmat *up, const smq_act *act, int glu, float *h,
                             float *hd, int8_t *hq, float *gate_scratch) {
    if (!ready()) return t_status;
    if (!gate || !up) return set_status(SMQ_ERR_RANGE, "matmul_glu_q8: NULL matrix");
    if (gate->rows != up->rows || gate->cols != up->cols || gate->nb != up->nb)
        return set_status(SMQ_ERR_STATE, "matmul_glu_q8: gate %ux%u and up %ux%u differ", gate->rows, gate->cols,
                          up->rows, up->cols);
    if (glu != 1 && glu != 2) return set_status(SMQ_ERR_RANGE, "matmul_glu_q8: activation %d", glu);
    const uint32_t hb = (up->rows + smq::QK - 1) / smq::QK;
    if (!extent_ok(h, h ? (size_t)up->rows * 4 : 0, "h") || !extent_ok(hd, (size_t)hb * 4, "hd") ||
        !extent_ok(hq, (size_t)hb * smq::QK, "hq"))
        return t_status;
    if (!gate->rows) return SMQ_OK;
    if (gate->dtype == 1 && up->dtype == 1 && act && act->cols == gate->cols && !g.fast &&
        gate->nb == (gate->cols + smq::QK - 1) / smq::QK) {
        smq::FusedArgs f;
        memset(&f, 0, sizeof(f));
        f.nb = gate->nb;
        fused_act(f, act);
        f.nitems = 2;
        for (int k = 0; k < 2; ++k) {
            const smq_qmat *w = k ? up : gate;
            f.item[k].w = w->data;
            f.item[k].row_bytes = w->row_bytes;
            f.item[k].rows = w->rows;
        }
        f.h = h;
        f.hd = hd;
        f.hq = hq;
        f.rows = gate->rows;
        f.act = glu;
        if (smq::decode_ct_ok(f, false, act->kind, true)) {
            for (int k = 0; k < 2; ++k) {
                const smq_qmat *w = k ? up : gate;
                if (!extent_ok(w->data, (size_t)(w->rows - 1) * w->row_bytes + (size_t)w->nb * smq::Q8_BYTES, "weights"))
                    return t_status;
            }
            if (!act_ok(act, gate->cols, "matmul_glu_q8")) return t_status;
            return hip_ok(smq::launch_decode_ct(f, act->kind, true, g.cur), "matmul_glu_q8") ? SMQ_OK : t_status;
        }
    }
    /* the two-step form: h, then its Q8 blocks */
    if (!h) return set_status(SMQ_ERR_RANGE, "matmul_glu_q8: this shape needs h");
    const smq_status st = smq_matmul_glu(gate, up, act, glu, h, gate_scratch);
    if (st != SMQ_OK) return st;
    return hip_ok(smq::launch_quantize_q8(h, 1, up->rows, hd, hq, g.flag, g.cur), "matmul_glu_q8") ? SMQ_OK
                                                                                                    : t_status;
}

smq_status smq_matmul_glu(const smq_qmat *gate, const smq_qmat *up, const smq_act *act, int glu, float *h,
                          float *gate_scratch) {
    if (!ready()) return t_status;
    if (!gate || !up) return set_status(SMQ_ERR_RANGE, "matmul_glu: NULL matrix");
    if (gate->rows != up->rows || gate->cols != up->cols || gate->nb != up->nb)
        return set_status(SMQ_ERR_STATE, "matmul_glu: gate %ux%u and up %ux%u differ", gate->rows, gate->cols,
                          up->rows, up->cols);
    if (glu != 1 && glu != 2) return set_status(SMQ_ERR_RANGE, "matmul_glu: activation %d", glu);
    if (!extent_ok(h, (size_t)up->rows * 4, "h")) return t_status;
    smq_mat_item it[2];
    it[0].w = gate;
    it[0].bias = nullptr;
    it[0].y = gate_scratch;
    it[0].accumulate = 0;
    it[1].w = up;
    it[1].bias = nullptr;
    it[1].y = h;
    it[1].accumulate = 0;
    if (gate->dtype == up->dtype && (gate->dtype == 1 || gate->dtype == 2) && act && act->cols == gate->cols &&
        gate->nb == (gate->cols + smq::QK - 1) / smq::QK) {
        smq::FusedArgs f;
        memset(&f, 0, sizeof(f));
        f.nb = gate->nb;
        fused_act(f, act);
        f.nitems = 2;
        for (int k = 0; k < 2; ++k) {
            const smq_qmat *w = k ? up : gate;
            f.item[k].w = w->data;
            f.item[k].row_bytes = w->row_bytes;
            f.item[k].rows = w->rows;
        }
        f.h = h;
        f.rows = gate->rows;
        f.act = glu;
        const bool q5 = gate->dtype == 2;
        if (!g.fast && act->kind == SMQ_ACT_NORM && smq::fused_layout_ok(f, q5, act->kind) &&
            gate->rows / 4 <= FUSED_MAX_TILES) {
            for (int k = 0; k < 2; ++k) {
                const smq_qmat *w = k ? up : gate;
                if (w->row_bytes < (size_t)w->nb * block_bytes(q5))
                    return set_status(SMQ_ERR_RANGE, "matmul_glu: row_bytes %zu < nb*%u", w->row_bytes, block_bytes(q5));
                if (!extent_ok(w->data, w->rows ? (size_t)(w->rows - 1) * w->row_bytes + (size_t)w->nb * block_bytes(q5) : 0,
                               "weights"))
                    return t_status;
            }
            if (!act_ok(act, gate->cols, "matmul_glu")) return t_status;
            if (!gate->rows) return SMQ_OK;
            return hip_ok(smq::launch_matmul_fused(f, q5, act->kind, true, g.cur), "matmul_glu")
                       ? SMQ_OK
                       : t_status;
        }
    }
    /* the two-call form: gate and up, then h = up * act(gate) */
    if (!gate_scratch) return set_status(SMQ_ERR_RANGE, "matmul_glu: this shape needs gate_scratch");
    const smq_status st = smq_matmul_act(it, 2, act);
    if (st != SMQ_OK) return st;
    return hip_ok(smq::launch_glu(h, gate_scratch, up->rows, glu, g.cur), "matmul_glu") ? SMQ_OK : t_status;
}

smq_status smq_numeric_check(void) {
    if (!ready()) return t_status;
    int bad = 0;
    if (!hip_ok(hipStreamSynchronize(g.cur), "numeric_check") ||
        !hip_ok(hipMemcpy(&bad, g.flag, sizeof(int), hipMemcpyDeviceToHost), "numeric_check"))
        return t_status;
    if (!bad) return SMQ_OK;
    if (!hip_ok(hipMemset(g.flag, 0, sizeof(int)), "numeric_check")) return t_status;
    /* the reference's message, model.c:309 */
    return set_status(SMQ_ERR_NUMERIC, "non-finite activation; the checkpoint is outside the supported numeric range");
}

static bool attn_shape(const smq_attn_shape *in, smq::AttnShape *out, const char *who) {
    if (!in) {
        set_status(SMQ_ERR_RANGE, "%s: shape is NULL", who);
        return false;
    }
    if (!in->heads || !in->kv_heads || in->heads % in->kv_heads || !in->head_dim || in->head_dim % 2 ||
        in->head_dim > smq::MAX_HEAD_DIM || 2 * in->rotary_pairs > in->head_dim || !in->context ||
        in->context > smq::MAX_ATT_POSITIONS) {
        set_status(SMQ_ERR_RANGE, "%s: unsupported shape (heads %u, kv_heads %u, head_dim %u <= %u, pairs %u, context %u <= %u)",
                   who, in->heads, in->kv_heads, in->head_dim, smq::MAX_HEAD_DIM, in->rotary_pairs, in->context,
                   smq::MAX_ATT_POSITIONS);
        return false;
    }
    out->heads = in->heads;
    out->kv_heads = in->kv_heads;
    out->head_dim = in->head_dim;
    out->q_dim = in->heads * in->head_dim;
    out->kv_dim = in->kv_heads * in->head_dim;
    out->pairs = in->rotary_pairs;
    out->window = in->window;
    out->context = in->context;
    return true;
}

smq_status smq_rope_kv(float *q, float *k, const float *v, uint32_t ntok, const smq_attn_shape *shape,
                       const float *cos_table, const float *sin_table, float *keys, float *values, uint32_t pos0,
                       const int32_t *pos_dev) {
    if (!ready()) return t_status;
    smq::AttnShape sh;
    if (!attn_shape(shape, &sh, "rope_kv")) return t_status;
    if (!ntok) return SMQ_OK;
    if (!pos_dev && (pos0 > sh.context || ntok > sh.context - pos0))
        return set_status(SMQ_ERR_RANGE, "token batch exceeds context"); /* model.c:667-668 */
    const size_t table = (size_t)sh.context * sh.pairs * 4, cache = (size_t)sh.context * sh.kv_dim * 4;
    if (!extent_ok(q, (size_t)ntok * sh.q_dim * 4, "q") || !extent_ok(k, (size_t)ntok * sh.kv_dim * 4, "k") ||
        !extent_ok(v, (size_t)ntok * sh.kv_dim * 4, "v") || !extent_ok(cos_table, table, "cos table") ||
        !extent_ok(sin_table, table, "sin table") || !extent_ok(keys, cache, "keys") ||
        !extent_ok(values, cache, "values") || !extent_ok(pos_dev, pos_dev ? 4 : 0, "pos"))
        return t_status;
    return hip_ok(smq::launch_rope_kv(q, k, v, ntok, sh, cos_table, sin_table, keys, values, pos0, pos_dev, g.flag,
                                      g.cur),
                  "rope_kv")
               ? SMQ_OK
               : t_status;
}

smq_status smq_attention(const float *q, const float *keys, const float *values, float *att, uint32_t ntok,
                         const smq_attn_shape *shape, uint32_t pos0, const int32_t *pos_dev) {
    if (!ready()) return t_status;
    smq::AttnShape sh;
    if (!attn_shape(shape, &sh, "attention")) return t_status;
    if (!ntok) return SMQ_OK;
    if (!pos_dev && (pos0 > sh.context || ntok > sh.context - pos0))
        return set_status(SMQ_ERR_RANGE, "token batch exceeds context");
    const size_t cache = (size_t)sh.context * sh.kv_dim * 4;
    if (!extent_ok(q, (size_t)ntok * sh.q_dim * 4, "q") || !extent_ok(att, (size_t)ntok * sh.q_dim * 4, "att") ||
        !extent_ok(keys, cache, "keys") || !extent_ok(values, cache, "values") ||
        !extent_ok(pos_dev, pos_dev ? 4 : 0, "pos"))
        return t_status;
    return hip_ok(smq::launch_attention(q, keys, values, att, ntok, sh, pos0, pos_dev, g.flag, nullptr, nullptr, g.cur,
                                        g.scores),
                  "attention")
               ? SMQ_OK
               : t_status;
}

smq_status smq_attention_q8(const float *q, const float *keys, const float *values, float *att, uint32_t ntok,
                            const smq_attn_shape *shape, uint32_t pos0, const int32_t *pos_dev, float *xd,
                            int8_t *xq) {
    if (!ready()) return t_status;
    smq::AttnShape sh;
    if (!attn_shape(shape, &sh, "attention_q8")) return t_status;
    if (!ntok) return SMQ_OK;
    if (!pos_dev && (pos0 > sh.context || ntok > sh.context - pos0))
        return set_status(SMQ_ERR_RANGE, "token batch exceeds context");
    const size_t cache = (size_t)sh.context * sh.kv_dim * 4, nbq = (sh.q_dim + smq::QK - 1) / smq::QK;
    if (!extent_ok(q, (size_t)ntok * sh.q_dim * 4, "q") || !extent_ok(att, (size_t)ntok * sh.q_dim * 4, "att") ||
        !extent_ok(keys, cache, "keys") || !extent_ok(values, cache, "values") ||
        !extent_ok(pos_dev, pos_dev ? 4 : 0, "pos") || !extent_ok(xd, ntok * nbq * 4, "xd") ||
        !extent_ok(xq, ntok * nbq * smq::QK, "xq"))
        return t_status;
    if (sh.head_dim % smq::QK == 0) /* each head owns whole blocks: quantized in the same kernel */
        return hip_ok(smq::launch_attention(q, keys, values, att, ntok, sh, pos0, pos_dev, g.flag, xd, xq, g.cur,
                                            g.scores),
                      "attention_q8")
                   ? SMQ_OK
                   : t_status;
    return hip_ok(smq::launch_attention(q, keys, values, att, ntok, sh, pos0, pos_dev, g.flag, nullptr, nullptr,
                                        g.cur, g.scores),
                  "attention_q8") &&
                   hip_ok(smq::launch_quantize_q8(att, ntok, sh.q_dim, xd, xq, g.flag, g.cur), "attention_q8")
               ? SMQ_OK
               : t_status;
}

smq_status smq_attention_rope_q8(float *q, float *k, const float *v, const smq_attn_shape *shape,
                                 const float *cos_table, const float *sin_table, float *keys, float *values,
                                 float *att, uint32_t pos0, const int32_t *pos_dev, float *xd, int8_t *xq) {
    if (!ready()) return t_status;
    smq::AttnShape sh;
    if (!attn_shape(shape, &sh, "attention_rope_q8")) return t_status;
    if (!pos_dev && pos0 >= sh.context) return set_status(SMQ_ERR_RANGE, "token batch exceeds context");
    const size_t table = (size_t)sh.context * sh.pairs * 4, cache = (size_t)sh.context * sh.kv_dim * 4;
    const size_t nbq = (sh.q_dim + smq::QK - 1) / smq::QK;
    if (!extent_ok(q, (size_t)sh.q_dim * 4, "q") || !extent_ok(k, (size_t)sh.kv_dim * 4, "k") ||
        !extent_ok(v, (size_t)sh.kv_dim * 4, "v") || !extent_ok(cos_table, table, "cos table") ||
        !extent_ok(sin_table, table, "sin table") || !extent_ok(keys, cache, "keys") ||
        !extent_ok(values, cache, "values") || !extent_ok(att, (size_t)sh.q_dim * 4, "att") ||
        !extent_ok(pos_dev, pos_dev ? 4 : 0, "pos") || !extent_ok(xd, nbq * 4, "xd") ||
        !extent_ok(xq, nbq * smq::QK, "xq"))
        return t_status;
    const bool aligned = !((uintptr_t)q & 15) && !((uintptr_t)k & 15) && !((uintptr_t)v & 15);
    if (aligned && smq::attention_rows_ok(sh, q, keys, values))
        return hip_ok(smq::launch_attention_rope(q, k, v, cos_table, sin_table, keys, values, att, sh, pos0, pos_dev,
                                                 g.flag, xd, xq, g.scores, g.cur),
                      "attention_rope_q8")
                   ? SMQ_OK
                   : t_status;
    /* other shapes: the two-step form (q and k are left rotated) */
    if (smq_rope_kv(q, k, v, 1, shape, cos_table, sin_table, keys, values, pos0, pos_dev) != SMQ_OK) return t_status;
    return smq_attention_q8(q, keys, values, att, 1, shape, pos0, pos_dev, xd, xq);
}

smq_status smq_matmul_act_rope(const smq_mat_item *items, const smq_act *act, const smq_attn_shape *shape,
                               const float *cos_table, const float *sin_table, float *keys, float *values,
                               uint32_t pos0, const int32_t *pos_dev) {
    if (!ready()) return t_status;
    smq::AttnShape sh;
    if (!attn_shape(shape, &sh, "matmul_act_rope")) return t_status;
    if (!items || !items[0].w || !items[1].w || !items[2].w)
        return set_status(SMQ_ERR_RANGE, "matmul_act_rope: items q, k and v need matrices");
    if (items[0].w->rows != sh.q_dim || items[1].w->rows != sh.kv_dim || items[2].w->rows != sh.kv_dim)
        return set_status(SMQ_ERR_RANGE, "matmul_act_rope: q, k, v rows %u, %u, %u against q_dim %u, kv_dim %u",
                          items[0].w->rows, items[1].w->rows, items[2].w->rows, sh.q_dim, sh.kv_dim);
    if (items[0].accumulate || items[1].accumulate || items[2].accumulate)
        return set_status(SMQ_ERR_RANGE, "matmul_act_rope: q, k and v do not accumulate");
    if (!pos_dev && pos0 >= sh.context) return set_status(SMQ_ERR_RANGE, "token batch exceeds context");
    const size_t table = (size_t)sh.context * sh.pairs * 4, cache = (size_t)sh.context * sh.kv_dim * 4;
    if (!extent_ok(cos_table, table, "cos table") || !extent_ok(sin_table, table, "sin table") ||
        !extent_ok(keys, cache, "keys") || !extent_ok(values, cache, "values") ||
        !extent_ok(pos_dev, pos_dev ? 4 : 0, "pos"))
        return t_status;
    const smq_qmat *w0 = items[0].w;
    bool fused = !g.fast && act && act->kind == SMQ_ACT_NORM && act_ok(act, w0->cols, "matmul_act_rope");
    for (uint32_t i = 0; i < 3 && fused; ++i) {
        const smq_qmat *w = items[i].w;
        fused = w->dtype == 1 && w->nb == w0->nb && w->cols == w0->cols && w->nb == (w->cols + smq::QK - 1) / smq::QK &&
                extent_ok(w->data, (size_t)(w->rows - 1) * w->row_bytes + (size_t)w->nb * smq::Q8_BYTES, "weights") &&
                extent_ok(items[i].y, (size_t)w->rows * 4, "output") &&
                extent_ok(items[i].bias, items[i].bias ? (size_t)w->rows * 4 : 0, "bias");
    }
    if (fused) {
        smq::FusedArgs f;
        memset(&f, 0, sizeof(f));
        f.nb = w0->nb;
        fused_act(f, act);
        for (uint32_t i = 0; i < 3; ++i) {
            smq::Item &it = f.item[f.nitems++];
            it.w = items[i].w->data;
            it.row_bytes = items[i].w->row_bytes;
            it.bias = items[i].bias;
            it.y = items[i].y;
            it.y_stride = items[i].w->rows;
            it.rows = items[i].w->rows;
        }
        f.rope.cs = cos_table;
        f.rope.sn = sin_table;
        f.rope.kcache = keys;
        f.rope.vcache = values;
        f.rope.pos_dev = pos_dev;
        f.rope.pos0 = pos0;
        f.rope.head_dim = sh.head_dim;
        f.rope.pairs = sh.pairs;
        f.rope.kv_dim = sh.kv_dim;
        f.rope.context = sh.context;
        if (smq::decode_ct_ok(f, false, act->kind, false))
            return hip_ok(smq::launch_decode_ct(f, act->kind, false, g.cur), "matmul_act_rope") ? SMQ_OK : t_status;
    }
    /* other layouts: the matmuls, then RoPE and the cache store (the same results) */
    if (smq_matmul_act(items, 3, act) != SMQ_OK) return t_status;
    return smq_rope_kv(items[0].y, items[1].y, items[2].y, 1, shape, cos_table, sin_table, keys, values, pos0,
                       pos_dev);
}

smq_status smq_argmax(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token) {
    if (!ready()) return t_status;
    if (!vocab) return set_status(SMQ_ERR_RANGE, "argmax: empty vocabulary");
    if (!extent_ok(logits, (size_t)vocab * 4, "logits") || !extent_ok(banned, banned ? vocab : 0, "banned") ||
        !extent_ok(token, 4, "token"))
        return t_status;
    return hip_ok(smq::launch_argmax(logits, vocab, banned, token, g.argmax_parts, nullptr, nullptr, nullptr, 0, g.cur),
                  "argmax")
               ? SMQ_OK
               : t_status;
}

smq_status smq_argmax_noalloc(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token) {
    if (!ready()) return t_status;
    if (!vocab) return set_status(SMQ_ERR_RANGE, "argmax_noalloc: empty vocabulary");
    if (vocab > smq::NOALLOC_MAX_VOCAB)
        return set_status(SMQ_ERR_RANGE, "argmax_noalloc: vocabulary of %u ids exceeds its static scratch (%u ids)",
                          vocab, smq::NOALLOC_MAX_VOCAB);
    void *parts = smq::noalloc_scratch(g.device);
    if (!parts) return set_status(SMQ_ERR_STATE, "argmax_noalloc: static scratch not bound on device %d", g.device);
    if (!extent_ok(logits, (size_t)vocab * 4, "logits") || !extent_ok(banned, banned ? vocab : 0, "banned") ||
        !extent_ok(token, 4, "token"))
        return t_status;
    return hip_ok(smq::launch_argmax(logits, vocab, banned, token, parts, nullptr, nullptr, nullptr, 0, g.cur),
                  "argmax_noalloc")
               ? SMQ_OK
               : t_status;
}

smq_status smq_argmax_advance(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token,
                              int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity) {
    if (!ready()) return t_status;
    if (!vocab) return set_status(SMQ_ERR_RANGE, "argmax: empty vocabulary");
    if (!extent_ok(logits, (size_t)vocab * 4, "logits") || !extent_ok(banned, banned ? vocab : 0, "banned") ||
        !extent_ok(token, 4, "token") || !extent_ok(pos, 4, "pos") || !extent_ok(count, 4, "count") ||
        !extent_ok(history, (size_t)capacity * 4, "history"))
        return t_status;
    if (!pos || !count || (capacity && !history)) return set_status(SMQ_ERR_RANGE, "argmax_advance: NULL argument");
    return hip_ok(smq::launch_argmax(logits, vocab, banned, token, g.argmax_parts, pos, count, history, capacity, g.cur),
                  "argmax_advance")
               ? SMQ_OK
               : t_status;
}

smq_status smq_argmax_advance_embed(const float *logits, uint32_t vocab, const unsigned char *banned, uint32_t *token,
                                    int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity,
                                    const smq_qmat *embed, float *x) {
    if (!ready()) return t_status;
    if (!vocab) return set_status(SMQ_ERR_RANGE, "argmax: empty vocabulary");
    if (!embed || (embed->dtype != 1 && embed->dtype != 2) || embed->nb != (embed->cols + smq::QK - 1) / smq::QK ||
        embed->row_bytes < (size_t)embed->nb * block_bytes(embed->dtype == 2))
        return set_status(SMQ_ERR_FORMAT, "argmax_advance_embed: invalid matrix descriptor");
    if (!extent_ok(logits, (size_t)vocab * 4, "logits") || !extent_ok(banned, banned ? vocab : 0, "banned") ||
        !extent_ok(token, 4, "token") || !extent_ok(pos, 4, "pos") || !extent_ok(count, 4, "count") ||
        !extent_ok(history, (size_t)capacity * 4, "history") ||
        !extent_ok(embed->data, (size_t)embed->rows * embed->row_bytes, "embed") ||
        !extent_ok(x, (size_t)embed->cols * 4, "x"))
        return t_status;
    if (!pos || !count || !x || (capacity && !history))
        return set_status(SMQ_ERR_RANGE, "argmax_advance_embed: NULL argument");
    const smq::EmbedArgs e = {embed->data, embed->row_bytes, embed->rows, embed->cols, embed->dtype == 2, x, g.flag};
    return hip_ok(smq::launch_argmax(logits, vocab, banned, token, g.argmax_parts, pos, count, history, capacity, g.cur,
                                     &e),
                  "argmax_advance_embed")
               ? SMQ_OK
               : t_status;
}

smq_status smq_embed(const smq_qmat *embed, const uint32_t *tokens, uint32_t ntok, float *x) {
    if (!ready()) return t_status;
    if (!embed || (embed->dtype != 1 && embed->dtype != 2) || embed->nb != (embed->cols + smq::QK - 1) / smq::QK ||
        embed->row_bytes < (size_t)embed->nb * block_bytes(embed->dtype == 2))
        return set_status(SMQ_ERR_FORMAT, "embed: invalid matrix descriptor");
    if (!ntok) return SMQ_OK;
    if (!extent_ok(embed->data, (size_t)embed->rows * embed->row_bytes, "embed") ||
        !extent_ok(tokens, (size_t)ntok * 4, "tokens") || !extent_ok(x, (size_t)ntok * embed->cols * 4, "x"))
        return t_status;
    return hip_ok(smq::launch_embed(embed->data, embed->row_bytes, embed->dtype == 2, embed->rows, tokens, ntok,
                                    embed->cols, x, g.flag, g.cur),
                  "embed")
               ? SMQ_OK
               : t_status;
}

smq_status smq_decode_advance(int32_t *pos, uint32_t *count, const uint32_t *token, uint32_t *history,
                              uint32_t capacity) {
    if (!ready()) return t_status;
    if (!extent_ok(pos, 4, "pos") || !extent_ok(count, 4, "count") || !extent_ok(token, 4, "token") ||
        !extent_ok(history, (size_t)capacity * 4, "history"))
        return t_status;
    return hip_ok(smq::launch_decode_advance(pos, count, token, history, capacity, g.cur), "decode_advance")
               ? SMQ_OK
               : t_status;
}

smq_status smq_quantize_q5_rows(const float *x, uint32_t rows, uint32_t cols, unsigned char *out) {
    if (!ready()) return t_status;
    if (!rows || !cols) return SMQ_OK;
    const size_t row_out = (size_t)((cols + smq::QK - 1) / smq::QK) * smq::Q5_BYTES;
    if (!extent_ok(x, (size_t)rows * cols * 4, "x") || !extent_ok(out, (size_t)rows * row_out, "out"))
        return t_status;
    return hip_ok(smq::launch_quantize_q5(x, rows, cols, out, g.cur), "quantize_q5") ? SMQ_OK : t_status;
}

void smq_quantize_q5_row(const float *x, uint32_t cols, unsigned char *out) { (void)smq_quantize_q5_rows(x, 1, cols, out); }

void smq_dequantize_q8_row(const unsigned char *w, uint32_t cols, float *out) {
    if (!ready()) return;
    const uint32_t nb = (cols + smq::QK - 1) / smq::QK;
    if (!extent_ok(w, (size_t)nb * smq::Q8_BYTES, "w") || !extent_ok(out, (size_t)cols * 4, "out")) return;
    hip_ok(smq::launch_dequantize_row(w, cols, out, false, g.cur), "dequantize_q8_row");
}

void smq_dequantize_q5_row(const unsigned char *w, uint32_t cols, float *out) {
    if (!ready()) return;
    const uint32_t nb = (cols + smq::QK - 1) / smq::QK;
    if (!extent_ok(w, (size_t)nb * smq::Q5_BYTES, "w") || !extent_ok(out, (size_t)cols * 4, "out")) return;
    hip_ok(smq::launch_dequantize_row(w, cols, out, true, g.cur), "dequantize_q5_row");
}

void *smq_malloc(size_t bytes) {
    if (!ready()) return nullptr;
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    g_allocs[(uintptr_t)p] = bytes ? bytes : 1;
    return p;
}

void smq_free(void *p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lock(g_alloc_mu);
        g_allocs.erase((uintptr_t)p);
    }
    (void)hipFree(p);
}

smq_status smq_memcpy_htod(void *dst, const void *src, size_t bytes) {
    if (!ready()) return t_status;
    if (!bytes) return SMQ_OK;
    if (!extent_ok(dst, bytes, "dst")) return t_status;
    if (!hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.cur), "memcpy htod") ||
        !hip_ok(hipStreamSynchronize(g.cur), "memcpy htod"))
        return t_status;
    return SMQ_OK;
}

smq_status smq_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    if (!ready()) return t_status;
    if (!bytes) return SMQ_OK;
    if (!extent_ok(src, bytes, "src")) return t_status;
    if (!hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.cur), "memcpy dtoh") ||
        !hip_ok(hipStreamSynchronize(g.cur), "memcpy dtoh"))
        return t_status;
    return SMQ_OK;
}

smq_status smq_memcpy_dtod(void *dst, const void *src, size_t bytes) {
    if (!ready()) return t_status;
    if (!bytes) return SMQ_OK;
    if (!extent_ok(src, bytes, "src") || !extent_ok(dst, bytes, "dst")) return t_status;
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g.cur), "memcpy dtod") ? SMQ_OK : t_status;
}

smq_status smq_memset(void *dst, int value, size_t bytes) {
    if (!ready()) return t_status;
    if (!bytes) return SMQ_OK;
    if (!extent_ok(dst, bytes, "dst")) return t_status;
    return hip_ok(hipMemsetAsync(dst, value, bytes, g.cur), "memset") ? SMQ_OK : t_status;
}

smq_status smq_capture_begin(void) {
    if (!ready()) return t_status;
    if (g.cur != g.own) return set_status(SMQ_ERR_STATE, "capture needs the library stream");
    /* thread-local mode: a call from this thread that may not be captured (a synchronizing copy, an
     * allocation) fails the capture instead of being recorded or run behind the graph's back */
    if (!hip_ok(hipStreamBeginCapture(g.cur, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"))
        return t_status;
    t_capturing = true;
    return SMQ_OK;
}

void *smq_capture_end(void) {
    if (!ready()) return nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    t_capturing = false;
    if (!hip_ok(hipStreamEndCapture(g.cur, &graph), "hipStreamEndCapture")) return nullptr;
    const bool ok = hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(graph);
    return ok ? (void *)exec : nullptr;
}

smq_status smq_graph_launch(void *graph) {
    if (!ready()) return t_status;
    if (!graph) return set_status(SMQ_ERR_RANGE, "graph is NULL");
    return hip_ok(hipGraphLaunch((hipGraphExec_t)graph, g.cur), "hipGraphLaunch") ? SMQ_OK : t_status;
}

void smq_graph_destroy(void *graph) {
    if (graph) (void)hipGraphExecDestroy((hipGraphExec_t)graph);
}

static bool anchor_shape_ok(const void *a, const void *b, size_t bytes, uint32_t wgs, uint32_t threads) {
    if (((uintptr_t)a | (uintptr_t)b | bytes) & 15u) {
        set_status(SMQ_ERR_RANGE, "stream: buffers and size must be 16-byte aligned");
        return false;
    }
    if (!wgs || threads < 64 || threads > 1024 || threads % 64) {
        set_status(SMQ_ERR_RANGE, "stream: grid %u x %u", wgs, threads);
        return false;
    }
    return true;
}

smq_status smq_stream_read(const void *p, size_t bytes, uint32_t workgroups, uint32_t threads, int nontemporal,
                           uint32_t *sink) {
    if (!ready()) return t_status;
    if (!anchor_shape_ok(p, nullptr, bytes, workgroups, threads)) return t_status;
    if (!extent_ok(p, bytes, "stream source") || !extent_ok(sink, 4, "sink")) return t_status;
    return hip_ok(smq::launch_stream_read(p, bytes, workgroups, threads, nontemporal != 0, sink, g.cur),
                  "stream_read")
               ? SMQ_OK
               : t_status;
}

smq_status smq_stream_copy(void *dst, const void *src, size_t bytes, uint32_t workgroups, uint32_t threads,
                           int nontemporal) {
    if (!ready()) return t_status;
    if (!anchor_shape_ok(dst, src, bytes, workgroups, threads)) return t_status;
    if (!extent_ok(src, bytes, "stream source") || !extent_ok(dst, bytes, "stream destination")) return t_status;
    return hip_ok(smq::launch_stream_copy(dst, src, bytes, workgroups, threads, nontemporal != 0, g.cur),
                  "stream_copy")
               ? SMQ_OK
               : t_status;
}

smq_status smq_grid_barrier_probe(uint32_t workgroups, uint32_t episodes, uint32_t kind, double *ms) {
    if (!ready()) return t_status;
    if (t_capturing) return set_status(SMQ_ERR_RANGE, "grid_barrier_probe: not under capture");
    int cus = 0;
    if (!hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g.device), "grid_barrier_probe"))
        return t_status;
    if (!workgroups || workgroups > (uint32_t)cus || workgroups > 1024 || episodes > 100000 || kind > 2 || !ms)
        return set_status(SMQ_ERR_RANGE, "grid_barrier_probe: %u workgroups (1..%d), %u episodes, kind %u", workgroups,
                          cus, episodes, kind);
    static uint32_t *words[64];
    if (g.device < 0 || g.device >= 64) return set_status(SMQ_ERR_RANGE, "grid_barrier_probe: device %d", g.device);
    if (!words[g.device] &&
        !hip_ok(hipMalloc((void **)&words[g.device], smq::GRID_BARRIER_WORDS * 4), "grid_barrier_probe"))
        return t_status;
    uint32_t *w = words[g.device];
    float t = 0.0f;
    uint32_t timed_out = 0;
    if (!hip_ok(hipEventRecord(g.t0, g.cur), "grid_barrier_probe") ||
        !hip_ok(smq::launch_grid_barrier(w, workgroups, episodes, kind, g.cur), "grid_barrier_probe") ||
        !hip_ok(hipEventRecord(g.t1, g.cur), "grid_barrier_probe") ||
        !hip_ok(hipEventSynchronize(g.t1), "grid_barrier_probe") ||
        !hip_ok(hipEventElapsedTime(&t, g.t0, g.t1), "grid_barrier_probe") ||
        !hip_ok(hipMemcpy(&timed_out, w + smq::GRID_BARRIER_TIMEOUTS, 4, hipMemcpyDeviceToHost), "grid_barrier_probe"))
        return t_status;
    if (timed_out)
        return set_status(SMQ_ERR_STATE, "grid_barrier_probe: %u workgroups gave up a wait", timed_out);
    *ms = (double)t;
    return SMQ_OK;
}

smq_status smq_timer_start(void) {
    if (!ready()) return t_status;
    return hip_ok(hipEventRecord(g.t0, g.cur), "timer") ? SMQ_OK : t_status;
}

double smq_timer_stop(void) {
    if (!ready()) return -1.0;
    float ms = 0.0f;
    if (!hip_ok(hipEventRecord(g.t1, g.cur), "timer") || !hip_ok(hipEventSynchronize(g.t1), "timer") ||
        !hip_ok(hipEventElapsedTime(&ms, g.t0, g.t1), "timer"))
        return -1.0;
    return (double)ms;
}

}  // extern "C"
