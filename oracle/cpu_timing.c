/* CPU-baseline timing driver (test infrastructure only; loaded by the
 * benchmark's cpu_baseline leg and by the tests, never by the GPU product).
 *
 * Runs a GemmQ8-shaped function (kernels.h:60-65) the way the reference's
 * forward pass does: rows of each matrix split statically with split_range
 * (threadpool.h:19-23) across a fixed pool whose caller is worker 0
 * (threadpool.c:293-309), one matrix after another, each thread writing its
 * row slice of out[t * rows + r] (model.c:252-279). Workers spin on a
 * generation counter between matrices, as the reference pool does before it
 * sleeps (threadpool.c:195-212). */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <time.h>

#include "smq_oracle.h"

typedef struct Pass {
    orc_gemm_fn gemm;
    const unsigned char *const *mats;
    const uint32_t *rows, *nbs;
    const float *const *xds;
    const int8_t *const *xqs;
    uint32_t nmats, ntok, threads, block_bytes;
    float *out;
    unsigned char *scratch;
    size_t scratch_bytes;
    uint32_t generation, stop, arrived;
} Pass;

typedef struct Worker {
    Pass *pass;
    uint32_t index;
} Worker;

static double now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Spin with a pause hint, then yield: the reference pool's SPIN_LIMIT of
 * 20000 (threadpool.c:94) before it gives up the core. */
static void relax(uint32_t *spins) {
    if (++*spins < 20000u) {
#if defined(__x86_64__) || defined(__i386__)
        __builtin_ia32_pause();
#endif
    } else {
        sched_yield();
    }
}

static void run_slice(Pass *p, uint32_t index, uint32_t m) {
    uint32_t begin, end, nb = p->nbs[m];
    size_t row_bytes = (size_t)nb * p->block_bytes;
    unsigned char *scratch = p->scratch ? p->scratch + (size_t)index * p->scratch_bytes : NULL;
    orc_split_range(p->rows[m], index, p->threads, &begin, &end);
    if (begin < end)
        p->gemm(p->mats[m] + (size_t)begin * row_bytes, row_bytes, p->xds[m], p->xqs[m], end - begin, p->ntok, nb,
                p->out + begin, p->rows[m], scratch);
}

/* Every thread runs every matrix of one pass, with a spin barrier between
 * matrices (the next matrix's input depends on the previous one in a real
 * forward pass, so no thread may run ahead). */
static void run_pass(Pass *p, uint32_t index, uint32_t *barrier_gen) {
    uint32_t m;
    for (m = 0; m < p->nmats; ++m) {
        uint32_t target, spins = 0;
        run_slice(p, index, m);
        target = ++*barrier_gen * p->threads;
        __atomic_add_fetch(&p->arrived, 1u, __ATOMIC_ACQ_REL);
        while (__atomic_load_n(&p->arrived, __ATOMIC_ACQUIRE) < target) relax(&spins);
    }
}

static void *worker_main(void *arg) {
    Worker *w = (Worker *)arg;
    Pass *p = w->pass;
    uint32_t seen = 0, barrier_gen = 0;
    for (;;) {
        uint32_t g, spins = 0;
        while ((g = __atomic_load_n(&p->generation, __ATOMIC_ACQUIRE)) == seen) relax(&spins);
        seen = g;
        if (__atomic_load_n(&p->stop, __ATOMIC_ACQUIRE)) return NULL;
        run_pass(p, w->index, &barrier_gen);
    }
}

double orc_time_gemm_pass(orc_gemm_fn gemm, const unsigned char *const *mats, const uint32_t *rows,
                          const uint32_t *nbs, const float *const *xds, const int8_t *const *xqs, uint32_t nmats,
                          uint32_t ntok, uint32_t block_bytes, float *out, uint32_t threads, uint32_t reps,
                          size_t scratch_bytes, double *times) {
    Pass p;
    pthread_t th[256];
    Worker wk[256];
    uint32_t i, rep, barrier_gen = 0;
    double best = 1e300;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    p.gemm = gemm;
    p.mats = mats;
    p.rows = rows;
    p.nbs = nbs;
    p.xds = xds;
    p.xqs = xqs;
    p.nmats = nmats;
    p.ntok = ntok;
    p.block_bytes = block_bytes;
    p.threads = threads;
    p.out = out;
    p.scratch_bytes = scratch_bytes;
    p.scratch = scratch_bytes ? (unsigned char *)calloc(threads, scratch_bytes) : NULL;
    p.generation = 0;
    p.stop = 0;
    p.arrived = 0;
    for (i = 1; i < threads; ++i) {
        wk[i].pass = &p;
        wk[i].index = i;
        if (pthread_create(&th[i], NULL, worker_main, &wk[i]) != 0) {
            threads = i; /* run with the threads that started */
            break;
        }
    }
    p.threads = threads;
    for (rep = 0; rep < reps; ++rep) {
        double t0 = now(), dt;
        __atomic_add_fetch(&p.generation, 1u, __ATOMIC_ACQ_REL);
        run_pass(&p, 0, &barrier_gen);
        dt = now() - t0;
        if (times) times[rep] = dt;
        if (dt < best) best = dt;
    }
    __atomic_store_n(&p.stop, 1u, __ATOMIC_RELEASE);
    __atomic_add_fetch(&p.generation, 1u, __ATOMIC_ACQ_REL);
    for (i = 1; i < threads; ++i) pthread_join(th[i], NULL);
    free(p.scratch);
    return best;
}

void orc_gemm_q8_fn(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    orc_gemm(0, 0, w, row_bytes, xd, xq, nrows, ntok, nb, out, stride);
}

void orc_gemm_q5_fn(const unsigned char *w, size_t row_bytes, const float *xd, const int8_t *xq, uint32_t nrows,
                    uint32_t ntok, uint32_t nb, float *out, size_t stride, unsigned char *scratch) {
    (void)scratch;
    orc_gemm(1, 0, w, row_bytes, xd, xq, nrows, ntok, nb, out, stride);
}
