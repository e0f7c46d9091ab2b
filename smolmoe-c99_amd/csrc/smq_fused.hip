/* Fused decode GEMV (one token) for gfx950: the activation producer of the
 * reference's decode step (model.c:334-415) run as the prologue of the
 * matmul that consumes it, and the gated product of a gate/up pair run as
 * its store (vecmath.c:78-93). */
#include <float.h>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

/* ------------------------------------------------------------------------
 * Fused decode GEMV (one token): the activation is formed inside the
 * launch, and for a gate/up pair the gated product is formed in the store.
 *  PRO_NORM  RMSNorm of the f32 row src with weights norm (model.c:334-342:
 *            squares in parallel, their sum in element order by one lane,
 *            inv = 1/sqrtf(sum/n + eps), (x*inv)*w) and its Q8 blocks
 *            (kernels.c:912-935), computed by every workgroup for itself;
 *  PRO_F32   the Q8 blocks of the f32 row src.
 *  EPI_STORE each item's rows: + bias, finiteness, y or y += (as k_gemv);
 *  EPI_GLU   items 0 and 1 are gate and up with the same rows; a workgroup
 *            owns RT/2 rows of each and stores h[r] = up[r] * (g / (1 +
 *            exp_det(-g))) (SwiGLU) or the GeGLU form (vecmath.c:78-93).
 * Every workgroup issues its first weight loads during the prologue (after
 * the RMSNorm's serial sum), and the prologue's barriers wait for LDS only,
 * so the weight fetch overlaps the activation's quantization. Products, chains
 * and the lane tree are those of k_gemv (exact per-lane order).
 * ---------------------------------------------------------------------- */
constexpr int PRO_NORM = 1, PRO_F32 = 2; /* SMQ_ACT_NORM, SMQ_ACT_F32 */
constexpr uint32_t FU_BATCH = 32; /* activation elements per thread of the widest RMSNorm row */
static_assert(FU_BATCH * WG == MAX_NORM_K, "the widest RMSNorm row");
constexpr uint32_t FU_SHORT = 8;  /* elements per thread loaded ahead of the weights (rows up to 2048) */
constexpr int EPI_STORE = 0, EPI_GLU = 1;

/* A workgroup barrier that orders LDS only: this thread's LDS accesses are
 * complete, global loads may stay in flight (s_barrier without the release
 * fence of __syncthreads, which would wait for them). */
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t find_fused_item(const FusedArgs &a, uint32_t tile) {
    uint32_t it = 0;
    if (a.nitems > 1 && tile >= a.item[1].tile_begin) it = 1;
    if (a.nitems > 2 && tile >= a.item[2].tile_begin) it = 2;
    if (a.nitems > 3 && tile >= a.item[3].tile_begin) it = 3;
    return it;
}

template <bool Q5, bool FAST, int RT, int PRO, int EPI>
__global__ __launch_bounds__(WG) void k_gemv_fused(FusedArgs a, uint32_t ntiles) {
    constexpr int TB = Q5 ? 2 : 1;    /* blocks per task */
    constexpr int TPR = WG / RT;      /* tasks per row per chunk */
    constexpr int CB = TPR * TB;      /* blocks per chunk */
    constexpr int GS = RT * 32 + 4;   /* floats per group of four blocks */
    constexpr int DS = RT * 4 + 4;    /* fast mode: scales per group */
    constexpr int NW = Q5 ? 11 : 9;   /* weight dwords per task */
    static_assert(EPI != EPI_GLU || (RT % 2 == 0 && RT * 8 <= 64), "gate/up slots share wave 0");
    __shared__ __attribute__((aligned(16))) float prod[2][(CB / 4) * GS];
    __shared__ __attribute__((aligned(16))) float dsc[FAST ? 2 : 1][FAST ? (CB / 4) * DS : 4];
    __shared__ float s_inv;
    __shared__ int s_bad;
    extern __shared__ __attribute__((aligned(16))) uint32_t dyn[];

    const uint32_t nb = a.nb, tid = threadIdx.x, np = nb * QK, n = a.n;
    const uint32_t n4 = PRO == PRO_NORM ? (n + 3) & ~3u : 0u;
    float *sq = (float *)dyn, *xs = sq + n4, *ws = xs + n4; /* PRO_NORM: squares, x, weights */
    uint32_t *act_q = dyn + 3 * n4;
    float *act_d = (float *)(act_q + nb * 8);
    int *act_b = (int *)(act_d + nb); /* Q5: -16 * lane sums of x */

    /* this workgroup's tiles: a contiguous range (the grid is at most one resident wave) */
    const uint32_t t0 = (uint32_t)((uint64_t)ntiles * blockIdx.x / gridDim.x);
    const uint32_t t1 = (uint32_t)((uint64_t)ntiles * (blockIdx.x + 1) / gridDim.x);
    if (t0 >= t1) return;
    /* this thread's weight row in a tile */
    const uint32_t tr = tid / TPR, ti = tid % TPR;
    struct Row {
        const unsigned char *w;
        size_t row_bytes;
        bool ok;
        uint32_t item, r0;
    };
    auto setup = [&](uint32_t tile, Row &R) __attribute__((always_inline)) {
        R.item = 0;
        R.r0 = 0;
        if (EPI == EPI_GLU) {
            constexpr uint32_t half = RT / 2 > 0 ? RT / 2 : 1;
            const uint32_t row = tile * half + tr % half;
            const Item &I = a.item[tr < half ? 0 : 1];
            R.ok = row < a.rows;
            R.row_bytes = I.row_bytes;
            R.w = I.w + (size_t)(R.ok ? row : 0) * R.row_bytes;
        } else {
            R.item = find_fused_item(a, tile);
            const Item &I = a.item[R.item];
            R.r0 = (tile - I.tile_begin) * RT;
            R.ok = R.r0 + tr < I.rows;
            R.row_bytes = I.row_bytes;
            R.w = I.w + (size_t)(R.ok ? R.r0 + tr : 0) * R.row_bytes;
        }
    };
    const uint32_t nchunks = (nb + CB - 1) / CB;
    uint32_t wr[NW] = {};
    auto load_task = [&](const Row &R, uint32_t b) __attribute__((always_inline)) {
        if (R.ok && b < nb) {
            const unsigned char *p = R.w + (size_t)b * (Q5 ? Q5_BYTES : Q8_BYTES);
            const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
            wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
            wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
            if constexpr (Q5) {
                const u3a v2 = *(const u3a *)(p + 32);
                wr[8] = v2.x; wr[9] = v2.y; wr[10] = v2.z;
            } else {
                wr[8] = *(const uint32_t *)(p + 32);
            }
        }
    };
    Row cur, nxt;
    setup(t0, cur);

    /* prologue: the activation into LDS. Rows of up to FU_SHORT elements per thread load x (and
     * the norm weights) before the first weight loads are issued: loads complete in order, so
     * the prologue waits for its own loads only. Wider rows load in batches of FU_SHORT per
     * thread inside a loop. The f32 form issues the weight loads right after its x loads. */
    static_assert(PRO == PRO_NORM || PRO == PRO_F32, "a given Q8 activation takes k_gemv");
    const uint32_t ke = (np + WG - 1) / WG; /* NORM: <= FU_BATCH (n <= MAX_NORM_K) */
    const bool short_row = ke <= FU_SHORT;
    float xv[FU_SHORT], wv[FU_SHORT];
    if (short_row) {
#pragma unroll
        for (uint32_t k = 0; k < FU_SHORT; ++k) {
            const uint32_t i = tid + k * WG;
            xv[k] = k < ke && i < n ? a.src[i] : 0.0f;
            if (PRO == PRO_NORM) wv[k] = k < ke && i < n ? a.norm[i] : 0.0f;
        }
    }
    if (PRO != PRO_NORM) load_task(cur, ti * TB);
    {
        int bad = 0;
        int8_t *q8 = (int8_t *)act_q;
        if (PRO == PRO_NORM) {
            /* x, w and the squares to LDS; then the sum in order; then (x*inv)*w */
            if (short_row) {
#pragma unroll
                for (uint32_t k = 0; k < FU_SHORT; ++k) {
                    const uint32_t i = tid + k * WG;
                    if (k < ke && i < n) {
                        sq[i] = xv[k] * xv[k];
                        xs[i] = xv[k];
                        ws[i] = wv[k];
                    }
                }
            } else {
                for (uint32_t k0 = 0; k0 < ke; k0 += FU_SHORT) {
#pragma unroll
                    for (uint32_t k = 0; k < FU_SHORT; ++k) {
                        const uint32_t i = tid + (k0 + k) * WG;
                        xv[k] = i < n ? a.src[i] : 0.0f;
                        wv[k] = i < n ? a.norm[i] : 0.0f;
                    }
#pragma unroll
                    for (uint32_t k = 0; k < FU_SHORT; ++k) {
                        const uint32_t i = tid + (k0 + k) * WG;
                        if (i < n) {
                            sq[i] = xv[k] * xv[k];
                            xs[i] = xv[k];
                            ws[i] = wv[k];
                        }
                    }
                }
            }
            lds_barrier();
            if (tid < 64) { /* the whole first wave runs the chain; lane 63 ends with the total */
                const float ss = serial_sum_wave(sq, n);
                if (tid == 63) {
                    const float iv = 1.0f / sqrtf(ss / (float)n + a.eps); /* model.c:338 */
                    s_inv = iv;
                    s_bad = !(fabsf(ss) <= FLT_MAX) || !(fabsf(iv) <= FLT_MAX);
                }
            }
            lds_barrier();
            load_task(cur, ti * TB); /* after the serial sum (measured faster than before it) */
            const float inv = s_inv;
            if (tid == 0 && s_bad && a.flag) *a.flag = 1;
            /* (x*inv)*w and its Q8 blocks; uniform: a block's 32 lanes are all below np or past it */
            auto stage = [&](uint32_t k) __attribute__((always_inline)) {
                const uint32_t i = tid + k * WG;
                if (i < np) {
                    const bool valid = i < n;
                    float v = 0.0f;
                    if (valid) {
                        const float t = xs[i] * inv;
                        v = t * ws[i]; /* model.c:340 */
                    }
                    stage_q8(v, valid, i, q8, act_d, bad);
                }
            };
            if (short_row) {
#pragma unroll
                for (uint32_t k = 0; k < FU_SHORT; ++k)
                    if (k < ke) stage(k);
            } else {
                for (uint32_t k = 0; k < ke; ++k) stage(k);
            }
        } else if (short_row) {
#pragma unroll
            for (uint32_t k = 0; k < FU_SHORT; ++k) {
                const uint32_t i = tid + k * WG;
                if (k < ke && i < np) stage_q8(xv[k], i < n, i, q8, act_d, bad); /* uniform per block */
            }
        } else {
            for (uint32_t k0 = 0; k0 < ke; k0 += FU_SHORT) {
#pragma unroll
                for (uint32_t k = 0; k < FU_SHORT; ++k) {
                    const uint32_t i = tid + (k0 + k) * WG;
                    xv[k] = i < n ? a.src[i] : 0.0f;
                }
#pragma unroll
                for (uint32_t k = 0; k < FU_SHORT; ++k) {
                    const uint32_t i = tid + (k0 + k) * WG;
                    if (i < np) stage_q8(xv[k], i < n, i, q8, act_d, bad); /* uniform per block */
                }
            }
        }
        if (bad && a.flag) *a.flag = 1;
    }
    if (Q5) {
        lds_barrier();
        for (uint32_t i = tid; i < nb * 8; i += WG) act_b[i] = dot4(act_q[i], 0xf0f0f0f0u, 0); /* int8 0xf0 = -16 */
    }
    lds_barrier(); /* activation staged */

    uint32_t step = 0; /* products buffer parity */
    for (uint32_t tile = t0; tile < t1; ++tile) {
        if (tile + 1 < t1) setup(tile + 1, nxt);
        float acc = 0.0f;
        for (uint32_t c = 0; c < nchunks; ++c, ++step) {
            const uint32_t bt = c * CB + ti * TB;
            uint32_t cw[NW];
#pragma unroll
            for (int k = 0; k < NW; ++k) cw[k] = wr[k];
            if (c + 1 < nchunks) load_task(cur, bt + CB); /* the next chunk, or the next tile's first, in flight */
            else if (tile + 1 < t1) load_task(nxt, ti * TB);
            float *pb = prod[step & 1];
            if (cur.ok && bt < nb) {
                Q5Fields f[2];
                if (Q5) q5_parse_pair(cw, f[0], f[1]);
#pragma unroll
                for (int k = 0; k < TB; ++k) {
                    const uint32_t b = bt + k, bb = ti * TB + k;
                    const float wscale = Q5 ? f[k].scale : __uint_as_float(cw[0]);
                    const float d = wscale * act_d[b];
                    float *dst = pb + (bb / 4) * GS + tr * 32 + (bb % 4);
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        const uint32_t x = act_q[b * 8 + l];
                        int sv;
                        if (Q5) sv = dot4(q5_codes(f[k], l), x, act_b[b * 8 + l]);
                        else sv = dot4(cw[1 + l], x, 0);
                        dst[l * 4] = FAST ? (float)sv : d * (float)sv;
                    }
                    if (FAST) dsc[step & 1][(bb / 4) * DS + tr * 4 + (bb % 4)] = d;
                }
            }
            __syncthreads();
            if (tid < RT * 8) {
                const uint32_t count = nb - c * CB < (uint32_t)CB ? nb - c * CB : (uint32_t)CB;
                chain_sum<FAST, CB / 4>(acc, (const float4 *)pb + tid, GS / 4,
                                        FAST ? (const float4 *)dsc[step & 1] + tid / 8 : nullptr, DS / 4, count);
            }
        }

        if (EPI == EPI_GLU) {
            if (tid < 64) { /* every row slot is in wave 0 */
                const float v = reduce8_to_lane7(acc);
                const float u = __shfl_down(v, RT * 4, 64); /* up slot tr + RT/2 */
                const uint32_t row = tile * (RT / 2 > 0 ? RT / 2 : 1) + tid / 8;
                if ((tid & 7) == 7 && tid < RT * 4 && row < a.rows) {
                    const float gv = v;
                    if (a.flag && (!(fabsf(gv) <= FLT_MAX) || !(fabsf(u) <= FLT_MAX))) *a.flag = 1; /* model.c:309 */
                    float e;
                    if (a.act == 2) {
                        const float g3 = 0.044715f * gv * gv * gv;
                        const float uu = 1.5957691216f * (gv + g3);
                        e = exp_det(-uu);
                    } else {
                        e = exp_det(-gv);
                    }
                    const float den = 1.0f + e;
                    const float sg = gv / den;
                    a.h[row] = u * sg;
                }
            }
        } else if (tid < RT * 8) {
            const float v = reduce8_to_lane7(acc);
            const Item &I = a.item[cur.item];
            const uint32_t r = cur.r0 + tid / 8;
            if ((tid & 7) == 7 && r < I.rows) store_out(I, a.flag, 0, r, v);
        }
        cur = nxt;
    }
}

/* Dynamic LDS limit of every k_gemv_fused instance, raised once at smq_init (before any
 * capture) to the widest row fused_layout_ok admits: 3 x MAX_NORM_K RMSNorm floats plus
 * MAX_FAST_NB Q5 blocks of 17 floats. */
constexpr size_t FUSED_MAX_LDS = (3 * (size_t)MAX_NORM_K + (size_t)MAX_FAST_NB * 17u) * 4u;
static_assert(FUSED_MAX_LDS <= 160u * 1024u, "within one CU's LDS");

template <bool Q5, int RT, int PRO, int EPI>
hipError_t launch_fused_rt(FusedArgs a, hipStream_t s) {
    uint32_t tiles = 0;
    if (EPI == EPI_GLU) {
        constexpr uint32_t half = RT / 2 > 0 ? RT / 2 : 1;
        tiles = (a.rows + half - 1) / half;
    } else {
        for (uint32_t i = 0; i < a.nitems; ++i) {
            a.item[i].tile_begin = tiles;
            tiles += (a.item[i].rows + RT - 1) / RT;
        }
    }
    if (!tiles) return hipSuccess;
    const size_t lds = ((PRO == PRO_NORM ? 3 * ((a.n + 3) / 4 * 4) : 0) + (size_t)a.nb * (Q5 ? 17u : 9u)) * 4u;
    if (lds > FUSED_MAX_LDS) return hipErrorInvalidValue; /* past the limit prepare_fused_attributes set */
    /* at most one resident wave of workgroups, each taking a range of tiles: the prologue runs
     * once per workgroup (the occupancy of this instantiation is read at the widest LDS seen) */
    static size_t queried_lds = 0;
    static int resident = 0;
    if (lds > queried_lds) {
        int per_cu = 0, dev = 0, cus = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_gemv_fused<Q5, false, RT, PRO, EPI>,
                                                                    WG, lds);
        if (e == hipSuccess) e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        resident = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
        queried_lds = lds;
    }
    const uint32_t grid = tiles < (uint32_t)resident ? tiles : (uint32_t)resident;
    hipLaunchKernelGGL((k_gemv_fused<Q5, false, RT, PRO, EPI>), dim3(grid), dim3(WG), lds, s, a, tiles);
    return hipGetLastError();
}

template <bool Q5, int RT, int PRO, int EPI>
hipError_t raise_fused_lds() { /* at most what the CU holds beside the kernel's static LDS */
    const void *fn = (const void *)k_gemv_fused<Q5, false, RT, PRO, EPI>;
    hipFuncAttributes at;
    const hipError_t e = hipFuncGetAttributes(&at, fn);
    if (e != hipSuccess) return e;
    const size_t room = (size_t)160 * 1024 - at.sharedSizeBytes;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(FUSED_MAX_LDS < room ? FUSED_MAX_LDS : room));
}

template <bool Q5>
hipError_t raise_fused_lds_typed() {
    const hipError_t es[] = {raise_fused_lds<Q5, 2, PRO_NORM, EPI_GLU>(),  raise_fused_lds<Q5, 4, PRO_NORM, EPI_GLU>(),
                             raise_fused_lds<Q5, 8, PRO_NORM, EPI_GLU>(),  raise_fused_lds<Q5, 1, PRO_NORM, EPI_STORE>(),
                             raise_fused_lds<Q5, 2, PRO_NORM, EPI_STORE>(), raise_fused_lds<Q5, 4, PRO_NORM, EPI_STORE>(),
                             raise_fused_lds<Q5, 8, PRO_NORM, EPI_STORE>(), raise_fused_lds<Q5, 1, PRO_F32, EPI_STORE>(),
                             raise_fused_lds<Q5, 2, PRO_F32, EPI_STORE>(),  raise_fused_lds<Q5, 4, PRO_F32, EPI_STORE>(),
                             raise_fused_lds<Q5, 8, PRO_F32, EPI_STORE>()};
    for (hipError_t e : es)
        if (e != hipSuccess) return e;
    return hipSuccess;
}

template <bool Q5, int PRO, int EPI>
hipError_t launch_fused_pe(const FusedArgs &a, int rt, hipStream_t s) {
    if constexpr (EPI == EPI_GLU) { /* two to eight rows: a gate/up pair per slot, all slots in wave 0 */
        switch (rt) {
        case 1:
        case 2: return launch_fused_rt<Q5, 2, PRO, EPI_GLU>(a, s);
        case 4: return launch_fused_rt<Q5, 4, PRO, EPI_GLU>(a, s);
        default: return launch_fused_rt<Q5, 8, PRO, EPI_GLU>(a, s);
        }
    } else {
    switch (rt) {
    case 1: return launch_fused_rt<Q5, 1, PRO, EPI_STORE>(a, s);
    case 2: return launch_fused_rt<Q5, 2, PRO, EPI_STORE>(a, s);
    case 4: return launch_fused_rt<Q5, 4, PRO, EPI_STORE>(a, s);
    default: return launch_fused_rt<Q5, 8, PRO, EPI_STORE>(a, s);
    }
    }
}

template <bool Q5>
hipError_t launch_fused_typed(const FusedArgs &a, int pro, bool glu, hipStream_t s) {
    const int rt = gemv_rows_per_tile(a.nb, Q5, 0);
    if (glu) /* the dense FFN's form: RMSNorm prologue */
        return pro == PRO_NORM ? launch_fused_pe<Q5, PRO_NORM, EPI_GLU>(a, rt, s) : hipErrorInvalidValue;
    if (pro == PRO_NORM) return launch_fused_pe<Q5, PRO_NORM, EPI_STORE>(a, rt, s);
    if (pro == PRO_F32) return launch_fused_pe<Q5, PRO_F32, EPI_STORE>(a, rt, s);
    return hipErrorInvalidValue; /* a given Q8 activation is smq_matmul's case */
}

}  // namespace

bool fused_layout_ok(const FusedArgs &a, bool q5, int pro) {
    if (!a.nb || a.nb > MAX_FAST_NB || (q5 && (a.nb & 1u))) return false;
    if (a.n > a.nb * QK || a.n + QK <= a.nb * QK) return false;
    if (pro == 1 && a.n > MAX_NORM_K) return false;
    if (pro == 0 && (((uintptr_t)a.xq | (uintptr_t)a.xd) & 3u)) return false;
    for (uint32_t i = 0; i < a.nitems; ++i)
        if ((((uintptr_t)a.item[i].w) | a.item[i].row_bytes) & 3u) return false;
    return true;
}

hipError_t prepare_fused_attributes() {
    const hipError_t e = raise_fused_lds_typed<false>();
    return e != hipSuccess ? e : raise_fused_lds_typed<true>();
}

hipError_t launch_matmul_fused(const FusedArgs &a, bool q5, int pro, bool glu, hipStream_t s) {
    return q5 ? launch_fused_typed<true>(a, pro, glu, s) : launch_fused_typed<false>(a, pro, glu, s);
}

}  // namespace smq
