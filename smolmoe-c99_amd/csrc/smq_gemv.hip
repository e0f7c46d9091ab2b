/* Coalesced-tile decode GEMV for Q8 rows of 36*nb bytes with nb % 4 == 0
 * (every row a whole number of 16-byte pieces) at 16-byte aligned row
 * starts; built for the 896-wide rows (nb 28) of the Qwen2.5-0.5B gate, up,
 * q, k, v and o matrices and the LM head.
 *
 * Arithmetic (src/kernels.c:36-79): for row r, block b, lane l the exact int32
 * sum s = w[b][4l..4l+3] . x[b][4l..4l+3] (v_dot4), the product
 * p = (wscale_b * xscale_b) * float(s) (two roundings; fast mode one fmaf),
 * acc_l = acc_l + p over b in increasing order, then
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
 *
 * Layout. A tile is RT consecutive rows, i.e. RT*36*nb contiguous bytes; each
 * thread loads fixed 16-byte pieces of it (piece tid + j*CT_NT), so every
 * load instruction of a wave reads 1 KiB of consecutive bytes, marked
 * non-temporal (the weights are read once). A row is 9*nb dwords: dword k is
 * field k % 9 of block k / 9 (field 0 the f32 scale, field 1 + l the four
 * int8 of lane l). The tile shape repeats every step, so each thread knows
 * once, for each of its dwords, the activation word it meets (the block's x
 * scale for field 0, x's lane-l word otherwise) and where its result goes in
 * LDS: a scale dword stores d = wscale * xscale into d[r][b], a lane dword
 * stores float(s) into sf[r][l][b] (exact: |s| < 2^24). After one barrier,
 * chain thread (r, l) forms p = d[r][b] * sf[r][l][b] and adds it in block
 * order, the eight lanes of a row meet in the DPP lane tree, and lane 7
 * stores (bias, finiteness, residual add as the other decode kernels). Two
 * LDS buffers alternate, and the next D tiles' loads stay in flight.
 */
#include <float.h>
#include <stddef.h>

#include <type_traits>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t CT_NT = 512;

template <class GA>
__device__ __forceinline__ uint32_t find_ct_item(const GA &g, uint32_t wg) {
    uint32_t lo = 0, hi = g.nitems; /* last item with wg_begin <= wg */
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (g.item[mid].wg_begin <= wg) lo = mid;
        else hi = mid;
    }
    return lo;
}

/* One step's LDS: lane sums sf[r][l][b] (pitch SP floats per (r, l)), block scale products
 * d[r][b] (pitch SP per row), and a sink for the writes of pieces past the tile. */
template <uint32_t RT, uint32_t SP>
struct CtBuf {
    float sf[RT * 8 * SP];
    float d[RT * SP];
    float sink[64];
};

/* LDS pitch of a tile's rows: a multiple of four floats (16-byte chain reads) that is 4 mod 32, so
 * the lane sums of one block's eight lanes (stored 8 pitches apart by one write) fall in distinct
 * banks, and the eight chain lanes of a row read distinct 16-byte bank groups (measured: a pitch of
 * 32 floats, where those writes collide, cost 7 %) */
template <uint32_t NB>
constexpr uint32_t ct_pitch() { return (NB + 3) / 4 * 4 + (36 - (NB + 3) / 4 * 4 % 32) % 32; }

/* Tiles t0..t1-1 (t1 > t0) of item I, RT rows each, through the two LDS buffers `buf`. */
template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT, uint32_t D>
__device__ __forceinline__ void ct_tiles(const GroupItem &I, uint32_t t0, uint32_t t1, int *flag,
                                         CtBuf<RT, ct_pitch<NB>()> (&buf)[2]) {
    static_assert(NB % 4 == 0, "rows of whole 16-byte pieces");
    constexpr uint32_t C16 = 9 * NB / 4;       /* 16-byte pieces per row */
    constexpr uint32_t TCH = RT * C16;         /* pieces per tile */
    constexpr uint32_t SP = ct_pitch<NB>();
    static_assert(SP % 32 == 4 && SP >= NB, "pitch 4 mod 32");
    constexpr uint32_t NQ = NB / 4;
    static_assert(TCH <= CPT * CT_NT, "each piece of a tile has a thread slot");
    using Buf = CtBuf<RT, SP>;

    const uint32_t tid = threadIdx.x;
    const uint32_t rows = I.rows;
    const uint32_t my_steps = t1 - t0;
    const unsigned char *wbase = I.w;
    const size_t row_bytes = I.row_bytes;
    const float *bias_p = I.bias, *xd = I.xd;
    float *y = I.y;
    const bool accum = I.accumulate != 0;

    /* this thread's piece slots j: piece c = tid + j*CT_NT of a tile (row c / C16, 16-byte
     * piece c % C16 of it); per dword q the activation word it meets and its LDS target */
    uint32_t xw[CPT][4], dst[CPT][4], prow[CPT], poff[CPT], scale_mask = 0;
    const uint32_t *xq32 = (const uint32_t *)I.xq;
#pragma unroll
    for (uint32_t j = 0; j < CPT; ++j) {
        const uint32_t c = tid + j * CT_NT, cc = c < TCH ? c : 0, r = cc / C16, pc = cc % C16;
        prow[j] = r;
        poff[j] = 16 * pc;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t k = 4 * pc + q, b = k / 9, f = k % 9;
            const uint32_t sw = __float_as_uint(xd[b]), lw = xq32[8 * b + (f ? f - 1 : 0)];
            xw[j][q] = f == 0 ? sw : lw;
            if (f == 0) scale_mask |= 1u << (4 * j + q);
            const uint32_t at = f == 0 ? (uint32_t)(offsetof(Buf, d) / 4) + r * SP + b
                                       : (uint32_t)(offsetof(Buf, sf) / 4) + (r * 8 + f - 1) * SP + b;
            dst[j][q] = c < TCH ? at : (uint32_t)(offsetof(Buf, sink) / 4) + (tid & 63u);
        }
    }

    /* a tile's bytes, coalesced and non-temporal; rows past the matrix re-read its last row (in
     * bounds, never stored), so every thread issues the same loads at every step. A step past this
     * workgroup's range re-reads its own last tile (bytes it has just read, not the next workgroup's
     * first tile: that was 5 % more HBM reads, measured) */
    auto load = [&](u4a (&w)[CPT], uint32_t tile) __attribute__((always_inline)) {
        const uint32_t tc = tile < t1 ? tile : t1 - 1; /* t1 > t0: every workgroup has a tile */
        const uint32_t last = (rows - tc * RT < RT ? rows - tc * RT : RT) - 1;
        const unsigned char *base = wbase + (size_t)tc * RT * row_bytes;
#pragma unroll
        for (uint32_t j = 0; j < CPT; ++j) {
            const uint32_t r = prow[j] < last ? prow[j] : last;
            w[j] = __builtin_nontemporal_load((const u4a *)(base + (size_t)r * row_bytes + poff[j]));
        }
    };
    /* chain thread (row cr, lane cl): its row's bias and prior output (BP: some item of the launch
     * has a bias or adds into y; otherwise no such loads at all, so the only loads in flight are
     * the tiles' and each step waits for its own tile only) */
    const uint32_t cr = tid / 8, cl = tid % 8;
    auto load_bp = [&](float &bias, float &prior, uint32_t tile) __attribute__((always_inline)) {
        if constexpr (!BP) {
            bias = 0.0f;
            prior = 0.0f;
            return;
        }
        const uint32_t orow = tile * RT + (cr < RT ? cr : 0), oc = orow < rows ? orow : rows - 1;
        bias = *(bias_p ? bias_p + oc : xd);
        prior = *(accum ? y + oc : xd);
    };

    u4a W[D][CPT];
    float B[D], P[D];
#pragma unroll
    for (uint32_t j = 0; j < D; ++j) {
        load(W[j], t0 + j);
        load_bp(B[j], P[j], t0 + j);
    }
    /* D steps per trip with no early exit (a straight trip keeps the in-flight tiles in their
     * registers); a step past the range computes and does not store. Every trip but the last
     * requests the next tiles; the last trip requests nothing (no re-read of bytes already read) */
    auto trip = [&](uint32_t k, auto next) __attribute__((always_inline)) {
        constexpr bool NEXT = decltype(next)::value;
#pragma unroll
        for (uint32_t j = 0; j < D; ++j) {
            const uint32_t step = k + j, tile = t0 + step;
            const bool live = step < my_steps;
            float *lb = (float *)&buf[step & 1];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (uint32_t c = 0; c < CPT; ++c) {
                const uint32_t wv[4] = {W[j][c].x, W[j][c].y, W[j][c].z, W[j][c].w};
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    const float fs = (float)dot4(wv[q], xw[c][q], 0);
                    const float dv = __uint_as_float(wv[q]) * __uint_as_float(xw[c][q]);
                    lb[dst[c][q]] = (scale_mask >> (4 * c + q)) & 1u ? dv : fs;
                }
            }
            if constexpr (NEXT) load(W[j], tile + D); /* consumed: the next tile for these registers */
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            if (tid < RT * 8) {
                const Buf &bb = buf[step & 1];
                const float4 *sp = (const float4 *)&bb.sf[(cr * 8 + cl) * SP];
                const float4 *dp = (const float4 *)&bb.d[cr * SP];
                float acc = 0.0f;
#pragma unroll 7
                for (uint32_t qq = 0; qq < NQ; ++qq) {
                    const float4 sv = sp[qq], dv = dp[qq];
                    if (FAST) {
                        acc = __builtin_fmaf(dv.x, sv.x, acc);
                        acc = __builtin_fmaf(dv.y, sv.y, acc);
                        acc = __builtin_fmaf(dv.z, sv.z, acc);
                        acc = __builtin_fmaf(dv.w, sv.w, acc);
                    } else {
                        float p;
                        p = dv.x * sv.x; acc = acc + p;
                        p = dv.y * sv.y; acc = acc + p;
                        p = dv.z * sv.z; acc = acc + p;
                        p = dv.w * sv.w; acc = acc + p;
                    }
                }
                const float v = reduce8_to_lane7(acc);
                const uint32_t row = tile * RT + cr;
                if (live && cl == 7 && row < rows) {
                    float o = v;
                    if (bias_p) o = o + B[j]; /* model.c:259-262 */
                    if (flag && !(fabsf(o) <= FLT_MAX)) *flag = 1;
                    if (accum) o = P[j] + o;
                    y[row] = o;
                }
            }
            if constexpr (NEXT) load_bp(B[j], P[j], tile + D);
        }
    };
    uint32_t k = 0;
    for (; k + D < my_steps; k += D) trip(k, std::true_type{});
    trip(k, std::false_type{}); /* my_steps >= 1: the last trip */
}

template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT, uint32_t D, class GA>
__global__ __launch_bounds__(CT_NT) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gemv_ct(GA g) {
    __shared__ __attribute__((aligned(16))) CtBuf<RT, ct_pitch<NB>()> buf[2];
    const GroupItem &I = g.item[find_ct_item(g, blockIdx.x)];
    const uint32_t tiles = (I.rows + RT - 1) / RT, wg = blockIdx.x - I.wg_begin;
    const uint32_t t0 = (uint32_t)((uint64_t)tiles * wg / I.nwg), t1 = (uint32_t)((uint64_t)tiles * (wg + 1) / I.nwg);
    ct_tiles<FAST, BP, NB, RT, CPT, D>(I, t0, t1, g.flag, buf);
}

/* Wide rows (nb > CK_KC, 152 blocks = the 4864-wide down projection): the same coalesced pieces
 * over K chunks of CK_KC blocks. A step is RT rows x one chunk (RT*9*CK_KC/4 contiguous-per-row
 * pieces); the chain thread (row, lane) keeps its sum in a register across the chunks of a tile,
 * so every lane chain still adds its row's blocks 0..nb-1 in order, and the lane tree and store
 * follow the last chunk. The item's activation is staged once in LDS in the rows' own layout
 * (dword 9b = block b's scale, 9b + 1.. its 32 int8), so the four dwords of a piece meet the four
 * activation words of one 16-byte LDS read. */
constexpr uint32_t CK_KC = 32;

constexpr uint32_t CK_SP = CK_KC + (36 - CK_KC % 32) % 32; /* LDS pitch of a chunk's rows */

/* Tiles t0..t1-1 (t1 > t0) of item I, RT rows each, K chunk by K chunk, through the two LDS buffers
 * `buf`; `act` holds the item's activation in the rows' layout. */
template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT>
__device__ __forceinline__ void ck_tiles(const GroupItem &I, uint32_t t0, uint32_t t1, int *flag,
                                         CtBuf<RT, CK_SP> (&buf)[2], uint32_t (&act)[NB * 9]) {
    constexpr uint32_t KC = CK_KC;
    constexpr uint32_t NCH = (NB + KC - 1) / KC;    /* chunks per row */
    constexpr uint32_t KL = NB - (NCH - 1) * KC;    /* blocks of the last chunk */
    static_assert(NB % 4 == 0 && NB > KC && KL % 4 == 0, "whole 16-byte pieces in every chunk");
    constexpr uint32_t P = 9 * KC / 4, PL = 9 * KL / 4; /* pieces per row of a chunk, of the last */
    constexpr uint32_t TCH = RT * P;
    constexpr uint32_t SP = CK_SP;
    static_assert(SP % 32 == 4 && SP >= KC, "pitch 4 mod 32");
    static_assert(TCH <= CPT * CT_NT, "each piece of a step has a thread slot");
    using Buf = CtBuf<RT, SP>;

    const uint32_t tid = threadIdx.x;
    const uint32_t rows = I.rows;
    const uint32_t my_steps = (t1 - t0) * NCH;
    const unsigned char *wbase = I.w;
    const size_t row_bytes = I.row_bytes;
    const float *bias_p = I.bias, *xd = I.xd;
    float *y = I.y;
    const bool accum = I.accumulate != 0;

    /* slot j: piece c = tid + j*CT_NT of a step (row c / P, piece c % P of the row's chunk);
     * its dwords' LDS targets in a full chunk and in the last one (pieces past it go to the sink) */
    uint32_t prow[CPT], ppc[CPT], dst[CPT][4], dstl[CPT][4], scale_mask = 0;
#pragma unroll
    for (uint32_t j = 0; j < CPT; ++j) {
        const uint32_t c = tid + j * CT_NT, cc = c < TCH ? c : 0, r = cc / P, pc = cc % P;
        prow[j] = r;
        ppc[j] = pc;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t k = 4 * pc + q, b = k / 9, f = k % 9;
            if (f == 0) scale_mask |= 1u << (4 * j + q);
            const uint32_t at = f == 0 ? (uint32_t)(offsetof(Buf, d) / 4) + r * SP + b
                                       : (uint32_t)(offsetof(Buf, sf) / 4) + (r * 8 + f - 1) * SP + b;
            const uint32_t sink = (uint32_t)(offsetof(Buf, sink) / 4) + (tid & 63u);
            dst[j][q] = c < TCH ? at : sink;
            dstl[j][q] = c < TCH && pc < PL ? at : sink;
        }
    }

    /* step s = (tile t0 + s / NCH, chunk s % NCH); rows past the matrix re-read its last row and
     * pieces past the last chunk its last piece (in bounds, never stored) */
    auto load = [&](u4a (&w)[CPT], uint32_t step) __attribute__((always_inline)) {
        const uint32_t tile = t0 + step / NCH, ch = step % NCH;
        const uint32_t last = (rows - tile * RT < RT ? rows - tile * RT : RT) - 1;
        const unsigned char *base = wbase + (size_t)tile * RT * row_bytes + (size_t)ch * KC * Q8_BYTES;
#pragma unroll
        for (uint32_t j = 0; j < CPT; ++j) {
            const uint32_t r = prow[j] < last ? prow[j] : last;
            const uint32_t pc = ch == NCH - 1 && ppc[j] >= PL ? PL - 1 : ppc[j];
            w[j] = __builtin_nontemporal_load((const u4a *)(base + (size_t)r * row_bytes + 16 * pc));
        }
    };
    const uint32_t cr = tid / 8, cl = tid % 8;
    auto load_bp = [&](float &bias, float &prior, uint32_t tile) __attribute__((always_inline)) {
        if constexpr (BP) {
            const uint32_t orow = tile * RT + (cr < RT ? cr : 0), oc = orow < rows ? orow : rows - 1;
            bias = *(bias_p ? bias_p + oc : xd);
            prior = *(accum ? y + oc : xd);
        }
    };

    /* the activation's words, all requested first (loads complete in order, so storing them waits
     * for nothing later; a loop of load-then-store after the first tile's loads waited one memory
     * round trip per iteration, each also taking the tile's loads) */
    constexpr uint32_t AW = (NB * 9 + CT_NT - 1) / CT_NT;
    uint32_t av[AW];
    {
        const uint32_t *xq32 = (const uint32_t *)I.xq;
#pragma unroll
        for (uint32_t k = 0; k < AW; ++k) {
            const uint32_t i = tid + k * CT_NT, ic = i < NB * 9 ? i : 0, b = ic / 9, f = ic % 9;
            av[k] = *(f == 0 ? (const uint32_t *)xd + b : xq32 + 8 * b + f - 1);
        }
    }
    float B = 0.0f, Pr = 0.0f;
    load_bp(B, Pr, t0);
    u4a W[CPT];
    load(W, 0);
#pragma unroll
    for (uint32_t k = 0; k < AW; ++k)
        if (tid + k * CT_NT < NB * 9) act[tid + k * CT_NT] = av[k];
    __syncthreads();

    float acc = 0.0f;
    for (uint32_t s = 0; s < my_steps; ++s) {
        const uint32_t ch = s % NCH, tile = t0 + s / NCH;
        const bool lastc = ch == NCH - 1;
        float *lb = (float *)&buf[s & 1];
#pragma unroll
        for (uint32_t j = 0; j < CPT; ++j) {
            const uint32_t pc = lastc && ppc[j] >= PL ? PL - 1 : ppc[j];
            const u4a A = *(const u4a *)&act[ch * 9 * KC + 4 * pc];
            const uint32_t wv[4] = {W[j].x, W[j].y, W[j].z, W[j].w}, av[4] = {A.x, A.y, A.z, A.w};
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                const float fs = (float)dot4(wv[q], av[q], 0);
                const float dv = __uint_as_float(wv[q]) * __uint_as_float(av[q]);
                lb[lastc ? dstl[j][q] : dst[j][q]] = (scale_mask >> (4 * j + q)) & 1u ? dv : fs;
            }
        }
        /* the next tile's bias and prior (older than the next weights, so no extra wait), then the
         * next step's weights into the registers just consumed */
        float Bn = B, Pn = Pr;
        if (lastc && tid < RT * 8 && s + 1 < my_steps) load_bp(Bn, Pn, tile + 1);
        if (s + 1 < my_steps) load(W, s + 1);
        __syncthreads();
        if (tid < RT * 8) {
            const Buf &bb = buf[s & 1];
            const float4 *sp = (const float4 *)&bb.sf[(cr * 8 + cl) * SP];
            const float4 *dp = (const float4 *)&bb.d[cr * SP];
            const uint32_t nq = (lastc ? KL : KC) / 4;
#pragma unroll
            for (uint32_t qq = 0; qq < KC / 4; ++qq) {
                if (qq < nq) { /* uniform */
                    const float4 sv = sp[qq], dv = dp[qq];
                    if (FAST) {
                        acc = __builtin_fmaf(dv.x, sv.x, acc);
                        acc = __builtin_fmaf(dv.y, sv.y, acc);
                        acc = __builtin_fmaf(dv.z, sv.z, acc);
                        acc = __builtin_fmaf(dv.w, sv.w, acc);
                    } else {
                        float p;
                        p = dv.x * sv.x; acc = acc + p;
                        p = dv.y * sv.y; acc = acc + p;
                        p = dv.z * sv.z; acc = acc + p;
                        p = dv.w * sv.w; acc = acc + p;
                    }
                }
            }
            if (lastc) {
                const float v = reduce8_to_lane7(acc);
                const uint32_t row = tile * RT + cr;
                if (cl == 7 && row < rows) {
                    float o = v;
                    if (bias_p) o = o + B; /* model.c:259-262 */
                    if (flag && !(fabsf(o) <= FLT_MAX)) *flag = 1;
                    if (accum) o = Pr + o;
                    y[row] = o;
                }
                acc = 0.0f;
            }
        }
        B = Bn;
        Pr = Pn;
    }
}

template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT, class GA>
__global__ __launch_bounds__(CT_NT) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gemv_ck(GA g) {
    __shared__ __attribute__((aligned(16))) CtBuf<RT, CK_SP> buf[2];
    __shared__ __attribute__((aligned(16))) uint32_t act[NB * 9];
    const GroupItem &I = g.item[find_ct_item(g, blockIdx.x)];
    const uint32_t tiles = (I.rows + RT - 1) / RT, wg = blockIdx.x - I.wg_begin;
    const uint32_t t0 = (uint32_t)((uint64_t)tiles * wg / I.nwg), t1 = (uint32_t)((uint64_t)tiles * (wg + 1) / I.nwg);
    ck_tiles<FAST, BP, NB, RT, CPT>(I, t0, t1, g.flag, buf, act);
}

/* A planned launch (smq_gemv_plan): one workgroup per descriptor, each a contiguous tile range of
 * one item, 28-block items on the coalesced tiles and 152-block items on the K chunks, in one
 * launch. The descriptor is read at a uniform address (scalar loads, one round trip); the two
 * forms share the LDS. */
constexpr uint32_t PLAN_CT_RT = 8, PLAN_CK_RT = 14;
union PlanLds {
    CtBuf<PLAN_CT_RT, ct_pitch<28>()> ct[2];
    struct {
        CtBuf<PLAN_CK_RT, CK_SP> buf[2];
        uint32_t act[152 * 9];
    } ck;
};

template <bool FAST, bool BP>
__global__ __launch_bounds__(CT_NT) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gemv_plan(const PlanWg *wgs,
                                                                                                int *flag) {
    __shared__ __attribute__((aligned(16))) PlanLds lds;
    const PlanWg &d = wgs[blockIdx.x];
    const GroupItem I = d.item;
    if (d.kind == 0) ct_tiles<FAST, BP, 28, PLAN_CT_RT, 1, 2>(I, d.t0, d.t1, flag, lds.ct);
    else ck_tiles<FAST, BP, 152, PLAN_CK_RT, 2>(I, d.t0, d.t1, flag, lds.ck.buf, lds.ck.act);
}

/* every item a share of the resident workgroups of kernel k (at most max_per_cu per CU) in proportion
 * to its tiles of rt rows (at least one, at most one per tile), each a contiguous tile range */
template <class GA>
hipError_t launch_tiles(const void *k, int &resident, uint32_t rt, GA &g, hipStream_t s, int max_per_cu = 0) {
    if (!resident) {
        int per_cu = 0, dev = 0, cus = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, CT_NT, 0);
        if (e == hipSuccess) e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        if (max_per_cu > 0 && per_cu > max_per_cu) per_cu = max_per_cu;
        resident = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    }
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < g.nitems; ++i) tiles += (g.item[i].rows + rt - 1) / rt;
    if (!tiles) return hipSuccess;
    uint32_t wgs = 0;
    for (uint32_t i = 0; i < g.nitems; ++i) {
        const uint32_t t = (g.item[i].rows + rt - 1) / rt;
        uint32_t n = (uint32_t)(((uint64_t)resident * t + tiles / 2) / tiles);
        n = n < 1 ? 1 : (n > t ? t : n);
        g.item[i].wg_begin = wgs;
        g.item[i].nwg = n;
        wgs += n;
    }
    void *args[] = {&g};
    const hipError_t e = hipLaunchKernel(k, dim3(wgs), dim3(CT_NT), args, 0, s);
    return e != hipSuccess ? e : hipGetLastError();
}

/* a launch of few items takes the kernel built for the small argument struct */
template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT, uint32_t D, int PER_CU>
hipError_t launch_ct_shape(GroupArgs &g, hipStream_t s) {
    if (g.nitems <= FEW_GROUP_ITEMS) {
        static int resident = 0;
        GroupArgsFew f = group_args_few(g);
        return launch_tiles((const void *)k_gemv_ct<FAST, BP, NB, RT, CPT, D, GroupArgsFew>, resident, RT, f, s,
                            PER_CU);
    }
    static int resident = 0;
    return launch_tiles((const void *)k_gemv_ct<FAST, BP, NB, RT, CPT, D, GroupArgs>, resident, RT, g, s, PER_CU);
}

template <bool FAST, bool BP, uint32_t NB, uint32_t RT, uint32_t CPT>
hipError_t launch_ck_shape(GroupArgs &g, hipStream_t s) {
    if (g.nitems <= FEW_GROUP_ITEMS) {
        static int resident = 0;
        GroupArgsFew f = group_args_few(g);
        return launch_tiles((const void *)k_gemv_ck<FAST, BP, NB, RT, CPT, GroupArgsFew>, resident, RT, f, s);
    }
    static int resident = 0;
    return launch_tiles((const void *)k_gemv_ck<FAST, BP, NB, RT, CPT, GroupArgs>, resident, RT, g, s);
}

/* 8 rows of 28 blocks per step: 504 pieces, one per thread of 512; two tiles in flight per workgroup
 * while the previous one is reduced, three workgroups per CU (about 12 MB requested chip-wide, where a
 * plain streaming read peaks). Measured on the 48 gate/up GEMVs of Qwen2.5-0.5B (235 MB): 38.8 us
 * against 40.8-42.1 us for 16-row tiles with one in flight; two or four workgroups per CU, or three
 * tiles in flight, were slower; configs[0]'s 48 x 896 x 896 group 11.7 against 12.3 us. */
template <bool FAST, bool BP>
hipError_t launch_ct_bp(GroupArgs &g, hipStream_t s) {
    if (g.nb == 28) return launch_ct_shape<FAST, BP, 28, 8, 1, 2, 3>(g, s);
    if (g.nb == 152) return launch_ck_shape<FAST, BP, 152, 14, 2>(g, s); /* 14 rows x 32-block chunks: 1008 pieces */
    return hipErrorInvalidValue;
}

template <bool FAST>
hipError_t launch_ct_fast(GroupArgs &g, hipStream_t s) {
    bool bp = false;
    for (uint32_t i = 0; i < g.nitems; ++i) bp = bp || g.item[i].bias || g.item[i].accumulate;
    return bp ? launch_ct_bp<FAST, true>(g, s) : launch_ct_bp<FAST, false>(g, s);
}

}  // namespace

uint32_t plan_rows_per_tile(bool wide) { return wide ? PLAN_CK_RT : PLAN_CT_RT; }

hipError_t plan_resident(int &per_cu) {
    static int resident = 0;
    if (!resident) {
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, (const void *)k_gemv_plan<false, false>,
                                                                          CT_NT, 0);
        if (e != hipSuccess) return e;
        if (resident > 3) resident = 3; /* as the grouped launches: about 12 MB in flight chip-wide */
        if (resident < 1) resident = 1;
    }
    per_cu = resident;
    return hipSuccess;
}

hipError_t launch_gemv_plan(const PlanWg *wgs, uint32_t n, bool fast, bool bp, int *flag, hipStream_t s) {
    if (!n) return hipSuccess;
    if (fast) {
        if (bp) hipLaunchKernelGGL((k_gemv_plan<true, true>), dim3(n), dim3(CT_NT), 0, s, wgs, flag);
        else hipLaunchKernelGGL((k_gemv_plan<true, false>), dim3(n), dim3(CT_NT), 0, s, wgs, flag);
    } else {
        if (bp) hipLaunchKernelGGL((k_gemv_plan<false, true>), dim3(n), dim3(CT_NT), 0, s, wgs, flag);
        else hipLaunchKernelGGL((k_gemv_plan<false, false>), dim3(n), dim3(CT_NT), 0, s, wgs, flag);
    }
    return hipGetLastError();
}

bool gemv_ct_ok(const GroupArgs &g, bool q5) {
    if (q5 || (g.nb != 28 && g.nb != 152)) return false;
    for (uint32_t i = 0; i < g.nitems; ++i) {
        const GroupItem &it = g.item[i];
        if ((((uintptr_t)it.w) | it.row_bytes) & 15u) return false;
        if (it.row_bytes != (size_t)g.nb * Q8_BYTES) return false; /* a tile is contiguous rows */
        if (((uintptr_t)it.xq | (uintptr_t)it.xd) & 3u) return false;
        if (!it.rows) return false;
    }
    return true;
}

hipError_t launch_gemv_ct(GroupArgs &g, bool fast, hipStream_t s) {
    return fast ? launch_ct_fast<true>(g, s) : launch_ct_fast<false>(g, s);
}

}  // namespace smq
