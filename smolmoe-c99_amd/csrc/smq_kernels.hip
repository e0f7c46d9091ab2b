/* gfx950 kernels of the quantized matrix-product path.
 *
 * Arithmetic contract (reference: src/kernels.c:36-79, docs/FORMAT.md:152-171):
 * for weight row r and activation t, block b contributes eight exact int32 lane
 * sums s_l (products 4l..4l+3); lane l accumulates acc_l = acc_l + d_b*float(s_l)
 * with d_b = wscale_b * xscale_b, two roundings per step (one fmaf in fast
 * mode), blocks in increasing order; the result is
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). Each lane is a serial f32 chain of
 * nb adds, so nothing below splits K across threads: parallelism comes from
 * rows, tokens and the eight lanes, and from computing the per-block products
 * away from the chain that adds them.
 *
 * Compiled with -ffp-contract=off (no fused multiply-add unless written as
 * fmaf), correctly rounded f32 division and f32 denormals preserved.
 */
#include <float.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

__device__ __forceinline__ uint32_t find_item(const MatArgs &a, uint32_t tile) {
    uint32_t it = 0;
    if (a.nitems > 1 && tile >= a.item[1].tile_begin) it = 1;
    if (a.nitems > 2 && tile >= a.item[2].tile_begin) it = 2;
    if (a.nitems > 3 && tile >= a.item[3].tile_begin) it = 3;
    return it;
}

/* ------------------------------------------------------------------------
 * Decode GEMV (ntok == 1), one tile per workgroup. Workgroup = RT rows x all
 * K. K is walked in chunks of CB blocks (the launcher sizes RT so that one
 * chunk usually covers K). In each chunk every thread owns one task (one Q8
 * block, or one pair of Q5 blocks, of one row): it loads the block and its
 * activation block straight from memory (the next chunk's task is prefetched
 * into registers), and writes the eight lane products d*float(s_l) (fast
 * mode: float(s_l) and d) into LDS. Then the RT*8 chain threads, one per
 * (row, lane), add their CB products in block order. The serial part per
 * thread is one add per block; the loads, dot4s and multiplies are spread
 * over all 256 threads.
 * LDS products: group g of four blocks holds [thread (r*8+l)][b%4], padded by
 * four floats per group so writes from a wave fall in distinct banks.
 * ---------------------------------------------------------------------- */
template <bool Q5, bool FAST, int RT>
__global__ __launch_bounds__(WG) void k_gemv(MatArgs a) {
    constexpr int TB = Q5 ? 2 : 1;    /* blocks per task */
    constexpr int TPR = WG / RT;      /* tasks per row per chunk */
    constexpr int CB = TPR * TB;      /* blocks per chunk */
    constexpr int GS = RT * 32 + 4;   /* floats per group of four blocks */
    constexpr int DS = RT * 4 + 4;    /* fast mode: scales per group */
    constexpr int NW = Q5 ? 11 : 9;   /* weight dwords per task */
    constexpr int NX = TB * 8;        /* activation words per task */
    __shared__ __attribute__((aligned(16))) float prod[2][(CB / 4) * GS];
    __shared__ __attribute__((aligned(16))) float dsc[FAST ? 2 : 1][FAST ? (CB / 4) * DS : 4];

    const uint32_t nb = a.nb, tid = threadIdx.x;
    const Item I = pick_item(a, blockIdx.x);
    const uint32_t r0 = (blockIdx.x - I.tile_begin) * RT;
    sgpr_now(a.xq);
    sgpr_now(a.xd);

    const uint32_t tr = tid / TPR, ti = tid % TPR;
    const bool row_ok = r0 + tr < I.rows;
    const unsigned char *wrow = I.w + (size_t)(row_ok ? r0 + tr : 0) * I.row_bytes;
    const uint32_t nchunks = (nb + CB - 1) / CB;

    uint32_t wr[NW] = {}, xr[NX] = {};
    float xs[TB] = {};
    auto load_task = [&](uint32_t b) {
        if (row_ok && b < nb) {
            const unsigned char *p = wrow + (size_t)b * (Q5 ? Q5_BYTES : Q8_BYTES);
            const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
            wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
            wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
            if constexpr (Q5) {
                const u3a v2 = *(const u3a *)(p + 32);
                wr[8] = v2.x; wr[9] = v2.y; wr[10] = v2.z;
            } else {
                wr[8] = *(const uint32_t *)(p + 32);
            }
            const unsigned char *xp = (const unsigned char *)a.xq + (size_t)b * QK;
#pragma unroll
            for (int k = 0; k < TB * 2; ++k) {
                const u4a v = *(const u4a *)(xp + 16 * k);
                xr[4 * k] = v.x; xr[4 * k + 1] = v.y; xr[4 * k + 2] = v.z; xr[4 * k + 3] = v.w;
            }
#pragma unroll
            for (int k = 0; k < TB; ++k) xs[k] = a.xd[b + k];
        }
    };
    load_task(ti * TB);
    OutPre pre = {0.0f, 0.0f}; /* the store's own reads, issued now */
    if (tid < RT * 8 && (tid & 7) == 7 && r0 + tid / 8 < I.rows) pre = load_out(I, 0, r0 + tid / 8);

    float acc = 0.0f;
    for (uint32_t c = 0; c < nchunks; ++c) {
        const uint32_t bt = c * CB + ti * TB; /* first block of this task */
        uint32_t cw[NW], cx[NX];
        float cs[TB];
#pragma unroll
        for (int k = 0; k < NW; ++k) cw[k] = wr[k];
#pragma unroll
        for (int k = 0; k < NX; ++k) cx[k] = xr[k];
#pragma unroll
        for (int k = 0; k < TB; ++k) cs[k] = xs[k];
        if (c + 1 < nchunks) load_task(bt + CB);

        float *pb = prod[c & 1];
        if (row_ok && bt < nb) {
            Q5Fields f[2];
            if (Q5) q5_parse_pair(cw, f[0], f[1]);
#pragma unroll
            for (int k = 0; k < TB; ++k) {
                const uint32_t bb = ti * TB + k;
                const float wscale = Q5 ? f[k].scale : __uint_as_float(cw[0]);
                const float d = wscale * cs[k];
                float *dst = pb + (bb / 4) * GS + tr * 32 + (bb % 4);
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    const uint32_t x = cx[k * 8 + l];
                    int s;
                    if (Q5) s = dot4(q5_codes(f[k], l), x, dot4(x, 0xf0f0f0f0u, 0));
                    else s = dot4(cw[1 + l], x, 0);
                    dst[l * 4] = FAST ? (float)s : d * (float)s;
                }
                if (FAST) dsc[c & 1][(bb / 4) * DS + tr * 4 + (bb % 4)] = d;
            }
        }
        __syncthreads();

        if (tid < RT * 8) {
            const uint32_t count = nb - c * CB < (uint32_t)CB ? nb - c * CB : (uint32_t)CB;
            const float4 *pp = (const float4 *)pb + tid, *dp = FAST ? (const float4 *)dsc[c & 1] + tid / 8 : nullptr;
            if (CB <= 32 && count % 4 == 0) /* whole groups: plain adds, the groups past count added as zeros */
                chain_sum_padded<FAST, CB / 4 <= 8 ? CB / 4 : 8>(acc, pp, GS / 4, dp, DS / 4, count / 4);
            else
                chain_sum<FAST, CB / 4>(acc, pp, GS / 4, dp, DS / 4, count);
        }
    }

    if (tid < RT * 8) {
        const float v = reduce8_to_lane7(acc);
        const uint32_t r = r0 + tid / 8;
        if ((tid & 7) == 7 && r < I.rows) store_out_pre(I, a.flag, 0, r, v, pre);
    }
}

/* ------------------------------------------------------------------------
 * Pinned streaming GEMV (Q8 nb <= MAX_FAST_NB; Q5 nb even, <= MAX_FAST_NB):
 * each workgroup belongs to one item (the launcher gives every item a share
 * of the resident workgroups in proportion to its rows) and walks a
 * contiguous range of that item's tiles. Its activation is staged in LDS
 * once, so a task is just the weight dwords of one Q8 block or one Q5 pair
 * (plus the row's bias and prior output for the chain threads), and D tasks
 * stay in flight per thread. Products and chains as in k_gemv: exact
 * per-lane order, the fixed lane tree.
 *
 * The tile is shaped to the row at launch: a row of ppr tasks is cut into
 * nch chunks of cpr tasks (pin_cpr at most; for Q5 rows of several chunks the
 * count whose slowest workgroup takes the fewest steps), and a tile is rt rows
 * (NT / cpr, within PIN_RT and the product buffer), so rt * cpr of the NT
 * threads hold a task (row tid / cpr, task tid % cpr): 28-block Q8 rows run
 * 18 rows of 28 threads of 512, 24-pair Q5 rows 32 rows of 24 of 768, 140-pair
 * Q5 rows (16 items) 7 chunks of 20 pairs, 24 rows of 20 of 512. ONE: a single
 * chunk per row.
 * ---------------------------------------------------------------------- */
/* Tasks per chunk at most: a Q8 chunk stays within 32 blocks (the chain
 * threads' short path), a Q5 chunk within 64 pairs (measured: the 280-block
 * rows as one chunk of 140 pairs, 3 rows per step, took 64 us per grouped
 * launch against 48 us in three chunks, their 280-add chains serialised). */
template <bool Q5, bool FAST>
constexpr uint32_t pin_cpr() { return Q5 ? 64u : 32u; }
constexpr uint32_t PIN_RT = 32; /* rows per tile at most */
constexpr uint32_t PIN_OOB = 0x80000000u; /* a buffer offset past every tile's records: reads zeros */
/* row strides the pinned kernel's 32-bit tile offsets hold: PIN_RT rows of this many bytes stay below
 * PIN_OOB (wider strides take the per-tile kernels) */
constexpr size_t PIN_MAX_ROW_BYTES = (size_t)1 << 25;

/* Rows per tile for chunks of c tasks: as many as the threads allow, at most
 * PIN_RT, and within a product buffer of pf floats (ceil(tb*c/4) groups of
 * rt*32 + 4: eight lanes of four blocks per row and a pad). */
__host__ __device__ constexpr uint32_t pin_rows(uint32_t nt, uint32_t tb, uint32_t c, uint32_t pf) {
    const uint32_t groups = (tb * c + 3) / 4, by_lds = (pf / groups - 4) / 32;
    const uint32_t r = nt / c < PIN_RT ? nt / c : PIN_RT;
    return r < by_lds ? r : by_lds;
}

template <bool Q5>
struct PinTask {
    uint32_t w[Q5 ? 11 : 9];
    float bias, prior;
    bool ok;
};

template <class GA>
__device__ __forceinline__ uint32_t find_pin_item(const GA &g, uint32_t wg) {
    uint32_t lo = 0, hi = g.nitems; /* last item with wg_begin <= wg */
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (g.item[mid].wg_begin <= wg) lo = mid;
        else hi = mid;
    }
    return lo;
}

/* occupancy floor: exact Q8 6 waves per SIMD (three 512-thread workgroups per CU), exact Q5 of several
 * chunks 4 (two per CU);
 * PF: floats of one product buffer (the launcher keeps rt within it) */
template <bool Q5, bool FAST, bool ONE, int NT, int D, uint32_t MAXNB, uint32_t PF, class GA>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(Q5 ? (ONE || FAST ? 3 : 4) : (FAST ? 4 : 6), 8))) void k_gemv_pin(
    GA g) {
    constexpr int TB = Q5 ? 2 : 1;
    constexpr bool HOIST = ONE && Q5;
    constexpr uint32_t BYTES = Q5 ? Q5_BYTES : Q8_BYTES;
    /* each buffer ends in a sink for the product writes of idle task lanes */
    __shared__ __attribute__((aligned(16))) float prod[2][PF + 32];
    __shared__ __attribute__((aligned(16))) float dsc[FAST ? 2 : 1][FAST ? PF / 8 + 128 + 4 : 4];
    /* the staged activation (a hoisting launch reads its words straight into registers), piece-major:
     * the 16-byte piece k of task t's activation (TB blocks, 2 TB pieces) at act_q[(k * ATASKS + t) * 4],
     * so the lanes of one read instruction (consecutive tasks, one k) read consecutive 16-byte pieces
     * and meet no bank twice (task-major, 32 or 64 bytes apart, cost 2- and 4-way conflicts) */
    constexpr uint32_t ACT_NB = HOIST ? 1 : MAXNB, ATASKS = (ACT_NB + TB - 1) / TB;
    __shared__ __attribute__((aligned(16))) uint32_t act_q[ATASKS * TB * 8];
    __shared__ float act_d[ACT_NB];

    const uint32_t tid = threadIdx.x, nb = g.nb, cpr = g.cpr, nch = ONE ? 1u : g.nch, rt = g.rt;
    const uint32_t tr = tid / cpr, ti = tid % cpr, cb = cpr * TB; /* cb: blocks per chunk */
    const uint32_t gs = rt * 32 + 4, ds = rt * 4 + 4, chains = rt * 8;
    const GroupItem &I = g.item[find_pin_item(g, blockIdx.x)];
    const uint32_t wg = blockIdx.x - I.wg_begin, item_tiles = (I.rows + rt - 1) / rt;
    const uint32_t t0 = (uint32_t)((uint64_t)item_tiles * wg / I.nwg);
    const uint32_t t1 = (uint32_t)((uint64_t)item_tiles * (wg + 1) / I.nwg);
    const uint32_t my_steps = (t1 - t0) * nch;
    const unsigned char *wbase = I.w;
    const size_t row_bytes = I.row_bytes;
    const uint32_t rows = I.rows;
    const float *bias_p = I.bias, *xd = I.xd;
    float *y = I.y;
    const bool accum = I.accumulate != 0, worker = tr < rt;

    /* the activation, once (kernels.c:912-935 layout: nb scales, nb*8 words) */
    const uint32_t *xq32 = (const uint32_t *)I.xq;
    /* the activation's 16-byte pieces (piece p: words 4(p % 2).. of block p / 2) and scales, all
     * requested before the first task and stored into LDS after the first tasks are requested (a
     * loop of load-then-store waited one memory round trip per iteration) */
    constexpr uint32_t SPT = HOIST ? 1 : (ACT_NB * 2 + NT - 1) / NT, SDT = HOIST ? 1 : (ACT_NB + NT - 1) / NT;
    u4a pv[SPT];
    float dv[SDT];
    if constexpr (!HOIST) {
#pragma unroll
        for (uint32_t k = 0; k < SPT; ++k) {
            const uint32_t pp = tid + k * NT, pc = pp < nb * 2 ? pp : 0;
            pv[k] = *(const u4a *)&xq32[4 * pc];
        }
#pragma unroll
        for (uint32_t k = 0; k < SDT; ++k) {
            const uint32_t i = tid + k * NT;
            dv[k] = xd[i < nb ? i : 0];
        }
    }
    if constexpr (ONE) {
        /* +0.0 in the slots past the last block, never written after (chain_sum_padded: a one-chunk
         * row's blocks fill the same slots at every step): both buffers whole, sinks included (the
         * launcher keeps every chain read below PF) */
        constexpr uint32_t PROD_FLOATS = sizeof(prod) / sizeof(float), DSC_FLOATS = sizeof(dsc) / sizeof(float);
        for (uint32_t i = tid; i < PROD_FLOATS; i += NT) (&prod[0][0])[i] = 0.0f;
        if constexpr (FAST)
            for (uint32_t i = tid; i < DSC_FLOATS; i += NT) (&dsc[0][0])[i] = 0.0f;
    }

    /* step s: tile t0 + s / nch, chunk s % nch (counters, no division per step). A step's tile is one
     * buffer resource formed by scalar arithmetic: its first row, and records covering its rows within
     * the matrix (none for a step past this workgroup's range). A lane's offset into it is fixed (its
     * row of the tile, its task's blocks; the chunk is a scalar offset), and a row past the matrix, a
     * step past the range or an idle task (an out-of-range offset) reads zeros without touching memory.
     * Every thread issues the same loads at every step, outside any branch, so the compiler's in-order
     * wait counts stay exact and the next task stays in flight across the step. (Before, 64-bit
     * addresses with clamps took 13 VALU instructions a task, and a step past the range re-read the
     * range's last tile.) */
    const uint32_t rb32 = (uint32_t)row_bytes;
    const uint32_t lane_off = worker ? tr * rb32 + ti * TB * BYTES : PIN_OOB;
    auto load = [&](PinTask<Q5> &T, uint32_t tile, uint32_t chunk, bool real) __attribute__((always_inline)) {
        const uint32_t row0 = tile * rt, b = chunk * cb + ti * TB;
        T.ok = real && worker && row0 + tr < rows && b < nb;
        const uint32_t in_rows = real ? (rows - row0 < rt ? rows - row0 : rt) : 0u;
        const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(wbase + (size_t)row0 * row_bytes), (short)0, (int)(in_rows * rb32), 0x00020000);
        const uint32_t voff = b < nb ? lane_off : PIN_OOB, soff = chunk * cb * BYTES;
        const u4a v0 = __builtin_bit_cast(u4a, __builtin_amdgcn_raw_buffer_load_b128(src, voff, soff, 0));
        const u4a v1 = __builtin_bit_cast(u4a, __builtin_amdgcn_raw_buffer_load_b128(src, voff + 16, soff, 0));
        T.w[0] = v0.x; T.w[1] = v0.y; T.w[2] = v0.z; T.w[3] = v0.w;
        T.w[4] = v1.x; T.w[5] = v1.y; T.w[6] = v1.z; T.w[7] = v1.w;
        if constexpr (Q5) { /* a pair: 44 bytes */
            const auto v2 = __builtin_amdgcn_raw_buffer_load_b96(src, voff + 32, soff, 0);
            T.w[8] = v2[0]; T.w[9] = v2[1]; T.w[10] = v2[2];
        } else {
            T.w[8] = __builtin_amdgcn_raw_buffer_load_b32(src, voff + 32, soff, 0);
        }
    };
    /* one chunk: the chain threads' row, its bias and prior output (the other threads read the
     * tile's first row; an absent one reads the activation's first scale: unused). Requested
     * after the previous use of the task's registers is complete (its store), so no loaded
     * value is copied while its load is in flight */
    auto load_bp = [&](PinTask<Q5> &T, uint32_t tile, bool real) __attribute__((always_inline)) {
        const uint32_t tl = real ? tile : t1 - 1;
        const uint32_t orow = tl * rt + (tid < chains ? tid / 8 : 0), oc = orow < rows ? orow : rows - 1;
        T.bias = *(bias_p ? bias_p + oc : xd);
        T.prior = *(accum ? y + oc : xd);
    };
    /* Q5, one chunk: a thread's blocks are the same at every step, so their activation words and
     * scales live in registers (idle threads read clamped, unused indices). Requested before the first
     * tasks: loads complete in order, so no wait for them inside the step loop counts later loads (one
     * requested after the tasks made every step wait for all loads in flight) */
    uint32_t hx_q[HOIST ? TB : 1][8];
    float hx_d[HOIST ? TB : 1];
    if constexpr (HOIST) {
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            const uint32_t b0 = ti * TB + q, b = b0 < nb ? b0 : nb - 1;
            hx_d[q] = xd[b];
            const u4a xa = *(const u4a *)&xq32[b * 8], xb = *(const u4a *)&xq32[b * 8 + 4];
            hx_q[q][0] = xa.x; hx_q[q][1] = xa.y; hx_q[q][2] = xa.z; hx_q[q][3] = xa.w;
            hx_q[q][4] = xb.x; hx_q[q][5] = xb.y; hx_q[q][6] = xb.z; hx_q[q][7] = xb.w;
        }
    }
    PinTask<Q5> T[D];
    uint32_t lt = t0, lc = 0; /* load cursor */
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load(T[j], lt, lc, (uint32_t)j < my_steps);
        if constexpr (ONE) load_bp(T[j], lt, (uint32_t)j < my_steps);
        if (++lc == nch) { lc = 0; ++lt; }
    }
    /* several chunks per row: the bias and prior output of the chain threads' rows, requested for a
     * tile right after the store of the previous one (a whole tile of steps ahead of their use) */
    auto load_tile_bp = [&](float &bias, float &prior, uint32_t tile) __attribute__((always_inline)) {
        const uint32_t tl = tile < t1 ? tile : t1 - 1;
        const uint32_t orow = tl * rt + (tid < chains ? tid / 8 : 0), oc = orow < rows ? orow : rows - 1;
        bias = *(bias_p ? bias_p + oc : xd);
        prior = *(accum ? y + oc : xd);
    };
    float mbias = 0.0f, mprior = 0.0f;
    if constexpr (!ONE) load_tile_bp(mbias, mprior, t0);
    if constexpr (!HOIST) {
#pragma unroll
        for (uint32_t k = 0; k < SPT; ++k) {
            const uint32_t pp = tid + k * NT, b = pp / 2, o = (b % TB) * 8 + (pp % 2) * 4; /* word o of task b / TB */
            if (pp < nb * 2) *(u4a *)&act_q[((o / 4) * ATASKS + b / TB) * 4] = pv[k];
        }
#pragma unroll
        for (uint32_t k = 0; k < SDT; ++k)
            if (tid + k * NT < nb) act_d[tid + k * NT] = dv[k];
    }
    __syncthreads(); /* activation staged */
    /* Q5, one chunk: the offsets c = -16 * (sum of the four int8 of a lane) of the activation words
     * requested above, formed once the task loads are on their way */
    uint32_t hx_c[HOIST ? TB : 1][8];
    if constexpr (HOIST) {
#pragma unroll
        for (int q = 0; q < TB; ++q)
#pragma unroll
            for (int l = 0; l < 8; ++l) hx_c[q][l] = dot4(hx_q[q][l], 0xf0f0f0f0u, 0);
    }
    /* one product step of task T: its lane products into pb (an idle task's to the sink) */
    auto products = [&](const PinTask<Q5> &Tk, float *pb, float *db, uint32_t chunk) __attribute__((always_inline)) {
        const bool ok = Tk.ok;
        Q5Fields f[2];
        if constexpr (Q5) q5_parse_pair(Tk.w, f[0], f[1]);
        float d[TB];
        uint32_t xs[TB][8];
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            const uint32_t bb = ti * TB + q, b0 = chunk * cb + bb, b = b0 < nb ? b0 : nb - 1;
            d[q] = (Q5 ? f[q].scale : __uint_as_float(Tk.w[0])) * (HOIST ? hx_d[q] : act_d[b]);
            if (FAST) db[ok ? (bb / 4) * ds + tr * 4 + (bb % 4) : PF / 8 + 128 + q] = d[q];
            if constexpr (HOIST) {
#pragma unroll
                for (int l = 0; l < 8; ++l) xs[q][l] = hx_q[q][l];
            } else {
                const uint32_t at = (2 * (b % TB) * ATASKS + b / TB) * 4;
                const u4a xa = *(const u4a *)&act_q[at], xb = *(const u4a *)&act_q[at + ATASKS * 4];
                xs[q][0] = xa.x; xs[q][1] = xa.y; xs[q][2] = xa.z; xs[q][3] = xa.w;
                xs[q][4] = xb.x; xs[q][5] = xb.y; xs[q][6] = xb.z; xs[q][7] = xb.w;
            }
        }
        const uint32_t bb0 = ti * TB;
        float *slot = ok ? pb + (bb0 / 4) * gs + tr * 32 + (bb0 % 4) : pb + PF;
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            float v[TB];
#pragma unroll
            for (int q = 0; q < TB; ++q) {
                int sv;
                if constexpr (Q5)
                    sv = dot4(q5_codes(f[q], l), xs[q][l], HOIST ? hx_c[q][l] : dot4(xs[q][l], 0xf0f0f0f0u, 0));
                else sv = dot4(Tk.w[1 + l], xs[q][l], 0);
                v[q] = FAST ? (float)sv : d[q] * (float)sv;
            }
            put_lane<TB>(slot, l, v[0], v[TB - 1]);
        }
    };
    if constexpr (ONE) {
        /* one chunk per row: every step is a whole tile. D steps per trip with no early exit (a
         * straight trip keeps the in-flight tasks in their registers); a step past the range is
         * computed (idle products, sink) and not stored */
        for (uint32_t k = 0; k < my_steps; k += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const uint32_t step = k + j, tile = t0 + step;
                const bool live = step < my_steps;
                float *pb = prod[step & 1];
                float *db = dsc[FAST ? step & 1 : 0];
                __builtin_amdgcn_sched_barrier(0);
                products(T[j], pb, db, 0);
                load(T[j], tile + D, 0, step + D < my_steps); /* consumed: the next task for these registers */
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
                if (tid < chains) {
                    float acc = 0.0f;
                    const float4 *pp = (const float4 *)pb + tid, *dp = FAST ? (const float4 *)db + tid / 8 : nullptr;
                    if constexpr (!Q5) chain_sum_padded<FAST, 8>(acc, pp, gs / 4, dp, ds / 4, (nb + 3) / 4);
                    else if (!FAST && nb <= 48) /* every group read at once, plain adds (the 1536-wide rows: 37.2-38.7
                                                 * against 43.8-44.3 us with a count select per slot, same box) */
                        chain_sum_padded<FAST, 12>(acc, pp, gs / 4, dp, ds / 4, (nb + 3) / 4);
                    else if (nb <= 32) chain_sum<FAST, 8>(acc, pp, gs / 4, dp, ds / 4, nb);
                    else chain_sum<FAST, 32>(acc, pp, gs / 4, dp, ds / 4, nb);
                    const float v = reduce8_to_lane7(acc);
                    const uint32_t r = tile * rt + tid / 8;
                    if (live && (tid & 7) == 7 && r < rows) {
                        float o = v;
                        if (bias_p) o = o + T[j].bias; /* model.c:259-262 */
                        if (g.flag && !(fabsf(o) <= FLT_MAX)) *g.flag = 1;
                        if (accum) o = T[j].prior + o;
                        y[r] = o;
                    }
                }
                load_bp(T[j], tile + D, step + D < my_steps);
            }
        }
        return;
    }
    uint32_t ct = t0, cc = 0; /* chain cursor */
    float acc = 0.0f;
    /* a straight trip of D steps; a step past the range stores nothing. Every trip but the last
     * requests the next tasks, the last nothing (as for one chunk) */
    auto trip = [&](uint32_t k, auto next) __attribute__((always_inline)) {
        constexpr bool NEXT = decltype(next)::value;
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const bool live = k + j < my_steps;
            float *pb = prod[(k + j) & 1];
            float *db = dsc[FAST ? (k + j) & 1 : 0];
            /* every task's products, an idle one's to the sink: a branch around them left the
             * task's loads unwaited on one path, so reusing its registers waited for every load */
            products(T[j], pb, db, cc);
            /* this task is consumed: its slot reloads now, a barrier and a chain earlier than
             * at the end of the step */
            if constexpr (NEXT) {
                load(T[j], lt, lc, k + j + D < my_steps);
                if (++lc == nch) { lc = 0; ++lt; }
            }
            __syncthreads();
            if (tid < chains) {
                const uint32_t count = nb - cc * cb < cb ? nb - cc * cb : cb;
                const float4 *pp = (const float4 *)pb + tid, *dp = FAST ? (const float4 *)db + tid / 8 : nullptr;
                if (!Q5 || cb <= 32) chain_sum<FAST, 8>(acc, pp, gs / 4, dp, ds / 4, count);
                else chain_sum<FAST, 32>(acc, pp, gs / 4, dp, ds / 4, count);
                if (cc + 1 == nch) {
                    const float v = reduce8_to_lane7(acc);
                    const uint32_t r = ct * rt + tid / 8;
                    if (live && (tid & 7) == 7 && r < rows) {
                        float o = v;
                        if (bias_p) o = o + mbias; /* model.c:259-262 */
                        if (g.flag && !(fabsf(o) <= FLT_MAX)) *g.flag = 1;
                        if (accum) o = mprior + o;
                        y[r] = o;
                    }
                    acc = 0.0f;
                }
            }
            if (cc + 1 == nch) load_tile_bp(mbias, mprior, ct + 1); /* uniform; the store above used them */
            if (++cc == nch) { cc = 0; ++ct; }
        }
    };
    uint32_t k = 0;
    for (; k + D < my_steps; k += D) trip(k, std::true_type{});
    trip(k, std::false_type{}); /* my_steps >= 1: the last trip */
}

/* ------------------------------------------------------------------------
 * Exact prefill GEMM (ntok > 1). Workgroup tile = 32 rows x 16 tokens (x 8
 * tokens where 16-token tiles leave CUs idle); K in chunks of 16 blocks staged
 * in LDS (weights decoded once per block: Q5 becomes signed int8 words, so the
 * inner loop is the same for both formats). Thread (row pair, token), or
 * (row, token) in 8-token tiles, owns all eight lanes of its (row, token) outputs:
 * sixteen serial chains, each block one d = wscale * xscale per output and per
 * lane one dot4, one convert, one multiply and one add; the lane tree runs in
 * the thread. A block's eight words of a row or token are two 16-byte LDS
 * reads. (Thread per lane of 4 rows x 4 tokens, before: d formed in all eight
 * lanes, one LDS read per product, 88 VALU per 16 lane sums against 66.) The
 * next chunk's global loads are issued before the current chunk is computed.
 * ---------------------------------------------------------------------- */
constexpr int GT_R = 32, GT_CB = 16;
constexpr int WQ_PITCH = GT_CB * 8 + 4; /* dwords, 16-byte rows; 4 mod 64: the 16 tokens of a wave's
                                          * 16-byte reads start 4 banks apart */
constexpr int SC_PITCH = GT_CB + 1;

/* TT tokens per tile: 16, or 8 where 16-token tiles would leave CUs idle (a thread then owns one row) */
template <bool Q5, bool FAST, int TT>
__global__ __launch_bounds__(WG) void k_gemm_exact(MatArgs a, uint32_t tok_tiles) {
    static_assert(TT == 16 || TT == 8, "token tile");
    constexpr uint32_t TPT = WG / TT;          /* staging threads per token */
    constexpr uint32_t NP = 32 / TPT;          /* 16-byte activation pieces per staging thread */
    constexpr int RPT = GT_R * TT / WG;        /* rows per thread */
    __shared__ float wsl[GT_R][SC_PITCH];
    __shared__ __attribute__((aligned(16))) uint32_t wql[GT_R][WQ_PITCH];
    __shared__ float xdl[TT][SC_PITCH];
    __shared__ __attribute__((aligned(16))) uint32_t xql[TT][WQ_PITCH];

    const uint32_t tid = threadIdx.x, nb = a.nb;
    /* XCD-aware order: workgroup i runs on XCD i % 8; give each XCD a
     * contiguous range of tiles so the token tiles of one row tile share an L2. */
    const uint32_t G = gridDim.x, xcd = blockIdx.x % 8u, k = blockIdx.x / 8u;
    const uint32_t per = G / 8u, extra = G % 8u;
    const uint32_t L = xcd * per + (xcd < extra ? xcd : extra) + k;
    const uint32_t row_tile = L / tok_tiles, tok_tile = L % tok_tiles;

    const Item &I = a.item[find_item(a, row_tile)];
    const uint32_t r0 = (row_tile - I.tile_begin) * GT_R, t0 = tok_tile * TT;

    /* staging roles */
    const uint32_t srow = tid / 8, spart = tid % 8; /* weights: row, pair of blocks */
    const bool srow_ok = r0 + srow < I.rows;
    const unsigned char *wrow = I.w + (size_t)(srow_ok ? r0 + srow : 0) * I.row_bytes;
    const uint32_t stok = tid / TPT, spiece = tid % TPT; /* activations */
    const bool stok_ok = t0 + stok < a.ntok;
    const size_t tok_base = (size_t)(stok_ok ? t0 + stok : 0) * a.xstride;

    uint32_t wr[Q5 ? 11 : 18] = {};
    u4a xr[NP] = {};
    float xs = 0.0f;
    auto fetch = [&](uint32_t c) {
        const uint32_t b = c * GT_CB + spart * 2;
        if (Q5) {
            if (srow_ok && b < nb) {
                const unsigned char *p = wrow + (size_t)b * Q5_BYTES;
                const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                const u3a v2 = *(const u3a *)(p + 32);
                wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
                wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
                wr[8] = v2.x; wr[9] = v2.y; wr[10] = v2.z;
            }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (srow_ok && b + h < nb) {
                    const unsigned char *p = wrow + (size_t)(b + h) * Q8_BYTES;
                    const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                    wr[9 * h + 0] = v0.x; wr[9 * h + 1] = v0.y; wr[9 * h + 2] = v0.z; wr[9 * h + 3] = v0.w;
                    wr[9 * h + 4] = v1.x; wr[9 * h + 5] = v1.y; wr[9 * h + 6] = v1.z; wr[9 * h + 7] = v1.w;
                    wr[9 * h + 8] = *(const uint32_t *)(p + 32);
                }
            }
        }
        /* token stok, 16-byte pieces spiece + TPT h of the chunk's 512 bytes */
#pragma unroll
        for (uint32_t h = 0; h < NP; ++h) {
            const uint32_t piece = spiece + TPT * h, b = c * GT_CB + piece / 2;
            if (stok_ok && b < nb) xr[h] = *(const u4a *)(a.xq + (tok_base + c * GT_CB) * QK + piece * 16);
        }
        const uint32_t bx = c * GT_CB + spiece;
        if (stok_ok && spiece < (uint32_t)GT_CB && bx < nb) xs = a.xd[tok_base + bx];
    };
    /* Q5: no select on the staged words (a row past the matrix or a token past the batch stages whatever its
     * registers hold and is never stored, each output taking only its own row's and token's operands; a
     * block past the row is skipped by the block loop): 1536x8960 at 128 tokens 79.5-82.0 -> 75.6-76.7 us.
     * Q8 keeps them (without: 896x4864 at 192 tokens 43.0-43.5 -> 44.6-44.7) */
    auto stage = [&](uint32_t c) {
        const uint32_t b = c * GT_CB + spart * 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t bb = spart * 2 + h;
            const bool ok = Q5 || (srow_ok && b + h < nb);
            uint32_t words[8];
            float sc = 0.0f;
            if (Q5) {
                Q5Fields f[2];
                q5_parse_pair(wr, f[0], f[1]);
#pragma unroll
                for (int l = 0; l < 8; ++l) words[l] = q5_signed(f[h], l);
                sc = f[h].scale;
            } else {
#pragma unroll
                for (int l = 0; l < 8; ++l) words[l] = ok ? wr[9 * h + 1 + l] : 0u;
                sc = ok ? __uint_as_float(wr[9 * h]) : 0.0f;
            }
            wsl[srow][bb] = sc;
            uint2 *dst = (uint2 *)&wql[srow][bb * 8];
#pragma unroll
            for (int l = 0; l < 4; ++l) dst[l] = make_uint2(words[2 * l], words[2 * l + 1]);
        }
#pragma unroll
        for (uint32_t h = 0; h < NP; ++h) {
            const uint32_t piece = spiece + TPT * h, b = c * GT_CB + piece / 2;
            const bool ok = Q5 || (stok_ok && b < nb);
            uint2 *dst = (uint2 *)&xql[stok][piece * 4];
            dst[0] = ok ? make_uint2(xr[h].x, xr[h].y) : make_uint2(0u, 0u);
            dst[1] = ok ? make_uint2(xr[h].z, xr[h].w) : make_uint2(0u, 0u);
        }
        const uint32_t bx = c * GT_CB + spiece;
        if (spiece < (uint32_t)GT_CB) xdl[stok][spiece] = (Q5 || (stok_ok && bx < nb)) ? xs : 0.0f;
    };

    const uint32_t tg = tid % TT, rg = tid / TT; /* token tg, rows RPT rg .. RPT rg + RPT - 1 */
    static_assert(TT * GT_R / RPT == WG, "one thread per (RPT rows, token)");
    float acc[RPT][8];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[i][l] = 0.0f;

    const uint32_t nchunks = (nb + GT_CB - 1) / GT_CB;
    fetch(0);
    for (uint32_t c = 0; c < nchunks; ++c) {
        stage(c);
        __syncthreads();
        if (c + 1 < nchunks) fetch(c + 1);
        const uint32_t count = nb - c * GT_CB < (uint32_t)GT_CB ? nb - c * GT_CB : (uint32_t)GT_CB;
        auto block = [&](uint32_t bb) __attribute__((always_inline)) {
            const u4a x0 = *(const u4a *)&xql[tg][bb * 8], x1 = *(const u4a *)&xql[tg][bb * 8 + 4];
            const uint32_t x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const float xsc = xdl[tg][bb];
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const u4a w0 = *(const u4a *)&wql[RPT * rg + i][bb * 8], w1 = *(const u4a *)&wql[RPT * rg + i][bb * 8 + 4];
                const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                const float d = wsl[RPT * rg + i][bb] * xsc;
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[i][l] = lane_step<FAST>(acc[i][l], d, dot4(w[l], x[l], 0));
            }
        };
        if (count == (uint32_t)GT_CB) { /* whole chunks two blocks per trip (down 896x4864x128: 40.6 -> 38.4 us;
                                          * four per trip was slower, 52.7 us) */
#pragma unroll 2
            for (uint32_t bb = 0; bb < (uint32_t)GT_CB; ++bb) block(bb);
        } else {
            for (uint32_t bb = 0; bb < count; ++bb) block(bb);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const float *a8 = acc[i]; /* the lane tree of reduce8: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
        const float v = ((a8[0] + a8[4]) + (a8[2] + a8[6])) + ((a8[1] + a8[5]) + (a8[3] + a8[7]));
        const uint32_t r = r0 + RPT * rg + i, t = t0 + tg;
        if (r < I.rows && t < a.ntok) store_out(I, a.flag, t, r, v);
    }
}

/* ------------------------------------------------------------------------
 * Prefill GEMM on int8 MFMA (relaxed block order). A Q8 block is exactly the
 * K = 32 of v_mfma_i32_16x16x32_i8, so one MFMA per (16 rows x 16 tokens,
 * block) yields the exact int32 block sums S; the epilogue then applies the
 * block's scales, acc = fma(wscale * xscale, float(S), acc), blocks in order.
 * The per-block integer sums are bit-exact; the f32 result differs from the
 * eight-lane contract only in rounding (within 1e-5 relative).
 * Workgroup tile: 32 rows x 64 tokens; wave w owns rows 16*(w/2).. and tokens
 * 32*(w%2).. (two 16x16 tiles). K is staged in chunks of MT_CB blocks, stored in
 * MFMA operand order so that a wave's operand read is one contiguous 512-byte
 * run: A[block][k8 chunk][row] and B[block][k8 chunk][token], 8 bytes each.
 * Operand layout (16x16x32 i8): lane l supplies A[l%16][8*(l/16)+0..7] and
 * B[8*(l/16)+0..7][l%16]; it receives D[4*(l/16)+v][l%16], v = 0..3.
 * SUMS writes the raw block sums instead (test entry point).
 * K split: with few tiles (e.g. 1536 x 8960 at 64 tokens: 48 workgroups of 20
 * chunks each) the chunks are cut into `slices` ranges, one workgroup per
 * (slice, tile); each writes its partial tile to the library workspace and
 * k_mfma_reduce adds the slices in order, then bias, finiteness and the
 * residual add.
 * ---------------------------------------------------------------------- */
constexpr int MT_R = 32, MT_T = 64, MT_CB = 14; /* 14 blocks: a 896-wide row in two chunks */
constexpr int MT_WT = 32 * MT_CB / 2;           /* staging threads of the weights (two blocks each) */
constexpr int MT_XP = 64 * MT_CB * 2 / 256;     /* 16-byte activation pieces per thread */
constexpr int MT_XS = (64 * MT_CB + 255) / 256; /* activation scales per thread (last one partial) */
typedef int v4i __attribute__((ext_vector_type(4)));

struct MfmaSplit {
    uint32_t slices, cps; /* K slices, chunks per slice */
    uint32_t total_rows;  /* tiles x MT_R: the partials' row pitch */
    float *part;          /* slices > 1: [slice][ntok][total_rows] partial sums */
};

template <bool Q5, bool SUMS>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(3, 8))) void k_gemm_mfma(MatArgs a, uint32_t tok_tiles, int32_t *sums,
                                                                                   MfmaSplit sp) {
    __shared__ __attribute__((aligned(16))) uint2 wqa[MT_CB][4][MT_R];
    __shared__ __attribute__((aligned(16))) uint2 xqb[MT_CB][4][MT_T];
    __shared__ __attribute__((aligned(16))) float wsl[MT_CB][MT_R];
    __shared__ __attribute__((aligned(16))) float xsl[MT_CB][MT_T];

    const uint32_t tid = threadIdx.x, nb = a.nb, l = tid % 64, w = tid / 64;
    const uint32_t G = gridDim.x, xcd = blockIdx.x % 8u, kk = blockIdx.x / 8u;
    const uint32_t per = G / 8u, extra = G % 8u;
    const uint32_t L = xcd * per + (xcd < extra ? xcd : extra) + kk;
    const uint32_t tiles_all = G / sp.slices, slice = L / tiles_all, rem = L % tiles_all;
    const uint32_t row_tile = rem / tok_tiles, tok_tile = rem % tok_tiles;
    const Item &I = a.item[find_item(a, row_tile)];
    const uint32_t r0 = (row_tile - I.tile_begin) * MT_R, t0 = tok_tile * MT_T;

    /* staging roles: weights (row, pair of blocks), threads 0..127; a wave
     * writes 32 consecutive rows of one block. Activations: a wave stages one
     * (block, half) for 64 consecutive tokens (one contiguous LDS run). */
    const uint32_t srow = tid % 32, spair = tid / 32;
    const bool srow_ok = tid < MT_WT && r0 + srow < I.rows;
    const unsigned char *wrow = I.w + (size_t)(srow_ok ? r0 + srow : 0) * I.row_bytes;

    uint32_t wr[Q5 ? 11 : 18] = {};
    u4a xr[MT_XP] = {};
    float xs[MT_XS] = {};
    auto fetch = [&](uint32_t c) {
        const uint32_t b = c * MT_CB + spair * 2;
        if (tid < MT_WT) {
            if (Q5) {
                if (srow_ok && b < nb) {
                    const unsigned char *p = wrow + (size_t)b * Q5_BYTES;
                    const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                    const u3a v2 = *(const u3a *)(p + 32);
                    wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
                    wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
                    wr[8] = v2.x; wr[9] = v2.y; wr[10] = v2.z;
                }
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    if (srow_ok && b + h < nb) {
                        const unsigned char *p = wrow + (size_t)(b + h) * Q8_BYTES;
                        const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                        wr[9 * h + 0] = v0.x; wr[9 * h + 1] = v0.y; wr[9 * h + 2] = v0.z; wr[9 * h + 3] = v0.w;
                        wr[9 * h + 4] = v1.x; wr[9 * h + 5] = v1.y; wr[9 * h + 6] = v1.z; wr[9 * h + 7] = v1.w;
                        wr[9 * h + 8] = *(const uint32_t *)(p + 32);
                    }
            }
        }
        /* 64 tokens x MT_CB blocks x 32 bytes in 16-byte pieces, MT_XP per thread */
#pragma unroll
        for (int h = 0; h < MT_XP; ++h) {
            const uint32_t piece = tid + WG * h, tok = piece % 64, rest = piece / 64, bb = rest / 2, half = rest % 2;
            const uint32_t t = t0 + tok, b = c * MT_CB + bb;
            if (t < a.ntok && b < nb)
                xr[h] = *(const u4a *)(a.xq + ((size_t)t * a.xstride + b) * QK + half * 16);
        }
#pragma unroll
        for (int h = 0; h < MT_XS; ++h) {
            const uint32_t e = tid + WG * h, tok = e / MT_CB, bb = e % MT_CB;
            const uint32_t t = t0 + tok, b = c * MT_CB + bb;
            if (e < 64u * MT_CB && t < a.ntok && b < nb) xs[h] = a.xd[(size_t)t * a.xstride + b];
        }
    };
    auto stage = [&](uint32_t c) {
        if (tid < MT_WT) {
            const uint32_t b = c * MT_CB + spair * 2;
            Q5Fields f[2];
            if (Q5) q5_parse_pair(wr, f[0], f[1]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t bb = spair * 2 + h;
                const bool ok = srow_ok && b + h < nb;
                uint32_t wv[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) wv[k] = ok ? (Q5 ? q5_signed(f[h], k) : wr[9 * h + 1 + k]) : 0u;
                wsl[bb][srow] = ok ? (Q5 ? f[h].scale : __uint_as_float(wr[9 * h])) : 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) wqa[bb][k][srow] = make_uint2(wv[2 * k], wv[2 * k + 1]);
            }
        }
#pragma unroll
        for (int h = 0; h < MT_XP; ++h) {
            const uint32_t piece = tid + WG * h, tok = piece % 64, rest = piece / 64, bb = rest / 2, half = rest % 2;
            const bool ok = t0 + tok < a.ntok && c * MT_CB + bb < nb;
            xqb[bb][2 * half][tok] = ok ? make_uint2(xr[h].x, xr[h].y) : make_uint2(0u, 0u);
            xqb[bb][2 * half + 1][tok] = ok ? make_uint2(xr[h].z, xr[h].w) : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int h = 0; h < MT_XS; ++h) {
            const uint32_t e = tid + WG * h, tok = e / MT_CB, bb = e % MT_CB;
            if (e < 64u * MT_CB) xsl[bb][tok] = (t0 + tok < a.ntok && c * MT_CB + bb < nb) ? xs[h] : 0.0f;
        }
    };

    const uint32_t wrow0 = 16 * (w / 2), wtok0 = 32 * (w % 2);
    float acc[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[j][v] = 0.0f;
    const v4i zero = {0, 0, 0, 0};

    const uint32_t nchunks = (nb + MT_CB - 1) / MT_CB;
    const uint32_t c_begin = slice * sp.cps, c_end = c_begin + sp.cps < nchunks ? c_begin + sp.cps : nchunks;
    fetch(c_begin);
    for (uint32_t c = c_begin; c < c_end; ++c) {
        stage(c);
        __syncthreads();
        if (c + 1 < c_end) fetch(c + 1);
        const uint32_t count = nb - c * MT_CB < (uint32_t)MT_CB ? nb - c * MT_CB : (uint32_t)MT_CB;
        auto block_sums = [&](uint32_t bb, v4i S[2]) {
            const uint2 av = wqa[bb][l / 16][wrow0 + l % 16];
            const long A = (long)(((unsigned long)av.y << 32) | av.x);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint2 bv = xqb[bb][l / 16][wtok0 + 16 * j + l % 16];
                const long B = (long)(((unsigned long)bv.y << 32) | bv.x);
                S[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, zero, 0, 0, 0);
            }
        };
        auto epilogue = [&](uint32_t bb, const v4i S[2]) {
            const float4 ws4 = *(const float4 *)&wsl[bb][wrow0 + 4 * (l / 16)];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (SUMS) {
                    const uint32_t t = t0 + wtok0 + 16 * j + l % 16, b = c * MT_CB + bb;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const uint32_t r = r0 + wrow0 + 4 * (l / 16) + v;
                        if (r < I.rows && t < a.ntok) sums[((size_t)t * I.rows + r) * nb + b] = S[j][v];
                    }
                } else {
                    const float xsc = xsl[bb][wtok0 + 16 * j + l % 16];
                    acc[j][0] = __builtin_fmaf(ws4.x * xsc, (float)S[j][0], acc[j][0]);
                    acc[j][1] = __builtin_fmaf(ws4.y * xsc, (float)S[j][1], acc[j][1]);
                    acc[j][2] = __builtin_fmaf(ws4.z * xsc, (float)S[j][2], acc[j][2]);
                    acc[j][3] = __builtin_fmaf(ws4.w * xsc, (float)S[j][3], acc[j][3]);
                }
            }
        };
        if (count == (uint32_t)MT_CB) {
            /* four blocks' MFMAs at a time (eight independent ones per wave),
             * then their scale epilogue in block order: few accumulation
             * registers live, so three waves fit per SIMD */
#pragma unroll
            for (int h0 = 0; h0 < MT_CB; h0 += 4) {
                constexpr int G = 4;
                v4i S[G][2];
#pragma unroll
                for (int bb = 0; bb < G; ++bb)
                    if (h0 + bb < MT_CB) block_sums(h0 + bb, S[bb]);
#pragma unroll
                for (int bb = 0; bb < G; ++bb)
                    if (h0 + bb < MT_CB) epilogue(h0 + bb, S[bb]);
            }
        } else {
            for (uint32_t bb = 0; bb < count; ++bb) {
                v4i S[2];
                block_sums(bb, S);
                epilogue(bb, S);
            }
        }
        __syncthreads();
    }
    if (!SUMS) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t r = r0 + wrow0 + 4 * (l / 16) + v, t = t0 + wtok0 + 16 * j + l % 16;
                if (r < I.rows && t < a.ntok) {
                    if (sp.slices > 1)
                        sp.part[((size_t)slice * a.ntok + t) * sp.total_rows + I.tile_begin * MT_R + r] = acc[j][v];
                    else
                        store_out(I, a.flag, t, r, acc[j][v]);
                }
            }
    }
}

/* The slices' partial sums added in slice order, then bias, finiteness and the residual add. */
__global__ __launch_bounds__(WG) void k_mfma_reduce(MatArgs a, MfmaSplit sp) {
    const uint64_t gi = (uint64_t)blockIdx.x * WG + threadIdx.x;
    if (gi >= (uint64_t)a.ntok * sp.total_rows) return;
    const uint32_t t = (uint32_t)(gi / sp.total_rows), rr = (uint32_t)(gi % sp.total_rows);
    const Item &I = a.item[find_item(a, rr / MT_R)]; /* tile_begin counts MT_R-row tiles */
    const uint32_t r = rr - I.tile_begin * MT_R;
    if (r >= I.rows) return;
    float v = sp.part[(size_t)t * sp.total_rows + rr];
    for (uint32_t k = 1; k < sp.slices; ++k) v = v + sp.part[((size_t)k * a.ntok + t) * sp.total_rows + rr];
    store_out(I, a.flag, t, r, v);
}

/* ------------------------------------------------------------------------
 * Generic path: any alignment, any width. One thread per (row, token), byte
 * reads. Used for shapes the tiled kernels do not take (unaligned rows, odd
 * Q5 widths, nb > MAX_FAST_NB); same contract, bit for bit.
 * ---------------------------------------------------------------------- */
__device__ __forceinline__ uint32_t ld_u32_bytes(const unsigned char *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

template <bool Q5, bool FAST>
__global__ __launch_bounds__(WG) void k_generic(MatArgs a, uint32_t total_rows) {
    const uint64_t gi = (uint64_t)blockIdx.x * WG + threadIdx.x;
    if (gi >= (uint64_t)total_rows * a.ntok) return;
    const uint32_t t = (uint32_t)(gi / total_rows), fr = (uint32_t)(gi % total_rows);
    const Item &I = a.item[find_item(a, fr)];
    const uint32_t r = fr - I.tile_begin;
    const unsigned char *row = I.w + (size_t)r * I.row_bytes;
    const float *xd = a.xd + (size_t)t * a.xstride;
    const int8_t *xq = a.xq + (size_t)t * a.xstride * QK;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < a.nb; ++b) {
        float ws;
        int8_t wv[32];
        if (Q5) {
            const unsigned char *blk = row + (size_t)b * Q5_BYTES;
            ws = half_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            const uint32_t high = ld_u32_bytes(blk + 2);
            for (int j = 0; j < 16; ++j) {
                wv[j] = (int8_t)((int)((blk[6 + j] & 15u) | (((high >> j) & 1u) << 4)) - 16);
                wv[j + 16] = (int8_t)((int)((blk[6 + j] >> 4) | (((high >> (j + 16)) & 1u) << 4)) - 16);
            }
        } else {
            const unsigned char *blk = row + (size_t)b * Q8_BYTES;
            ws = __uint_as_float(ld_u32_bytes(blk));
            for (int j = 0; j < 32; ++j) wv[j] = (int8_t)blk[4 + j];
        }
        const float d = ws * xd[b];
        for (int l = 0; l < 8; ++l) {
            int s = 0;
            for (int k = 0; k < 4; ++k) s += (int)wv[4 * l + k] * (int)xq[b * QK + 4 * l + k];
            acc[l] = lane_step<FAST>(acc[l], d, s);
        }
    }
    const float p04 = acc[0] + acc[4], p15 = acc[1] + acc[5], p26 = acc[2] + acc[6], p37 = acc[3] + acc[7];
    const float e = p04 + p26, o = p15 + p37;
    store_out(I, a.flag, t, r, e + o);
}

/* ------------------------------------------------------------------------
 * Activation quantizer (reference: src/kernels.c:912-935). One thread per
 * element of the zero-padded row; a block of 32 is half a wave. amax is a
 * max-reduction (order-free: max is exact); scale = amax / 127 (correctly
 * rounded); inv = 1/scale when scale >= FLT_MIN, else 0; q = clamp(rint(x*inv)).
 * ---------------------------------------------------------------------- */
__global__ __launch_bounds__(WG) void k_quantize_q8(const float *x, uint32_t rows, uint32_t n, uint32_t nb, float *d,
                                                    int8_t *q, int *flag) {
    const uint64_t gi = (uint64_t)blockIdx.x * WG + threadIdx.x;
    const uint64_t per_row = (uint64_t)nb * QK;
    const bool in_range = gi < per_row * rows;
    const uint32_t row = in_range ? (uint32_t)(gi / per_row) : 0u;
    const uint32_t rem = (uint32_t)(gi % per_row), b = rem / QK, j = rem % QK;
    const bool valid = in_range && b * QK + j < n;
    const float v = valid ? x[(size_t)row * n + b * QK + j] : 0.0f;
    const float av = fabsf(v);
    int bad = valid && !(av <= FLT_MAX);
    float m = av;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 32);
        m = o > m ? o : m;
        bad |= __shfl_xor(bad, off, 32);
    }
    if (!in_range) return;
    const float scale = m / 127.0f;
    const float inv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
    int qv = 0;
    if (valid) {
        const float p = v * inv;
        qv = (int)__builtin_rintf(p);
        qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
    }
    q[(size_t)row * per_row + rem] = (int8_t)qv;
    if (j == 0) {
        d[(size_t)row * nb + b] = scale;
        if (bad && flag) *flag = 1;
    }
}

/* ------------------------------------------------------------------------
 * Activation producers (reference: src/model.c:334-415, src/vecmath.c:61-93).
 * One workgroup of NT threads per token row (256 for rows up to 4096
 * elements, so that many rows run at once; 1024 for longer ones; 512 for
 * rows up to 8192 measured no faster on the 4864-wide SwiGLU rows): optional
 * RMSNorm (sequential f32 sum of squares, model.c:337 — the squares are formed
 * in parallel, one wave adds them in element order), optional SwiGLU / GeGLU
 * with the binary64 exp below, then the Q8 block quantization of
 * kernels.c:912-935, written straight to d/q. Element i lives in thread
 * i % NT, register i / NT.
 * ---------------------------------------------------------------------- */
constexpr int RW_WG = 1024, RW_NARROW = 256;
constexpr int RW_EPT = 16; /* elements per thread: rows up to 16384 (4096 at 256 threads) */

template <bool NORM, int ACT, int NT>
__global__ __launch_bounds__(NT) void k_row_quantize(const float *src, const float *norm, float eps,
                                                       const float *gate, uint32_t n, float *yout, float *d,
                                                       int8_t *q, int *flag) {
    extern __shared__ __attribute__((aligned(16))) float sq_lds[]; /* NORM: the n squares (4*ceil(n/4) floats) */
    __shared__ float s_inv;
    __shared__ int s_bad;
    const uint32_t tid = threadIdx.x, row = blockIdx.x, nb = (n + QK - 1) / QK, np = nb * QK;
    const float *x = src + (size_t)row * n;
    float v[RW_EPT];
#pragma unroll
    for (int k = 0; k < RW_EPT; ++k) {
        const uint32_t i = tid + k * NT;
        v[k] = i < n ? x[i] : 0.0f;
    }
    if (NORM) {
#pragma unroll
        for (int k = 0; k < RW_EPT; ++k) {
            const uint32_t i = tid + k * NT;
            if (i < n) sq_lds[i] = v[k] * v[k];
        }
        __syncthreads();
        if (tid < 64) { /* the whole first wave runs the chain; lane 63 ends with the sum */
            const float sq = serial_sum_wave(sq_lds, n);
            if (tid == 63) {
                const float inv = 1.0f / sqrtf(sq / (float)n + eps); /* model.c:338 */
                s_inv = inv;
                s_bad = !(fabsf(sq) <= FLT_MAX) || !(fabsf(inv) <= FLT_MAX);
            }
        }
        __syncthreads();
        const float inv = s_inv;
        if (s_bad && tid == 0 && flag) *flag = 1;
#pragma unroll
        for (int k = 0; k < RW_EPT; ++k) {
            const uint32_t i = tid + k * NT;
            if (i < n) {
                const float t = v[k] * inv;
                v[k] = t * norm[i]; /* model.c:340 */
            }
        }
    }
    if (ACT) {
        const float *g = gate + (size_t)row * n;
#pragma unroll
        for (int k = 0; k < RW_EPT; ++k) {
            const uint32_t i = tid + k * NT;
            if (i < n) {
                const float gv = g[i];
                float e;
                if (ACT == 1) {
                    e = exp_det(-gv);
                } else {
                    const float g3 = 0.044715f * gv * gv * gv;
                    const float u = 1.5957691216f * (gv + g3);
                    e = exp_det(-u);
                }
                const float den = 1.0f + e;
                const float sg = gv / den;
                v[k] = v[k] * sg;
            }
        }
    }
    if (yout) {
#pragma unroll
        for (int k = 0; k < RW_EPT; ++k) {
            const uint32_t i = tid + k * NT;
            if (i < n) yout[(size_t)row * n + i] = v[k];
        }
    }
    /* Q8 blocks: 32 consecutive elements = 32 consecutive threads of one k */
#pragma unroll
    for (int k = 0; k < RW_EPT; ++k) {
        const uint32_t i = tid + k * NT;
        if (k * NT >= np) break; /* uniform */
        const bool valid = i < n;
        const float av = fabsf(v[k]);
        int bad = valid && !(av <= FLT_MAX);
        float m = valid ? av : 0.0f;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) {
            const float o = __shfl_xor(m, off, 32);
            m = o > m ? o : m;
            bad |= __shfl_xor(bad, off, 32);
        }
        if (i < np) {
            const float scale = m / 127.0f;
            const float inv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
            int qv = 0;
            if (valid) {
                const float p = v[k] * inv;
                qv = (int)__builtin_rintf(p);
                qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
            }
            q[(size_t)row * np + i] = (int8_t)qv;
            if ((i & 31u) == 0) {
                d[(size_t)row * nb + i / QK] = scale;
                if (bad && flag) *flag = 1;
            }
        }
    }
}

/* h[i] = h[i] * (g / (1 + exp_det(-g))) with g = gate[i] (SwiGLU, act 1) or
 * the GeGLU form (act 2), vecmath.c:78-93: the gated product alone, for
 * callers that quantize later. */
__global__ __launch_bounds__(WG) void k_glu(float *h, const float *gate, uint32_t n, int act) {
    const uint32_t i = blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    const float gv = gate[i];
    float e;
    if (act == 2) {
        const float g3 = 0.044715f * gv * gv * gv;
        const float u = 1.5957691216f * (gv + g3);
        e = exp_det(-u);
    } else {
        e = exp_det(-gv);
    }
    const float den = 1.0f + e;
    const float sg = gv / den;
    h[i] = h[i] * sg;
}

/* ------------------------------------------------------------------------
 * Decoder pieces around the matmuls.
 * ---------------------------------------------------------------------- */

/* RoPE on q and k, then k and v into the KV cache (model.c:511-526): one
 * workgroup per token. Adjacent pairs (2i, 2i+1), i < pairs, of every head
 * rotate by the (cos, sin) table row of the token's absolute position
 * (model.c:442-450); the other coordinates pass through. The cache holds
 * kv_dim floats per position; a position at or past the context is refused
 * (flag) rather than written. */
__global__ __launch_bounds__(256) void k_rope_kv(float *q, float *k, const float *v, AttnShape sh, const float *cs,
                                                 const float *sn, float *kcache, float *vcache, uint32_t pos0,
                                                 const int32_t *pos_dev, int *flag) {
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t p = (pos_dev ? (uint32_t)*pos_dev : pos0) + t;
    if (p >= sh.context) {
        if (tid == 0 && flag) *flag = 1;
        return;
    }
    float *qt = q + (size_t)t * sh.q_dim;
    float *kt = k + (size_t)t * sh.kv_dim;
    const float *vt = v + (size_t)t * sh.kv_dim;
    const float *ct = cs + (size_t)p * sh.pairs, *st = sn + (size_t)p * sh.pairs;
    float *kslot = kcache + (size_t)p * sh.kv_dim;
    float *vslot = vcache + (size_t)p * sh.kv_dim;
    const uint32_t qpairs = sh.heads * sh.pairs, kpairs = sh.kv_heads * sh.pairs;
    for (uint32_t i = tid; i < qpairs + kpairs; i += 256) {
        const bool isq = i < qpairs;
        const uint32_t j = isq ? i : i - qpairs, h = j / sh.pairs, pr = j % sh.pairs;
        float *x = (isq ? qt : kt) + (size_t)h * sh.head_dim + 2 * pr;
        const float a = x[0], b = x[1];
        const float ac = a * ct[pr], bs = b * st[pr], as = a * st[pr], bc = b * ct[pr];
        const float r0 = ac - bs, r1 = as + bc;
        x[0] = r0;
        x[1] = r1;
        if (!isq) {
            kslot[(size_t)h * sh.head_dim + 2 * pr] = r0;
            kslot[(size_t)h * sh.head_dim + 2 * pr + 1] = r1;
        }
    }
    /* the unrotated tail of each k head, and all of v */
    for (uint32_t i = tid; i < sh.kv_dim; i += 256) {
        vslot[i] = vt[i];
        if (i % sh.head_dim >= 2 * sh.pairs) kslot[i] = kt[i];
    }
}

/* Attention of one query head of one token over KV positions [start, pos]
 * (kernels.c:1154-1176, model.c:459-491), for the 32 output coordinates
 * [32g, 32g+32) of the head: workgroup (t, h, g), 512 threads.
 *  0. the first pass of V rows and each thread's first two K rows are
 *     requested before anything else, so their latencies overlap;
 *  1. scores: one thread per position, the 8-lane dot_f32 of kernels.c:1119-
 *     1127 (acc[l] += q[e+l]*k[e+l] over groups of 8, lane tree, tail in
 *     order), times 1/sqrt(hd);
 *  2. the maximum (order-free) and exp_det(s - max) in parallel;
 *  3. the total in position order by one lane, inv = 1/total;
 *  4. the products (s_p*inv)*v_p[j] of ATT_CH rows at a time go to LDS in
 *     parallel, then lane j of wave 0 adds them in position order while the
 *     next rows load.
 * Every workgroup of a head recomputes steps 1-3 (the same values), so a
 * head's value sums spread over ceil(hd/32) workgroups. With xd/xq
 * (head_dim % 32 == 0) the workgroup also quantizes its block of the
 * attention row (quantize_attention, model.c:402-406). */
constexpr uint32_t ATT_WG = 512;
constexpr uint32_t ATT_JW = 32;   /* output coordinates per workgroup: one Q8 block */
constexpr uint32_t ATT_CH = 256;  /* value rows per LDS pass */
constexpr uint32_t ATT_CHP = ATT_CH + 4; /* products column pitch: lanes' 16-byte reads spread over banks */
constexpr uint32_t ATT_PRE = ATT_CH * ATT_JW / 4 / ATT_WG; /* float4 V loads per thread per pass */
constexpr uint32_t ATT_KT = 256;  /* K rows per LDS tile (head_dim <= 64) */
constexpr uint32_t ATT_KTL = ATT_KT * 16 / ATT_WG; /* float4 K loads per thread per tile */
constexpr uint32_t ATT_SHARED = ATT_KT * 68 > ATT_CHP * ATT_JW ? ATT_KT * 68 : ATT_CHP * ATT_JW; /* floats */

struct DotAcc {
    float a[8];
};

/* acc[l] += q[8g+l] * k[8g+l] for the groups g of kr (2 float4 each). */
__device__ __forceinline__ void dot_groups(DotAcc &acc, const float4 *kr, const float4 *q4, uint32_t g0,
                                           uint32_t ng) {
#pragma unroll
    for (uint32_t e = 0; e < 8; ++e) {
        if (e < ng) {
            const float4 ka = kr[2 * e], kb = kr[2 * e + 1];
            const float4 qa = q4[2 * (g0 + e)], qb = q4[2 * (g0 + e) + 1];
            float p;
            p = qa.x * ka.x; acc.a[0] = acc.a[0] + p;
            p = qa.y * ka.y; acc.a[1] = acc.a[1] + p;
            p = qa.z * ka.z; acc.a[2] = acc.a[2] + p;
            p = qa.w * ka.w; acc.a[3] = acc.a[3] + p;
            p = qb.x * kb.x; acc.a[4] = acc.a[4] + p;
            p = qb.y * kb.y; acc.a[5] = acc.a[5] + p;
            p = qb.z * kb.z; acc.a[6] = acc.a[6] + p;
            p = qb.w * kb.w; acc.a[7] = acc.a[7] + p;
        }
    }
}

/* The lane tree of kernels.c:40-50, then the tail elements in order. */
__device__ __forceinline__ float dot_finish(const DotAcc &acc, const float *qv, const float *kp, uint32_t from,
                                            uint32_t hd) {
    const float p04 = acc.a[0] + acc.a[4], p15 = acc.a[1] + acc.a[5], p26 = acc.a[2] + acc.a[6],
                p37 = acc.a[3] + acc.a[7];
    const float ev = p04 + p26, od = p15 + p37;
    float sum = ev + od;
    for (uint32_t e = from; e < hd; ++e) {
        const float p = qv[e] * kp[e];
        sum = sum + p;
    }
    return sum;
}

/* K tile rows [tb, tb + ATT_KT) of one head (head_dim = 4*q4n <= 64) into
 * registers: float4 f = tid + u*ATT_WG is element 4c of row f / q4n. Rows
 * past np re-read the last row (in bounds, never used). */
__device__ __forceinline__ void att_load_tile(float4 (&kr)[ATT_KTL], const float *kbase, uint32_t kvd, uint32_t q4n,
                                              uint32_t np, uint32_t tb, uint32_t tid) {
    const uint32_t trows = np - tb < ATT_KT ? np - tb : ATT_KT;
#pragma unroll
    for (uint32_t u = 0; u < ATT_KTL; ++u) {
        const uint32_t f = tid + u * ATT_WG, r = f / q4n, c = f - r * q4n;
        const uint32_t rr = r < trows ? r : trows - 1;
        kr[u] = *(const float4 *)(kbase + (size_t)(tb + rr) * kvd + 4 * c);
    }
}
__device__ __forceinline__ void att_store_tile(float *kt, const float4 (&kr)[ATT_KTL], uint32_t q4n, uint32_t kpitch,
                                               uint32_t trows, uint32_t tid) {
#pragma unroll
    for (uint32_t u = 0; u < ATT_KTL; ++u) {
        const uint32_t f = tid + u * ATT_WG, r = f / q4n, c = f - r * q4n;
        if (r < trows) *(float4 *)&kt[r * kpitch + 4 * c] = kr[u];
    }
}

__global__ __launch_bounds__(ATT_WG) void k_attend(const float *q, const float *kcache, const float *vcache, float *att,
                                                   AttnShape sh, uint32_t pos0, const int32_t *pos_dev, int *flag,
                                                   float *xd, int8_t *xq) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ __attribute__((aligned(16))) float qv[MAX_HEAD_DIM];
    __shared__ float red[ATT_WG / 64];
    __shared__ float s_inv;
    const uint32_t tid = threadIdx.x, hd = sh.head_dim, ngrp = (hd + ATT_JW - 1) / ATT_JW;
    const uint32_t g = blockIdx.x % ngrp, th = blockIdx.x / ngrp, t = th / sh.heads, h = th % sh.heads;
    const uint32_t kh = h / (sh.heads / sh.kv_heads), kvd = sh.kv_dim, j0 = g * ATT_JW;
    const uint32_t jw = hd - j0 < ATT_JW ? hd - j0 : ATT_JW; /* coordinates this group owns */
    const uint32_t pos = (pos_dev ? (uint32_t)*pos_dev : pos0) + t;
    if (pos >= sh.context) { /* the scores row holds at most context positions */
        if (tid == 0 && flag) *flag = 1;
        return;
    }
    const uint32_t start = sh.window && pos >= sh.window ? pos - sh.window + 1 : 0, np = pos - start + 1;
    float *sc = lds;
    float *prod = lds + ((sh.context + 3) & ~3u); /* [ATT_JW][ATT_CHP]: column j holds its rows in order */
    const bool vec = (hd & 3) == 0 && ((uintptr_t)kcache & 15) == 0 && ((uintptr_t)vcache & 15) == 0;
    const float *kbase = kcache + (size_t)start * kvd + (size_t)kh * hd;
    const float *vbase = vcache + (size_t)start * kvd + (size_t)kh * hd + j0;
    const uint32_t groups = hd / 8;

    /* 0. V pass 0 and the first K rows, requested up front */
    const uint32_t fq = ATT_JW / 4; /* float4 per row segment */
    const uint32_t frow = tid / fq, fcol = (tid % fq) * 4;
    float4 pre[ATT_PRE];
    auto load_pass = [&](uint32_t p0) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t u = 0; u < ATT_PRE; ++u) {
            const uint32_t r = frow + u * (ATT_WG / fq), p = p0 + r;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p < np) {
                const float *src = vbase + (size_t)p * kvd + fcol;
                if (vec && fcol + 4 <= jw) {
                    v = *(const float4 *)src;
                } else {
                    if (fcol + 0 < jw) v.x = src[0];
                    if (fcol + 1 < jw) v.y = src[1];
                    if (fcol + 2 < jw) v.z = src[2];
                    if (fcol + 3 < jw) v.w = src[3];
                }
            }
            pre[u] = v;
        }
    };
    load_pass(0);
    /* K tiles (head_dim <= 64): rows loaded coalesced (hd/4 float4 per row,
     * consecutive threads along a row), stored row-major in LDS with a pitch
     * of hd+4 floats so that the row-per-thread 16-byte reads below do not
     * conflict. */
    const bool fast = vec && hd <= 64;
    const uint32_t q4n = hd / 4, kpitch = hd + 4;
    float *kt = prod; /* shares the products region (used later) */
    const float *qh = q + (size_t)t * sh.q_dim + (size_t)h * hd;
    for (uint32_t j = tid; j < hd; j += ATT_WG) qv[j] = qh[j];
    __syncthreads();

    /* 1. scores */
    const float factor = 1.0f / sqrtf((float)hd);
    const float4 *q4 = (const float4 *)qv;
    uint32_t i = tid;
    if (fast) {
        for (uint32_t tb = 0; tb < np; tb += ATT_KT) {
            const uint32_t trows = np - tb < ATT_KT ? np - tb : ATT_KT;
            float4 kr[ATT_KTL];
            att_load_tile(kr, kbase, kvd, q4n, np, tb, tid);
            att_store_tile(kt, kr, q4n, kpitch, trows, tid);
            __syncthreads();
            if (tid < trows) {
                const float4 *row = (const float4 *)&kt[tid * kpitch];
                float4 k4[16];
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u) k4[u] = row[u < q4n ? u : q4n - 1];
                DotAcc acc = {{0, 0, 0, 0, 0, 0, 0, 0}};
                dot_groups(acc, k4, q4, 0, groups);
                sc[tb + tid] = dot_finish(acc, qv, kbase + (size_t)(tb + tid) * kvd, groups * 8, hd) * factor;
            }
            __syncthreads();
        }
        i = np;
    }
    for (; i < np; i += ATT_WG) { /* further rows, or head_dim > 64 */
        const float *kp = kbase + (size_t)i * kvd;
        DotAcc acc = {{0, 0, 0, 0, 0, 0, 0, 0}};
        if (vec) {
            const float4 *k4 = (const float4 *)kp;
            for (uint32_t g0 = 0; g0 < groups; g0 += 8) { /* 64 floats of the row in flight */
                const uint32_t ng = groups - g0 < 8 ? groups - g0 : 8, last = 2 * ng - 1;
                float4 kr[16];
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u) kr[u] = k4[2 * g0 + (u < last ? u : last)];
                dot_groups(acc, kr, q4, g0, ng);
            }
        } else {
            for (uint32_t e = 0; e < groups; ++e)
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    const float p = qv[8 * e + l] * kp[8 * e + l];
                    acc.a[l] = acc.a[l] + p;
                }
        }
        sc[i] = dot_finish(acc, qv, kp, groups * 8, hd) * factor;
    }
    __syncthreads();

    /* 2. max (order-free; NaN never wins, as in softmax_inv), exp */
    float m = -FLT_MAX;
    for (uint32_t r = tid; r < np; r += ATT_WG) m = sc[r] > m ? sc[r] : m;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float high = red[0];
#pragma unroll
    for (uint32_t w = 1; w < ATT_WG / 64; ++w) high = red[w] > high ? red[w] : high;
    for (uint32_t r = tid; r < np; r += ATT_WG) sc[r] = exp_det(sc[r] - high);
    __syncthreads();

    /* 3. the total in position order */
    if (tid < 64) { /* the whole first wave runs the chain; lane 63 ends with the total */
        const float tot = serial_sum_wave(sc, np);
        if (tid == 63) s_inv = 1.0f / tot;
    }
    __syncthreads();
    const float inv = s_inv;

    /* 4. weighted values: products in parallel, sums in order */
    float o = 0.0f;
    for (uint32_t p0 = 0; p0 < np; p0 += ATT_CH) {
        /* kernels.c:1165: w = scores[p] * inv, then w * v[j] */
#pragma unroll
        for (uint32_t u = 0; u < ATT_PRE; ++u) {
            const uint32_t r = frow + u * (ATT_WG / fq), p = p0 + r;
            if (p < np) {
                const float w = sc[p] * inv;
                prod[(fcol + 0) * ATT_CHP + r] = w * pre[u].x;
                prod[(fcol + 1) * ATT_CHP + r] = w * pre[u].y;
                prod[(fcol + 2) * ATT_CHP + r] = w * pre[u].z;
                prod[(fcol + 3) * ATT_CHP + r] = w * pre[u].w;
            }
        }
        __syncthreads();
        if (p0 + ATT_CH < np) load_pass(p0 + ATT_CH); /* next pass in flight during the sums */
        if (tid < ATT_JW) {
            /* lane j adds its column's rows in order: 16-byte reads, one batch of
             * 8 reads in flight while the previous batch is added */
            const uint32_t rows = np - p0 < ATT_CH ? np - p0 : ATT_CH;
            const float *colp = prod + tid * ATT_CHP;
            float acc = o;
            acc = chain_lds(acc, colp, rows); /* kernels.c:1165, position order */
            o = acc;
        }
        __syncthreads();
    }
    if (tid < ATT_JW) {
        const bool valid = tid < jw;
        if (valid) att[(size_t)t * sh.q_dim + (size_t)h * hd + j0 + tid] = o;
        if (xd) { /* this workgroup's 32 coordinates are one block (kernels.c:912-935) */
            const float v = valid ? o : 0.0f, av = fabsf(v);
            float mx = av;
            int bad = valid && !(av <= FLT_MAX);
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) {
                const float ot = __shfl_xor(mx, off, 32);
                mx = ot > mx ? ot : mx;
                bad |= __shfl_xor(bad, off, 32);
            }
            const float scale = mx / 127.0f;
            const float qinv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
            const uint32_t nbq = (sh.q_dim + QK - 1) / QK, blk = (h * hd + j0) / QK;
            if (valid) {
                const float pq = v * qinv;
                int qi = (int)__builtin_rintf(pq);
                qi = qi > 127 ? 127 : (qi < -127 ? -127 : qi);
                xq[((size_t)t * nbq + blk) * QK + tid] = (int8_t)qi;
            }
            if (tid == 0) {
                xd[(size_t)t * nbq + blk] = scale;
                if (bad && flag) *flag = 1;
            }
        }
    }
}

/* Attention for head_dim 64 (16-byte aligned caches): the arithmetic of
 * k_attend, laid out so that a decode step pays one memory round trip before
 * the two serial sums.
 *  0. every load is issued first: the K rows of up to AR_KR positions
 *     (coalesced: 16 threads per row, AR_KU float4 per thread held in
 *     registers), the first AR_VP value rows of this workgroup's 32
 *     coordinates, q and the exp table;
 *  1. scores: the rows pass through LDS AR_KT at a time; one thread per
 *     position forms the 8-lane dot_f32 of kernels.c:1119-1127 (lane tree,
 *     times 1/sqrt(hd));
 *  2. maximum (order-free) and exp_det(s - max) in parallel;
 *  3. the total in position order by one lane, inv = 1/total;
 *  4. the products (s_p*inv)*v_p[j] of AR_VP rows at a time to LDS, then lane
 *     j adds its column in position order while the next rows load.
 * ROPE (one token, decode): q and this position's k arrive unrotated, as the
 * QKV matmul left them; the workgroup rotates q and this position's k row
 * into LDS (model.c:442-450, 511-526), and the first workgroup of each KV
 * head stores the rotated k and the v row into the caches. The other workgroups read the caches only below
 * the current position, so no workgroup waits for another. */
constexpr uint32_t AR_WG = 512;
constexpr uint32_t AR_HD = 64;                           /* head_dim of this kernel */
constexpr uint32_t AR_Q4 = AR_HD / 4;                    /* float4 per K row */
constexpr uint32_t AR_KU = 32;                           /* float4 K loads per thread per round */
constexpr uint32_t AR_KR = AR_KU * AR_WG / AR_Q4;        /* positions per round: 1024 */
constexpr uint32_t AR_KT = 256;                          /* K rows per LDS tile */
constexpr uint32_t AR_KTU = AR_KT * AR_Q4 / AR_WG;       /* float4 loads per thread per tile: 8 */
constexpr uint32_t AR_KP = AR_HD + 4;                    /* K tile row pitch (floats) */
constexpr uint32_t AR_VP = 640;                          /* value rows per pass (a 512-token prompt and 128 steps: one) */
constexpr uint32_t AR_VPP = AR_VP + 4;                   /* products column pitch (floats) */
constexpr uint32_t AR_PF = ATT_JW * AR_VPP + ATT_JW / 4 * 8; /* products floats (see att_col) */
constexpr uint32_t AR_VL = AR_VP * ATT_JW / 4 / AR_WG;   /* float4 value loads per thread per pass */
constexpr uint32_t AR_FIXED = AR_PF > AR_KT * AR_KP ? AR_PF : AR_KT * AR_KP; /* LDS floats */

/* Start of product column j: pitch AR_VPP (4 mod 32) plus 8 floats per group of
 * four columns, so one wave's writes (8 rows x 8 groups of four columns) put
 * two lanes on a bank instead of four. 16-byte aligned for the chains' reads. */
__device__ __forceinline__ uint32_t att_col(uint32_t j) {
    static_assert(AR_VPP % 32 == 4, "bank pattern");
    return j * AR_VPP + j / 4 * 8;
}

struct RopeRows {
    const float *k, *v;    /* this token's k and v rows (kv_dim each), unrotated */
    const float *cs, *sn;  /* rotation tables, `pairs` floats per absolute position */
};

/* Rotation of float4 u of a head row (elements 4u..4u+3 = pairs 2u, 2u+1)
 * by table row (c, s): x0' = x0*c - x1*s, x1' = x0*s + x1*c (model.c:447-448). */
__device__ __forceinline__ float4 rope4(float4 x, uint32_t u, uint32_t pairs, const float *c, const float *s) {
    if (2 * u < pairs) {
        const float a = x.x, b = x.y, cc = c[2 * u], ss = s[2 * u];
        const float ac = a * cc, bs = b * ss, as = a * ss, bc = b * cc;
        x.x = ac - bs;
        x.y = as + bc;
    }
    if (2 * u + 1 < pairs) {
        const float a = x.z, b = x.w, cc = c[2 * u + 1], ss = s[2 * u + 1];
        const float ac = a * cc, bs = b * ss, as = a * ss, bc = b * cc;
        x.z = ac - bs;
        x.w = as + bc;
    }
    return x;
}

/* K rows p0 + krow + u*(AR_WG/AR_Q4), float4 kcol of each, for the slabs u
 * that start below np; rows at or past `lim` re-read row 0 (in bounds,
 * never used). */
__device__ __forceinline__ void att_rows_keys(f4v (&kr)[AR_KU], const float *kbase, uint32_t kvd, uint32_t p0,
                                              uint32_t np, uint32_t lim, uint32_t krow, uint32_t kcol) {
#pragma unroll
    for (uint32_t u = 0; u < AR_KU; ++u) {
        const uint32_t p = p0 + krow + u * (AR_WG / AR_Q4);
        if (p0 + u * (AR_WG / AR_Q4) < np) /* uniform across the workgroup */
            kr[u] = *(const f4v *)(kbase + (size_t)(p < lim ? p : 0) * kvd + 4 * kcol);
    }
}

/* V rows [p0, p0 + AR_VP) of a workgroup's 32 coordinates (vrow/vcol: this
 * thread's row and float4 column), ROPE: the current position's row from vrope. */
template <bool ROPE>
__device__ __forceinline__ void att_load_values(float4 (&pre)[AR_VL], const float *vbase, const float *vrope,
                                                uint32_t kvd, uint32_t p0, uint32_t np, uint32_t last,
                                                uint32_t vrow, uint32_t vcol) {
#pragma unroll
    for (uint32_t u = 0; u < AR_VL; ++u) {
        const uint32_t p = p0 + vrow + u * (AR_WG * 4 / ATT_JW);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (p < np)
            v = *(const float4 *)((ROPE && p == last) ? vrope + vcol : vbase + (size_t)p * kvd + vcol);
        pre[u] = v;
    }
}

/* Steps 2-4 of the row attention once the scaled scores sc[0, np) are in LDS
 * and each thread holds the maximum of its own (high): the maximum
 * (order-free, NaN never wins as in softmax_inv, kernels.c:1146-1148),
 * exp_det(s - max) in parallel, the total in position order by one lane,
 * then the products (s_p*inv)*v_p[j] of AR_VP rows at a time to LDS and lane
 * j's sum of its column in position order (kernels.c:1165), the next rows
 * loading meanwhile. pre holds the first value rows. The 32 outputs go to
 * out[0, 32); with xd, their Q8 block to *xd / xq[0, 32) (kernels.c:912-935). */
template <bool ROPE>
__device__ __forceinline__ void att_tail(float high, float *sc, float *prod, uint32_t np, uint32_t last,
                                         float4 (&pre)[AR_VL], const float *vbase, const float *vrope,
                                         uint32_t kvd, uint32_t vrow, uint32_t vcol, const uint64_t *etab,
                                         float *red, float *s_inv, float *out, float *xd, int8_t *xq, int *flag) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(high, off, 64);
        high = o > high ? o : high;
    }
    if ((tid & 63) == 0) red[tid >> 6] = high;
    __syncthreads();
    high = red[0];
#pragma unroll
    for (uint32_t w = 1; w < AR_WG / 64; ++w) high = red[w] > high ? red[w] : high;
    for (uint32_t p = tid; p < np; p += AR_WG) sc[p] = exp_det_tab(sc[p] - high, etab);
    __syncthreads();

    if (tid < 64) { /* the whole first wave runs the chain; lane 63 ends with the total */
        const float tot = serial_sum_wave(sc, np);
        if (tid == 63) *s_inv = 1.0f / tot;
    }
    __syncthreads();
    const float inv = *s_inv;

    float o = 0.0f;
    for (uint32_t p0 = 0; p0 < np; p0 += AR_VP) {
#pragma unroll
        for (uint32_t u = 0; u < AR_VL; ++u) { /* kernels.c:1165: w = scores[p] * inv, then w * v[j] */
            const uint32_t r = vrow + u * (AR_WG * 4 / ATT_JW), p = p0 + r;
            if (p < np) {
                const float w = sc[p] * inv;
                prod[att_col(vcol + 0) + r] = w * pre[u].x;
                prod[att_col(vcol + 1) + r] = w * pre[u].y;
                prod[att_col(vcol + 2) + r] = w * pre[u].z;
                prod[att_col(vcol + 3) + r] = w * pre[u].w;
            }
        }
        __syncthreads();
        if (p0 + AR_VP < np) /* next pass in flight during the sums */
            att_load_values<ROPE>(pre, vbase, vrope, kvd, p0 + AR_VP, np, last, vrow, vcol);
        if (tid < ATT_JW) {
            const uint32_t rows = np - p0 < AR_VP ? np - p0 : AR_VP;
            const float *colp = prod + att_col(tid);
            float acc = o;
            acc = chain_lds(acc, colp, rows); /* kernels.c:1165, position order */
            o = acc;
        }
        __syncthreads();
    }
    if (tid < ATT_JW) {
        out[tid] = o;
        if (xd) {
            const float av = fabsf(o);
            int bad = !(av <= FLT_MAX);
            const float mx = max32(av);
            bad = __ballot(bad) != 0;
            const float scale = mx / 127.0f;
            const float qinv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
            const float pq = o * qinv;
            int qi = (int)__builtin_rintf(pq);
            qi = qi > 127 ? 127 : (qi < -127 ? -127 : qi);
            xq[tid] = (int8_t)qi;
            if (tid == 0) {
                *xd = scale;
                if (bad && flag) *flag = 1;
            }
        }
    }
}

template <bool ROPE>
/* 2 waves per SIMD: the round's K rows stay in registers (no spills) */
__global__ __launch_bounds__(AR_WG) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_attend_rows(const float *q, float *kcache, float *vcache, float *att,
                                                       AttnShape sh, uint32_t pos0, const int32_t *pos_dev, int *flag,
                                                       float *xd, int8_t *xq, RopeRows rr) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ __attribute__((aligned(16))) float qv[AR_HD];
    __shared__ uint64_t etab[32];
    __shared__ float rtab[ROPE ? AR_HD : 1]; /* ROPE: cos then sin of this position (pairs <= 32 each) */
    __shared__ __attribute__((aligned(16))) float krot[ROPE ? AR_HD : 4]; /* ROPE: this position's rotated k */
    __shared__ float red[AR_WG / 64];
    __shared__ float s_inv;
    constexpr uint32_t ngrp = AR_HD / ATT_JW;
    const uint32_t tid = threadIdx.x;
    const uint32_t g = blockIdx.x % ngrp, th = blockIdx.x / ngrp, t = th / sh.heads, h = th % sh.heads;
    const uint32_t kh = h / (sh.heads / sh.kv_heads), kvd = sh.kv_dim, j0 = g * ATT_JW;
    const uint32_t pos = (pos_dev ? (uint32_t)*pos_dev : pos0) + t;
    if (pos >= sh.context) { /* the scores row holds at most context positions */
        if (tid == 0 && flag) *flag = 1;
        return;
    }
    const uint32_t start = sh.window && pos >= sh.window ? pos - sh.window + 1 : 0, np = pos - start + 1;
    const uint32_t last = np - 1; /* ROPE: the current position, taken from rr rather than the caches */
    float *sc = lds;
    float *shared = lds + ((sh.context + 3) & ~3u); /* K tiles, then the products (att_col) */
    float *prod = shared;
    float *kt = shared;
    const float *kbase = kcache + (size_t)start * kvd + (size_t)kh * AR_HD;
    const float *vbase = vcache + (size_t)start * kvd + (size_t)kh * AR_HD + j0;
    const float *crow = ROPE ? rtab : nullptr, *srow = ROPE ? rtab + AR_HD / 2 : nullptr;
    const bool keeper = ROPE && g == 0 && h % (sh.heads / sh.kv_heads) == 0; /* stores this KV head's cache row */

    /* 0. loads: value pass 0, the K rows of round 0, q, the exp table */
    const uint32_t vrow = tid / (ATT_JW / 4), vcol = (tid % (ATT_JW / 4)) * 4;
    float4 pre[AR_VL];
    const uint32_t krow = tid / AR_Q4, kcol = tid % AR_Q4; /* load u covers rows krow + u*(AR_WG/AR_Q4) */
    /* issue order = need order (loads complete in order): q, tables, K, V */
    const float *qh = q + (size_t)t * sh.q_dim + (size_t)h * AR_HD;
    float4 qx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (tid < AR_Q4) qx = *(const float4 *)(qh + 4 * tid);
    uint64_t ev = 0;
    if (tid >= 64 && tid < 96) ev = EXP2_TABLE[tid - 64];
    float rv = 0.0f;
    const uint32_t ri = tid - 256, rhalf = ri < sh.pairs ? 0 : 1, rj = ri - rhalf * sh.pairs;
    const bool rload = ROPE && tid >= 256 && tid < 256 + 2 * sh.pairs; /* pairs <= head_dim / 2 */
    if (rload) rv = (rhalf ? rr.sn : rr.cs)[(size_t)pos * sh.pairs + rj];
    float4 kx = make_float4(0.0f, 0.0f, 0.0f, 0.0f); /* ROPE: this position's k, float4 tid - 192 */
    const bool kown = ROPE && tid >= 192 && tid < 192 + AR_Q4;
    if (kown) kx = *(const float4 *)(rr.k + (size_t)kh * AR_HD + 4 * (tid - 192));
    f4v kr[AR_KU];
    att_rows_keys(kr, kbase, kvd, 0, np, ROPE ? last : np, krow, kcol);
    const float *vrope = ROPE ? rr.v + (size_t)kh * AR_HD + j0 : nullptr;
    att_load_values<ROPE>(pre, vbase, vrope, kvd, 0, np, last, vrow, vcol);
    if (rload) rtab[rhalf * (AR_HD / 2) + rj] = rv;
    if (ROPE) __syncthreads(); /* the table rows, before q and k are rotated */
    if (kown) {
        const uint32_t u = tid - 192;
        kx = rope4(kx, u, sh.pairs, crow, srow);
        *(float4 *)&krot[4 * u] = kx;
        if (keeper) *(float4 *)(kcache + (size_t)pos * kvd + (size_t)kh * AR_HD + 4 * u) = kx;
    }
    if (keeper && tid >= 128 && tid < 128 + AR_HD) /* v is stored as is (model.c:520-523) */
        vcache[(size_t)pos * kvd + (size_t)kh * AR_HD + (tid - 128)] = rr.v[(size_t)kh * AR_HD + (tid - 128)];
    if (tid < AR_Q4) {
        if (ROPE) qx = rope4(qx, tid, sh.pairs, crow, srow);
        *(float4 *)&qv[4 * tid] = qx;
    }
    if (tid >= 64 && tid < 96) etab[tid - 64] = ev;

    /* 1. scores */
    const float factor = 1.0f / sqrtf((float)AR_HD);
    float high = -FLT_MAX; /* NaN never wins, as in softmax_inv (kernels.c:1146-1148) */
    for (uint32_t p0 = 0; p0 < np; p0 += AR_KR) {
        if (p0) {
            __syncthreads(); /* the previous round's last tile is consumed */
            att_rows_keys(kr, kbase, kvd, p0, np, ROPE ? last : np, krow, kcol);
        }
#pragma unroll
        for (uint32_t tile = 0; tile < AR_KU / AR_KTU; ++tile) {
            const uint32_t tb = p0 + tile * AR_KT;
            if (tb < np) { /* uniform */
            if (tile || p0) __syncthreads(); /* the previous tile is consumed */
#pragma unroll
            for (uint32_t uu = 0; uu < AR_KTU; ++uu) {
                const uint32_t r = krow + uu * (AR_WG / AR_Q4);
                if (tb + r < np) *(f4v *)&kt[r * AR_KP + 4 * kcol] = kr[tile * AR_KTU + uu];
            }
            __syncthreads();
            if (tid < AR_KT && tb + tid < np) {
                const float4 *row = (ROPE && tb + tid == last) ? (const float4 *)krot : (const float4 *)&kt[tid * AR_KP];
                DotAcc acc = {{0, 0, 0, 0, 0, 0, 0, 0}};
                dot_groups(acc, row, (const float4 *)qv, 0, AR_HD / 8);
                const float p04 = acc.a[0] + acc.a[4], p15 = acc.a[1] + acc.a[5], p26 = acc.a[2] + acc.a[6],
                            p37 = acc.a[3] + acc.a[7];
                const float e2 = p04 + p26, o2 = p15 + p37;
                const float sv = (e2 + o2) * factor;
                sc[tb + tid] = sv;
                high = sv > high ? sv : high;
            }
            }
        }
    }

    const uint32_t nbq = sh.q_dim / QK, blk = (h * AR_HD + j0) / QK;
    att_tail<ROPE>(high, sc, prod, np, last, pre, vbase, vrope, kvd, vrow, vcol, etab, red,
                   &s_inv, att + (size_t)t * sh.q_dim + (size_t)h * AR_HD + j0, xd ? xd + (size_t)t * nbq + blk : nullptr,
                   xq ? xq + ((size_t)t * nbq + blk) * QK : nullptr, flag);
}

/* Decode attention in two launches (one token, head_dim 64): the K rows are
 * spread over many workgroups instead of being fetched by one workgroup per
 * head, the part of k_attend_rows that a single CU's load bandwidth bounds.
 * k_attend_scores: workgroup (block of AS_SP positions, KV head) forms the
 * scaled scores of every query head of the group (8-lane dot_f32, times
 * 1/sqrt(64)) into scores[h][p]; with ROPE it rotates q and this position's
 * k itself (model.c:442-450) and the workgroup holding the current position
 * stores the rotated k and the v row into the caches (model.c:511-526).
 * Workgroups past the current position leave at once (the grid covers the
 * context, so a captured step replays at any position). */
constexpr uint32_t AS_WG = 512;
constexpr uint32_t AS_SP = 32;                 /* positions per scores workgroup */
constexpr uint32_t AS_MAXG = 16;               /* query heads per KV head */
constexpr uint32_t MAX_SCORE_FLOATS = 1u << 22; /* the library's scores workspace: heads x context */

template <bool ROPE>
__global__ __launch_bounds__(AS_WG) void k_attend_scores(const float *q, float *kcache, float *vcache, AttnShape sh,
                                                         uint32_t pos0, const int32_t *pos_dev, int *flag,
                                                         RopeRows rr, float *scores) {
    __shared__ __attribute__((aligned(16))) float qs[AS_MAXG * AR_HD];
    __shared__ __attribute__((aligned(16))) float kt[AS_SP * AR_KP];
    __shared__ float rtab[ROPE ? AR_HD : 1];
    const uint32_t tid = threadIdx.x, grp = sh.heads / sh.kv_heads, kh = blockIdx.y, kvd = sh.kv_dim;
    const uint32_t pos = pos_dev ? (uint32_t)*pos_dev : pos0;
    if (pos >= sh.context) {
        if (tid == 0 && blockIdx.x == 0 && flag) *flag = 1;
        return;
    }
    const uint32_t start = sh.window && pos >= sh.window ? pos - sh.window + 1 : 0, np = pos - start + 1;
    const uint32_t last = np - 1, p0 = blockIdx.x * AS_SP;
    if (p0 >= np) return; /* uniform: past the current position */
    const uint32_t cnt = np - p0 < AS_SP ? np - p0 : AS_SP;
    const bool holds_last = ROPE && last < p0 + cnt;
    const float *kbase = kcache + (size_t)start * kvd + (size_t)kh * AR_HD;

    /* loads: q of the group's heads, the table rows, this block's K rows (the current one from rr.k) */
    constexpr uint32_t QL = (AS_MAXG * AR_Q4 + AS_WG - 1) / AS_WG, KL = AS_SP * AR_Q4 / AS_WG;
    static_assert(KL * AS_WG == AS_SP * AR_Q4, "whole K rows per load round");
    float4 qx[QL];
#pragma unroll
    for (uint32_t u = 0; u < QL; ++u) {
        const uint32_t f = tid + u * AS_WG, hh = f / AR_Q4, c = f % AR_Q4;
        qx[u] = hh < grp ? *(const float4 *)(q + (size_t)(kh * grp + hh) * AR_HD + 4 * c) : make_float4(0, 0, 0, 0);
    }
    float rv = 0.0f;
    const uint32_t ri = tid, rhalf = ri < sh.pairs ? 0 : 1, rj = ri - rhalf * sh.pairs;
    const bool rload = ROPE && ri < 2 * sh.pairs;
    if (rload) rv = (rhalf ? rr.sn : rr.cs)[(size_t)pos * sh.pairs + rj];
    float4 kx[KL];
#pragma unroll
    for (uint32_t u = 0; u < KL; ++u) {
        const uint32_t f = tid + u * AS_WG, r = f / AR_Q4, c = f % AR_Q4, p = p0 + r;
        const float *src = (ROPE && p == last) ? rr.k + (size_t)kh * AR_HD : kbase + (size_t)(r < cnt ? p : p0) * kvd;
        kx[u] = *(const float4 *)(src + 4 * c);
    }
    if (ROPE && holds_last && tid >= 64 && tid < 64 + AR_HD) /* v is stored as is (model.c:520-523) */
        vcache[(size_t)pos * kvd + (size_t)kh * AR_HD + (tid - 64)] = rr.v[(size_t)kh * AR_HD + (tid - 64)];
    if (rload) rtab[rhalf * (AR_HD / 2) + rj] = rv;
    if (ROPE) __syncthreads(); /* the table rows */
    const float *crow = ROPE ? rtab : nullptr, *srow = ROPE ? rtab + AR_HD / 2 : nullptr;
#pragma unroll
    for (uint32_t u = 0; u < QL; ++u) {
        const uint32_t f = tid + u * AS_WG, hh = f / AR_Q4, c = f % AR_Q4;
        if (hh < grp) *(float4 *)&qs[hh * AR_HD + 4 * c] = ROPE ? rope4(qx[u], c, sh.pairs, crow, srow) : qx[u];
    }
#pragma unroll
    for (uint32_t u = 0; u < KL; ++u) {
        const uint32_t f = tid + u * AS_WG, r = f / AR_Q4, c = f % AR_Q4, p = p0 + r;
        if (r < cnt) {
            float4 x = kx[u];
            if (ROPE && p == last) {
                x = rope4(x, c, sh.pairs, crow, srow);
                *(float4 *)(kcache + (size_t)pos * kvd + (size_t)kh * AR_HD + 4 * c) = x;
            }
            *(float4 *)&kt[r * AR_KP + 4 * c] = x;
        }
    }
    __syncthreads();

    /* (position, head) pairs: dot_f32 of kernels.c:1119-1127, lane tree, times 1/sqrt(hd). Two
     * adjacent threads per pair: thread half h keeps lanes 4h..4h+3 (element 8e + l added over e in
     * order, one 16-byte read of k and of q per e), then the even thread takes the odd one's four
     * lanes and forms the tree */
    const float factor = 1.0f / sqrtf((float)AR_HD);
    for (uint32_t i = tid; i < 2 * cnt * grp; i += AS_WG) { /* pairs of lanes stay together */
        const uint32_t d = i / 2, half = i & 1u, r = d % cnt, hh = d / cnt;
        const float4 *kr = (const float4 *)&kt[r * AR_KP], *q4 = (const float4 *)&qs[hh * AR_HD];
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (uint32_t e = 0; e < AR_HD / 8; ++e) {
            const float4 kv = kr[2 * e + half], qv = q4[2 * e + half];
            float p;
            p = qv.x * kv.x; a0 = a0 + p;
            p = qv.y * kv.y; a1 = a1 + p;
            p = qv.z * kv.z; a2 = a2 + p;
            p = qv.w * kv.w; a3 = a3 + p;
        }
        const float b0 = __shfl_xor(a0, 1, 64), b1 = __shfl_xor(a1, 1, 64), b2 = __shfl_xor(a2, 1, 64),
                    b3 = __shfl_xor(a3, 1, 64);
        if (!half) {
            const float p04 = a0 + b0, p15 = a1 + b1, p26 = a2 + b2, p37 = a3 + b3;
            const float e2 = p04 + p26, o2 = p15 + p37;
            scores[(size_t)(kh * grp + hh) * sh.context + p0 + r] = (e2 + o2) * factor;
        }
    }
}

/* k_attend_values: workgroup (head, 32 coordinates) loads its scores row and
 * its value rows up front, then steps 2-4 of the row attention (att_tail). */
template <bool ROPE>
__global__ __launch_bounds__(AR_WG) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_attend_values(
    const float *vcache, float *att, AttnShape sh, uint32_t pos0, const int32_t *pos_dev, float *xd, int8_t *xq,
    const float *vraw, const float *scores, int *flag) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ uint64_t etab[32];
    __shared__ float red[AR_WG / 64];
    __shared__ float s_inv;
    constexpr uint32_t ngrp = AR_HD / ATT_JW;
    const uint32_t tid = threadIdx.x, g = blockIdx.x % ngrp, h = blockIdx.x / ngrp;
    const uint32_t kh = h / (sh.heads / sh.kv_heads), kvd = sh.kv_dim, j0 = g * ATT_JW;
    const uint32_t pos = pos_dev ? (uint32_t)*pos_dev : pos0;
    if (pos >= sh.context) return; /* flagged by the scores launch */
    const uint32_t start = sh.window && pos >= sh.window ? pos - sh.window + 1 : 0, np = pos - start + 1;
    const uint32_t last = np - 1;
    float *sc = lds;
    float *prod = lds + ((sh.context + 3) & ~3u);
    const float *vbase = vcache + (size_t)start * kvd + (size_t)kh * AR_HD + j0;
    const float *vrope = ROPE ? vraw + (size_t)kh * AR_HD + j0 : nullptr;
    const float *srow = scores + (size_t)h * sh.context;
    const uint32_t vrow = tid / (ATT_JW / 4), vcol = (tid % (ATT_JW / 4)) * 4;

    /* issue order = need order: the table, the scores (a round of AR_WG x AS_LD), the first value rows */
    uint64_t ev = 0;
    if (tid < 32) ev = EXP2_TABLE[tid];
    constexpr uint32_t AS_LD = 4;
    float sv[AS_LD];
#pragma unroll
    for (uint32_t u = 0; u < AS_LD; ++u) {
        const uint32_t p = tid + u * AR_WG;
        sv[u] = p < np ? srow[p] : 0.0f;
    }
    float4 pre[AR_VL];
    att_load_values<ROPE>(pre, vbase, vrope, kvd, 0, np, last, vrow, vcol);
    if (tid < 32) etab[tid] = ev;
    float high = -FLT_MAX;
#pragma unroll
    for (uint32_t u = 0; u < AS_LD; ++u) {
        const uint32_t p = tid + u * AR_WG;
        if (p < np) {
            sc[p] = sv[u];
            high = sv[u] > high ? sv[u] : high;
        }
    }
    for (uint32_t p = tid + AS_LD * AR_WG; p < np; p += AR_WG) { /* long contexts */
        const float v = srow[p];
        sc[p] = v;
        high = v > high ? v : high;
    }
    const uint32_t blk = (h * AR_HD + j0) / QK;
    att_tail<ROPE>(high, sc, prod, np, last, pre, vbase, vrope, kvd, vrow, vcol, etab, red, &s_inv,
                   att + (size_t)h * AR_HD + j0, xd ? xd + blk : nullptr, xq ? xq + (size_t)blk * QK : nullptr, flag);
}

/* Prefill attention (many tokens, head_dim 64): workgroup (token, KV head)
 * serves all query heads of the group, so each K and V row is read once per
 * group instead of once per head and column half, and a workgroup's
 * registers and LDS are small enough for several per CU. Same arithmetic as
 * attend_f32 (kernels.c:1154-1176) and k_attend_rows, bit for bit:
 * 1. scores: eight threads per position, lane l accumulating q[8e+l]*k[8e+l]
 *    over e in order (the 8-lane dot_f32), the fixed lane tree, times 1/8;
 * 2. the maximum (order-free; NaN never wins), exp_det(s - max) in parallel;
 * 3. each head's total in position order by one wave (a register chain),
 *    then w_p = s_p * inv for every position in parallel;
 * 4. thread (head, j) sums w_p * v_p[j] in position order, the V rows
 *    staged in LDS in chunks of 64 by all waves, two chunks ahead;
 * 5. the 64 outputs of a head, and with xd their two Q8 blocks. */
constexpr uint32_t AG_WG = 512, AG_MAXG = 8, AG_MAXP = 1024, AG_VC = 64;

__global__ __launch_bounds__(AG_WG) void k_attend_group(const float *q, const float *kcache, const float *vcache,
                                                        float *att, AttnShape sh, uint32_t pos0,
                                                        const int32_t *pos_dev, int *flag, float *xd, int8_t *xq) {
    __shared__ __attribute__((aligned(16))) float sc[AG_MAXG * AG_MAXP];
    __shared__ __attribute__((aligned(16))) float vs[2][AG_VC * AR_HD]; /* V rows of two chunks */
    __shared__ float qs[AG_MAXG * AR_HD];
    __shared__ float hmax[AG_MAXG][AG_WG / 8];
    __shared__ float hinv[AG_MAXG];
    __shared__ uint64_t etab[32];
    const uint32_t tid = threadIdx.x, grp = sh.heads / sh.kv_heads, kvd = sh.kv_dim;
    /* the last token first: workgroups start in index order, so the longest rows start in the first wave of
     * workgroups and the short ones fill in behind them */
    const uint32_t t = gridDim.x / sh.kv_heads - 1 - blockIdx.x / sh.kv_heads, kh = blockIdx.x % sh.kv_heads;
    const uint32_t pos = (pos_dev ? (uint32_t)*pos_dev : pos0) + t;
    if (pos >= sh.context) { /* the scores row holds at most context positions */
        if (tid == 0 && flag) *flag = 1;
        return;
    }
    const uint32_t start = sh.window && pos >= sh.window ? pos - sh.window + 1 : 0, np = pos - start + 1;
    const float *kbase = kcache + (size_t)start * kvd + (size_t)kh * AR_HD;
    const float *vbase = vcache + (size_t)start * kvd + (size_t)kh * AR_HD;
    const float *qg = q + (size_t)t * sh.q_dim + (size_t)kh * grp * AR_HD;
    for (uint32_t i = tid; i < grp * AR_HD; i += AG_WG) qs[i] = qg[i];
    if (tid < 32) etab[tid] = EXP2_TABLE[tid];
    __syncthreads();

    /* 1. scores */
    const uint32_t l = tid & 7u, gi = tid >> 3;
    float qr[AG_MAXG][8], mx[AG_MAXG];
#pragma unroll
    for (uint32_t hh = 0; hh < AG_MAXG; ++hh) {
        mx[hh] = -FLT_MAX;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) qr[hh][e] = hh < grp ? qs[hh * AR_HD + 8 * e + l] : 0.0f;
    }
    const float factor = 1.0f / sqrtf((float)AR_HD);
    /* the next position's K row is requested before this one's products (a position past the context reads
     * row 0: in bounds, unused) */
    auto kload = [&](float (&k)[8], uint32_t pp) __attribute__((always_inline)) {
        const float *kr = kbase + (size_t)(pp < np ? pp : 0) * kvd + l;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) k[e] = kr[8 * e];
    };
    float kv[8], kn[8];
    kload(kv, gi);
    for (uint32_t p = gi; p < np; p += AG_WG / 8) { /* all eight threads of a group take the same positions */
        kload(kn, p + AG_WG / 8);
#pragma unroll
        for (uint32_t hh = 0; hh < AG_MAXG; ++hh) {
            if (hh < grp) { /* uniform */
                float a = 0.0f;
#pragma unroll
                for (uint32_t e = 0; e < 8; ++e) {
                    const float pr = qr[hh][e] * kv[e];
                    a = a + pr;
                }
                const float sv = reduce8_to_lane7(a) * factor;
                if (l == 7) {
                    sc[hh * AG_MAXP + p] = sv;
                    mx[hh] = sv > mx[hh] ? sv : mx[hh];
                }
            }
        }
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) kv[e] = kn[e];
    }
    /* the first two chunks of V rows requested now (thread: float4 tid%16 of rows tid/16 and tid/16 + 32 of a
     * chunk; a row past the context re-reads the last one: in bounds, unused) */
    const uint32_t nch = (np + AG_VC - 1) / AG_VC;
    float4 vr[2][2];
    auto vfetch = [&](float4 (&r)[2], uint32_t c) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) {
            const uint32_t p = c * AG_VC + tid / 16 + 32 * i;
            r[i] = *(const float4 *)(vbase + (size_t)(p < np ? p : np - 1) * kvd + 4 * (tid % 16));
        }
    };
    auto vstore = [&](const float4 (&r)[2], uint32_t buf) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) *(float4 *)&vs[buf][(tid / 16 + 32 * i) * AR_HD + 4 * (tid % 16)] = r[i];
    };
    vfetch(vr[0], 0);
    if (nch > 1) vfetch(vr[1], 1);
    if (l == 7)
#pragma unroll
        for (uint32_t hh = 0; hh < AG_MAXG; ++hh) hmax[hh][gi] = mx[hh];
    __syncthreads();
    if (tid < grp) {
        float m = -FLT_MAX;
        for (uint32_t k = 0; k < AG_WG / 8; ++k) m = hmax[tid][k] > m ? hmax[tid][k] : m;
        hmax[tid][0] = m;
    }
    __syncthreads();

    /* 2. exp_det(s - max) */
    for (uint32_t hh = 0; hh < grp; ++hh) {
        const float high = hmax[hh][0];
        for (uint32_t p = tid; p < np; p += AG_WG) sc[hh * AG_MAXP + p] = exp_det_tab(sc[hh * AG_MAXP + p] - high, etab);
    }
    __syncthreads();

    /* 3. totals in position order */
    {   /* wave h < grp sums head h's row in a register chain; lane 63 ends with the total */
        const uint32_t w = tid / 64;
        if (w < grp) {
            const float tot = serial_sum_wave(sc + w * AG_MAXP, np);
            if ((tid & 63u) == 63u) hinv[w] = 1.0f / tot;
        }
    }
    __syncthreads();
    /* kernels.c:1165: w = scores[p] * inv, formed for every position before the ordered sums */
    for (uint32_t hq = 0; hq < grp; ++hq) {
        const float inv = hinv[hq];
        for (uint32_t p = tid; p < np; p += AG_WG) sc[hq * AG_MAXP + p] = sc[hq * AG_MAXP + p] * inv;
    }
    vstore(vr[0], 0);
    if (nch > 2) vfetch(vr[0], 2);
    __syncthreads();

    /* 4. values: wave hh (64 threads) is head kh*grp + hh, thread j its column, adding w_p * v_p[j] in position
     * order from the chunk in LDS; every wave stages the chunks (chunk c+1 stored while c is summed, c+3
     * requested), one barrier per chunk */
    const uint32_t hh = tid / AR_HD, j = tid % AR_HD;
    const float *srow = sc + hh * AG_MAXP;
    float acc = 0.0f;
    auto vstep = [&](uint32_t c, float4 (&nxt)[2]) __attribute__((always_inline)) {
        if (hh < grp) { /* whole waves */
            const float *vc = vs[c & 1u] + j, *wc = srow + c * AG_VC;
            const uint32_t cnt = np - c * AG_VC < AG_VC ? np - c * AG_VC : AG_VC;
            if (cnt == AG_VC) {
#pragma unroll 16
                for (uint32_t u = 0; u < AG_VC; ++u) {
                    const float pr = wc[u] * vc[u * AR_HD];
                    acc = acc + pr;
                }
            } else {
                for (uint32_t u = 0; u < cnt; ++u) {
                    const float pr = wc[u] * vc[u * AR_HD];
                    acc = acc + pr;
                }
            }
        }
        if (c + 1 < nch) vstore(nxt, (c + 1) & 1u);
        if (c + 3 < nch) vfetch(nxt, c + 3);
        __syncthreads();
    };
    for (uint32_t c = 0; c < nch; c += 2) { /* register sets alternate: vr[1] holds chunk c+1, vr[0] chunk c+2 */
        vstep(c, vr[1]);
        if (c + 1 < nch) vstep(c + 1, vr[0]);
    }
    if (hh >= grp) return; /* whole waves */

    /* 5. the outputs and their Q8 blocks (lanes 0-31 and 32-63: one block each) */
    const uint32_t head = kh * grp + hh;
    att[(size_t)t * sh.q_dim + (size_t)head * AR_HD + j] = acc;
    if (xd) {
        const float av = fabsf(acc);
        const float mxa = max32(av);
        const uint64_t badm = __ballot(!(av <= FLT_MAX));
        const bool bad = ((j < 32 ? badm : badm >> 32) & 0xffffffffull) != 0;
        const float scale = mxa / 127.0f;
        const float qinv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
        const float pq = acc * qinv;
        int qi = (int)__builtin_rintf(pq);
        qi = qi > 127 ? 127 : (qi < -127 ? -127 : qi);
        const size_t blk = (size_t)t * (sh.q_dim / QK) + (size_t)head * (AR_HD / QK) + j / QK;
        xq[blk * QK + j % QK] = (int8_t)qi;
        if (j % QK == 0) {
            xd[blk] = scale;
            if (bad && flag) *flag = 1;
        }
    }
}

/* Element j of a dequantized embedding row (kernels.c:1044-1062): scale * float(q). */
template <bool Q5>
__device__ __forceinline__ float embed_value(const unsigned char *row, uint32_t j) {
    const uint32_t b = j / QK, kk = j % QK;
    float scale;
    int v;
    if (Q5) {
        const unsigned char *blk = row + (size_t)b * Q5_BYTES;
        scale = half_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const uint32_t high = ld_u32_bytes(blk + 2);
        const uint32_t lo = kk < 16 ? (blk[6 + kk] & 15u) : (uint32_t)(blk[6 + kk - 16] >> 4);
        v = (int)(lo | (((high >> kk) & 1u) << 4)) - 16;
    } else {
        const unsigned char *blk = row + (size_t)b * Q8_BYTES;
        scale = __uint_as_float(ld_u32_bytes(blk));
        v = (int)(int8_t)blk[4 + kk];
    }
    return scale * (float)v;
}

/* Greedy choice (sampler.c:57-63): the first non-banned id, replaced by any
 * later id with a strictly greater logit. Equivalently: the lowest id of the
 * largest non-NaN logit, unless the first candidate itself is NaN (then that
 * candidate: nothing compares greater than NaN). Two stages: AM_WG-thread
 * workgroups each reduce one contiguous span of ids to (largest non-NaN
 * logit, its lowest id, lowest non-banned id); one workgroup merges the
 * partials in any order (the merge is order-free: max with ties to the lower
 * id, min of first) and applies the NaN rule. */
constexpr uint32_t AM_WG = 256, AM_LOADS = 4, AM_SPAN = AM_WG * AM_LOADS, AM_FINAL_WG = 1024;

struct ArgBest {
    float v;
    uint32_t i, first; /* UINT32_MAX: none */
};
static_assert(sizeof(ArgBest) == ARGMAX_PART_BYTES, "argmax partial layout");

__device__ __forceinline__ void am_merge(ArgBest &a, float ov, uint32_t oi, uint32_t of) {
    if (oi != UINT32_MAX && (a.i == UINT32_MAX || ov > a.v || (ov == a.v && oi < a.i))) {
        a.v = ov;
        a.i = oi;
    }
    a.first = of < a.first ? of : a.first;
}

/* Workgroup-wide merge; the result is valid in thread 0. */
template <uint32_t NT>
__device__ __forceinline__ ArgBest am_reduce(ArgBest a, ArgBest *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        am_merge(a, __shfl_xor(a.v, off, 64), __shfl_xor(a.i, off, 64), __shfl_xor(a.first, off, 64));
    const uint32_t tid = threadIdx.x;
    if ((tid & 63) == 0) red[tid >> 6] = a;
    __syncthreads();
    if (tid == 0)
        for (uint32_t w = 1; w < NT / 64; ++w) am_merge(a, red[w].v, red[w].i, red[w].first);
    return a;
}

/* Stage 1: workgroup w covers ids [w*span, (w+1)*span), AM_SPAN at a time,
 * every load of a pass issued before the first compare. */
__global__ __launch_bounds__(AM_WG) void k_argmax_part(const float *logits, uint32_t n, uint32_t span,
                                                       const unsigned char *banned, ArgBest *part) {
    __shared__ ArgBest red[AM_WG / 64];
    const uint32_t tid = threadIdx.x, i0 = blockIdx.x * span, i1 = n - i0 < span ? n : i0 + span;
    ArgBest a = {0.0f, UINT32_MAX, UINT32_MAX};
    for (uint32_t base = i0; base < i1; base += AM_SPAN) {
        float v[AM_LOADS];
        unsigned char bn[AM_LOADS];
#pragma unroll
        for (uint32_t k = 0; k < AM_LOADS; ++k) {
            const uint32_t i = base + tid + k * AM_WG, ii = i < i1 ? i : i1 - 1;
            v[k] = logits[ii];
            bn[k] = banned ? banned[ii] : 0;
        }
#pragma unroll
        for (uint32_t k = 0; k < AM_LOADS; ++k) { /* ids rise with k: the first hit is this thread's lowest */
            const uint32_t i = base + tid + k * AM_WG;
            if (i >= i1 || bn[k]) continue;
            a.first = i < a.first ? i : a.first;
            if (v[k] != v[k]) continue;
            if (a.i == UINT32_MAX || v[k] > a.v) {
                a.v = v[k];
                a.i = i;
            }
        }
    }
    a = am_reduce<AM_WG>(a, red);
    if (tid == 0) part[blockIdx.x] = a;
}

/* Stage 2: merge the partials; optionally the decode bookkeeping of one
 * step (history[*count] = token, ++*count, ++*pos) and the chosen token's
 * embedding row into emb.out (the next step's input, model.c:669-677; a token
 * past the vocabulary, when every id is banned, raises the flag instead). */
struct ArgEmbed {
    const unsigned char *w;
    size_t row_bytes;
    uint32_t vocab, cols, q5;
    float *out; /* NULL: no embedding */
    int *flag;
};

__global__ __launch_bounds__(AM_FINAL_WG) void k_argmax_final(const float *logits, const ArgBest *part, uint32_t np,
                                                              uint32_t *out, int32_t *pos, uint32_t *count,
                                                              uint32_t *history, uint32_t capacity, ArgEmbed emb) {
    __shared__ ArgBest red[AM_FINAL_WG / 64];
    __shared__ uint32_t s_tok;
    const uint32_t tid = threadIdx.x;
    ArgBest a = {0.0f, UINT32_MAX, UINT32_MAX};
    for (uint32_t p = tid; p < np; p += AM_FINAL_WG) am_merge(a, part[p].v, part[p].i, part[p].first);
    a = am_reduce<AM_FINAL_WG>(a, red);
    if (tid == 0) {
        const uint32_t f = a.first;
        const uint32_t tok = (f != UINT32_MAX && logits[f] != logits[f]) ? f : a.i;
        *out = tok;
        s_tok = tok;
        if (count) {
            const uint32_t c = *count;
            if (c < capacity) history[c] = tok;
            *count = c + 1;
            *pos = *pos + 1;
        }
    }
    if (!emb.out) return; /* uniform */
    __syncthreads();
    const uint32_t tok = s_tok;
    if (tok >= emb.vocab) {
        if (tid == 0 && emb.flag) *emb.flag = 1;
        return;
    }
    const unsigned char *row = emb.w + (size_t)tok * emb.row_bytes;
    for (uint32_t j = tid; j < emb.cols; j += AM_FINAL_WG)
        emb.out[j] = emb.q5 ? embed_value<true>(row, j) : embed_value<false>(row, j);
}

/* Bookkeeping after one replayed decode step: history[*count] = *token
 * (bounded by capacity), then ++*count and ++*pos. One lane. */
__global__ __launch_bounds__(64) void k_decode_advance(int32_t *pos, uint32_t *count, const uint32_t *token,
                                                       uint32_t *history, uint32_t capacity) {
    if (threadIdx.x != 0) return;
    const uint32_t c = *count;
    if (c < capacity) history[c] = *token;
    *count = c + 1;
    *pos = *pos + 1;
}

/* Embedding rows (model.c:669-677): x[t] = dequantized row tokens[t]
 * (kernels.c:1044-1062). */
template <bool Q5>
__global__ __launch_bounds__(256) void k_embed(const unsigned char *w, size_t row_bytes, uint32_t vocab,
                                               const uint32_t *tokens, uint32_t cols, float *out, int *flag) {
    const uint32_t t = blockIdx.x, tok = tokens[t];
    if (tok >= vocab) { /* ids are checked on the host; this only keeps the read in bounds */
        if (threadIdx.x == 0 && flag) *flag = 1;
        return;
    }
    const unsigned char *row = w + (size_t)tok * row_bytes;
    for (uint32_t j = threadIdx.x; j < cols; j += 256) out[(size_t)t * cols + j] = embed_value<Q5>(row, j);
}

/* Row dequantization (reference: src/kernels.c:1044-1062): scale * float(q). */
template <bool Q5>
__global__ __launch_bounds__(WG) void k_dequantize_row(const unsigned char *w, uint32_t cols, float *out) {
    const uint32_t j = blockIdx.x * WG + threadIdx.x;
    if (j >= cols) return;
    const uint32_t b = j / QK, k = j % QK;
    float scale;
    int v;
    if (Q5) {
        const unsigned char *blk = w + (size_t)b * Q5_BYTES;
        scale = half_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const uint32_t high = ld_u32_bytes(blk + 2);
        const uint32_t lo = k < 16 ? (blk[6 + k] & 15u) : (uint32_t)(blk[6 + k - 16] >> 4);
        v = (int)(lo | (((high >> k) & 1u) << 4)) - 16;
    } else {
        const unsigned char *blk = w + (size_t)b * Q8_BYTES;
        scale = __uint_as_float(ld_u32_bytes(blk));
        v = (int)(int8_t)blk[4 + k];
    }
    out[j] = scale * (float)v;
}

bool fast_layout(const MatArgs &a, bool q5) {
    if (a.nb == 0 || a.nb > MAX_FAST_NB) return false;
    if (((uintptr_t)a.xq | (uintptr_t)a.xd) & 3u) return false;
    if (q5 && (a.nb & 1u)) return false;
    for (uint32_t i = 0; i < a.nitems; ++i)
        if ((((uintptr_t)a.item[i].w) | a.item[i].row_bytes) & 3u) return false;
    return true;
}

template <bool Q5, bool FAST, int RT>
hipError_t launch_gemv_rt(MatArgs a, hipStream_t s) {
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = tiles;
        tiles += (a.item[i].rows + RT - 1) / RT;
    }
    if (!tiles) return hipSuccess;
    hipLaunchKernelGGL((k_gemv<Q5, FAST, RT>), dim3(tiles), dim3(WG), 0, s, a);
    return hipGetLastError();
}

template <bool Q5, bool FAST>
hipError_t launch_gemv_tile(MatArgs a, int rt, hipStream_t s) {
    switch (rt) {
    case 1: return launch_gemv_rt<Q5, FAST, 1>(a, s);
    case 2: return launch_gemv_rt<Q5, FAST, 2>(a, s);
    case 4: return launch_gemv_rt<Q5, FAST, 4>(a, s);
    case 8: return launch_gemv_rt<Q5, FAST, 8>(a, s);
    default: return launch_gemv_rt<Q5, FAST, 16>(a, s);
    }
}

/* Single launches of many tiles (the LM head: 18992 tiles of 8 rows) run on
 * the pinned persistent kernel; a few thousand tiles fit the device in one
 * wave of workgroups and keep the one-tile-per-workgroup kernel. */
bool gemv_persistent(uint32_t total_rows, int rt) { return (total_rows + rt - 1) / rt > 4096; }

/* Tile rows of the one-tile-per-workgroup decode GEMV forced by smq_set_gemv_rows
 * (0: chosen per width). */
int g_forced_rt = 0;
/* set_att_grouped(false) sends prefill attention to k_attend_rows instead (tuning, tests) */
bool g_att_grouped = true;
/* set_exact_gemm: 0 = the exact prefill GEMM chosen by shape, 1 = always k_gemm_xm, 2 = never, 3 (4) = always
 * k_gemm_xm with each tile's lane sums split over two (four) waves */
int g_exact_mode = 0;

/* Workgroups of kernel k resident on the device (computed once per kernel by the caller's static). */
inline hipError_t resident_wgs(const void *k, int nt, int &resident) {
    if (resident) return hipSuccess;
    int per_cu = 0, dev = 0, cus = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, nt, 0);
    if (e == hipSuccess) e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    resident = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    return hipSuccess;
}

/* Each item's share of `resident` workgroups in proportion to its tiles of rt rows (at least one,
 * at most one per tile), each a contiguous tile range; returns the grid size (0: no tiles). */
template <class GA>
uint32_t pin_split(GA &g, uint32_t rt, uint64_t resident) {
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < g.nitems; ++i) tiles += (g.item[i].rows + rt - 1) / rt;
    if (!tiles) return 0;
    uint32_t wgs = 0;
    for (uint32_t i = 0; i < g.nitems; ++i) {
        const uint32_t t = (g.item[i].rows + rt - 1) / rt;
        uint32_t n = (uint32_t)((resident * t + tiles / 2) / tiles);
        n = n < 1 ? 1 : (n > t ? t : n);
        g.item[i].wg_begin = wgs;
        g.item[i].nwg = n;
        wgs += n;
    }
    return wgs;
}

/* Steps of the slowest workgroup for tiles of rt rows in nch chunks, under the split pin_split
 * would make (an item's workgroups take floor or ceil of its tiles / workgroups each). */
inline uint64_t pin_max_steps(const GroupArgs &g, uint32_t rt, uint32_t nch, uint64_t resident) {
    uint64_t tiles = 0, worst = 0;
    for (uint32_t i = 0; i < g.nitems; ++i) tiles += (g.item[i].rows + rt - 1) / rt;
    if (!tiles) return 0;
    for (uint32_t i = 0; i < g.nitems; ++i) {
        const uint64_t t = (g.item[i].rows + rt - 1) / rt;
        uint64_t n = (resident * t + tiles / 2) / tiles;
        n = n < 1 ? 1 : (n > t ? t : n);
        const uint64_t per = (t + n - 1) / n;
        worst = per > worst ? per : worst;
    }
    return worst * nch;
}

/* The pinned launch: the tile shape for the row width (see k_gemv_pin), then
 * each item's share of the resident workgroups in proportion to its tiles.
 * LDS per workgroup (product buffers, the staged activation) is sized for
 * three resident workgroups per CU (Q8, fast Q5: four for one-chunk rows), two
 * (exact Q5) or one (exact one-chunk Q5, 768 threads). A launch of few items
 * passes the small argument struct. */
template <bool Q5, bool FAST, bool ONE>
hipError_t launch_gemv_pin_shape(GroupArgs &g, hipStream_t s) {
    /* exact Q5: 512 threads, two workgroups per CU (measured 10-16 % faster than
     * four of 256 threads: larger tiles, fewer barriers per byte); one-chunk exact
     * Q5 rows 768 threads, one workgroup per CU: three waves per SIMD within its
     * 168 registers, 32-row tiles (16 x 8960x1536: 30.3-30.5 against 33.0-33.3 us
     * best at 512); fast Q5 keeps 256 (its registers allow three waves per SIMD) */
    constexpr int NT = Q5 && FAST ? 256 : (Q5 && ONE ? 768 : 512), D = 2;
    constexpr uint32_t TB = Q5 ? 2 : 1, CPR = pin_cpr<Q5, FAST>();
    constexpr uint32_t MAXNB = ONE ? CPR * TB : MAX_FAST_NB;
    /* floats of one product buffer; LDS is allocated in 512-byte units */
    constexpr uint32_t PF = Q5 ? (FAST ? (ONE ? 4480 : 4400) : (ONE ? 12336 : 7776)) : (ONE ? 4832 : 4400);
    const auto kf = k_gemv_pin<Q5, FAST, ONE, NT, D, MAXNB, PF, GroupArgsFew>;
    const auto km = k_gemv_pin<Q5, FAST, ONE, NT, D, MAXNB, PF, GroupArgs>;
    const bool few = g.nitems <= FEW_GROUP_ITEMS;
    static int res_few = 0, res_many = 0;
    const hipError_t e = few ? resident_wgs((const void *)kf, NT, res_few) : resident_wgs((const void *)km, NT, res_many);
    if (e != hipSuccess) return e;
    const uint64_t resident = (uint64_t)(few ? res_few : res_many);
    /* a chunk's tiles fit the product buffer (every chain read, groups of four blocks of a chunk, rt rows
     * each, lies below PF, clear of the sinks that idle tasks write past PF; in fast mode the scale
     * products, groups of rt * 4 + 4, below the scale buffer's sink at PF / 8 + 128) */
    auto fits = [&](uint32_t cpr, uint32_t rt) {
        const uint64_t groups = (cpr * TB + 3) / 4;
        return rt != 0 && groups * (rt * 32 + 4) <= PF && (!FAST || groups * (rt * 4 + 4) <= PF / 8 + 128);
    };
    const uint32_t ppr = (g.nb + TB - 1) / TB;
    g.nch = (ppr + CPR - 1) / CPR;
    if constexpr (Q5 && !ONE) {
        /* several chunks per row: the chunk count whose slowest workgroup takes the fewest steps, at a
         * tie the shorter chunks (shorter chains per step). 16 x 1536x8960 (140 pairs a row): 3 chunks of
         * 47 (10-row tiles, 5 tiles for the slowest workgroup) 44.8-46.7 us; 7 of 20 (24-row tiles, two
         * each) 37.8-39.0 us; 5 of 28 41.1, 6 of 24 42.9, 10 of 14 47.6 us, same box */
        uint32_t best_nch = g.nch;
        uint64_t best = ~0ull;
        for (uint32_t n = g.nch; n <= g.nch + 8 && n <= ppr; ++n) {
            const uint32_t c = (ppr + n - 1) / n, r = pin_rows(NT, TB, c, PF);
            if (!fits(c, r)) continue;
            const uint64_t st = pin_max_steps(g, r, n, resident);
            if (st <= best) {
                best = st;
                best_nch = n;
            }
        }
        g.nch = best_nch;
    }
    g.cpr = (ppr + g.nch - 1) / g.nch;
    g.rt = pin_rows(NT, TB, g.cpr, PF);
    if (g.nb > MAXNB || (ONE && g.nch != 1) || !fits(g.cpr, g.rt)) return hipErrorInvalidValue; /* launcher precondition */
    if (few) {
        GroupArgsFew f = group_args_few(g);
        const uint32_t wgs = pin_split(f, g.rt, resident);
        if (!wgs) return hipSuccess;
        hipLaunchKernelGGL(kf, dim3(wgs), dim3(NT), 0, s, f);
        return hipGetLastError();
    }
    const uint32_t wgs = pin_split(g, g.rt, resident);
    if (!wgs) return hipSuccess;
    hipLaunchKernelGGL(km, dim3(wgs), dim3(NT), 0, s, g);
    return hipGetLastError();
}

template <bool Q5, bool FAST>
hipError_t launch_gemv_pin(GroupArgs &g, hipStream_t s) {
    if (!Q5 && gemv_ct_ok(g, false)) return launch_gemv_ct(g, FAST, s); /* packed 28-block rows */
    const uint32_t ppr = Q5 ? (g.nb + 1) / 2 : g.nb;
    if (ppr <= pin_cpr<Q5, FAST>()) return launch_gemv_pin_shape<Q5, FAST, true>(g, s);
    return launch_gemv_pin_shape<Q5, FAST, false>(g, s);
}


template <bool Q5, bool FAST>
hipError_t launch_typed(MatArgs a, hipStream_t s) {
    uint32_t total_rows = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) total_rows += a.item[i].rows;
    if (!total_rows || !a.ntok || !a.nb) return hipSuccess;
    if (fast_layout(a, Q5)) {
        if (a.ntok == 1) {
            const int rt = gemv_rows_per_tile(a.nb, Q5, total_rows);
            bool pin_ok = true;
            for (uint32_t i = 0; i < a.nitems; ++i) pin_ok = pin_ok && a.item[i].row_bytes <= PIN_MAX_ROW_BYTES;
            if (!g_forced_rt && pin_ok && gemv_persistent(total_rows, rt)) {
                /* many tiles: the pinned persistent kernel streams them (same products and order) */
                GroupArgs g;
                memset(&g, 0, sizeof(g));
                g.nb = a.nb;
                g.flag = a.flag;
                for (uint32_t i = 0; i < a.nitems; ++i) {
                    GroupItem &it = g.item[g.nitems++];
                    it.w = a.item[i].w;
                    it.row_bytes = a.item[i].row_bytes;
                    it.bias = a.item[i].bias;
                    it.y = a.item[i].y;
                    it.xd = a.xd;
                    it.xq = a.xq;
                    it.rows = a.item[i].rows;
                    it.accumulate = a.item[i].accumulate;
                }
                return launch_gemv_pin<Q5, FAST>(g, s);
            }
            return launch_gemv_tile<Q5, FAST>(a, rt, s);
        }
        uint32_t tiles = 0, tiles32 = 0;
        for (uint32_t i = 0; i < a.nitems; ++i) {
            a.item[i].tile_begin = tiles;
            tiles += (a.item[i].rows + GT_R - 1) / GT_R;
            tiles32 += (a.item[i].rows + 31) / 32;
        }
        static int cus = 0;
        if (!cus) {
            int dev = 0, v = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
                v = 256;
            cus = v;
        }
        /* The lane sums on MFMA, by the count W of 32 x 32 tiles (rows x tokens) per CU: from 7/4, 32 x 32
         * workgroups, except from 2 to 3; from 7/8 (Q8 5/8; and from 2 to 3), 16-row tiles with each tile's lane sums
         * over two waves; from 1/4, 16 x 16 tiles over four waves (16-block K chunks); below, the v_dot4
         * kernel. Measured on MI355X (32 x 32 / two / four waves / v_dot4, us): 9728x896 at 128 tokens (W 4.75)
         * 26.4-27.0 / 27.7-28.5; at 96 (3.56) 21.0-21.3 / 23.3-23.5; at 64 (2.38) 17.4-17.6 / 16.6-17.1;
         * 1152x896 at 512 (2.25) 17.4-17.7 / 16.6-17.1; Q5 8960x1536 at 64 (2.19) 26.4-26.8 / 24.3-25.1;
         * 896x896 at 512 (1.75) 14.0 / 14.8; 896x4864 at 512 (1.75) 50.7-51.1 / 52.3-52.4; at 256 (0.88) 44.9 /
         * 35.8-36.1 / 45.1 / 53.0; at 128 (0.44) 44.6 / 32.3-32.5 / 30.4-30.8 / 34.6; Q5 1536x8960 at 64
         * (0.38) 83.1 / 60.5 / 52.2 / 62.5 */
        const uint64_t w32 = (uint64_t)tiles32 * ((a.ntok + 31) / 32), cu = (uint64_t)cus;
        const bool two_ahead = w32 >= 2 * cu && w32 < 3 * cu;
        if (g_exact_mode == 1 || (g_exact_mode == 0 && 4 * w32 >= 7 * cu && !two_ahead))
            return launch_gemm_xm(a, Q5, FAST, 1, s);
        /* Q8 takes the two-wave split from 5/8 (896x4864 at 192 tokens, W 0.66: 35.4-35.8 / 36.8-37.2 on four
         * waves), Q5 from 7/8 (1536x8960 at 128 tokens, W 0.75: 66.0-66.5 / 64.1-65.3) */
        if (g_exact_mode == 3 || (g_exact_mode == 0 && 8 * w32 >= (Q5 ? 7 : 5) * cu))
            return launch_gemm_xm(a, Q5, FAST, 2, s);
        if (g_exact_mode == 4 || (g_exact_mode == 0 && 4 * w32 >= cu)) return launch_gemm_xm(a, Q5, FAST, 4, s);
        /* 8-token tiles where 16-token ones would give fewer than two workgroups per CU (c1 down at 128
         * tokens: 224 workgroups) */
        if ((uint64_t)tiles * ((a.ntok + 15) / 16) < 2ull * (uint64_t)cus) {
            const uint32_t tok_tiles = (a.ntok + 7) / 8;
            hipLaunchKernelGGL((k_gemm_exact<Q5, FAST, 8>), dim3(tiles * tok_tiles), dim3(WG), 0, s, a, tok_tiles);
        } else {
            const uint32_t tok_tiles = (a.ntok + 15) / 16;
            hipLaunchKernelGGL((k_gemm_exact<Q5, FAST, 16>), dim3(tiles * tok_tiles), dim3(WG), 0, s, a, tok_tiles);
        }
        return hipGetLastError();
    }
    uint32_t begin = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = begin;
        begin += a.item[i].rows;
    }
    const uint64_t threads = (uint64_t)total_rows * a.ntok;
    hipLaunchKernelGGL((k_generic<Q5, FAST>), dim3((uint32_t)((threads + WG - 1) / WG)), dim3(WG), 0, s, a,
                       total_rows);
    return hipGetLastError();
}

/* Workgroups (tiles x token tiles) below which K is split over slices: 48 workgroups of 20 chunks
 * (1536 x 8960 Q5 at 64 tokens) leave most CUs idle; at 192 and more the split's second launch and
 * partial traffic do not pay (as for the Q8 split-K kernel). */
constexpr uint32_t MFMA_MIN_SPLIT_TILES = 192;

template <bool Q5, bool SUMS>
hipError_t launch_mfma_typed(MatArgs a, int32_t *sums, float *ws, size_t ws_bytes, hipStream_t s) {
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = tiles;
        tiles += (a.item[i].rows + MT_R - 1) / MT_R;
    }
    const uint32_t tok_tiles = (a.ntok + MT_T - 1) / MT_T;
    if (!tiles || !tok_tiles || !a.nb) return hipSuccess;
    const uint32_t grid1 = tiles * tok_tiles, nchunks = (a.nb + MT_CB - 1) / MT_CB;
    MfmaSplit sp = {1u, nchunks, tiles * MT_R, nullptr};
    if (!SUMS && ws && grid1 < MFMA_MIN_SPLIT_TILES && nchunks >= 4) {
        /* about 512 workgroups, at least two chunks each, the partials within the workspace */
        uint32_t slices = (512 + grid1 - 1) / grid1;
        slices = slices < nchunks / 2 ? slices : nchunks / 2;
        const size_t per = (size_t)a.ntok * sp.total_rows * sizeof(float);
        const size_t fit = per ? ws_bytes / per : 0;
        slices = (size_t)slices < fit ? slices : (uint32_t)fit;
        if (slices >= 2) {
            sp.cps = (nchunks + slices - 1) / slices;
            sp.slices = (nchunks + sp.cps - 1) / sp.cps; /* every slice holds at least one chunk */
            sp.part = ws;
        }
    }
    hipLaunchKernelGGL((k_gemm_mfma<Q5, SUMS>), dim3(grid1 * sp.slices), dim3(WG), 0, s, a, tok_tiles, sums, sp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || sp.slices == 1) return e;
    const uint64_t n = (uint64_t)a.ntok * sp.total_rows;
    hipLaunchKernelGGL(k_mfma_reduce, dim3((uint32_t)((n + WG - 1) / WG)), dim3(WG), 0, s, a, sp);
    return hipGetLastError();
}

}  // namespace

/* Rows per workgroup: the largest power of two (<= 8) whose chunk of 256
 * tasks covers all nb blocks, so each workgroup needs one round of loads
 * (Q5 keeps at least 2 rows: its wide rows run faster as two chunks of two
 * rows than as one chunk of one). Measured on MI355X over rotated weights:
 * 9728x896 Q8 4.7 us at 8 rows, 896x4864 Q8 4.6 us at 1 row, 1536x8960 Q5
 * 7.4 us at 2 rows (9.9 us at 1). set_gemv_rows overrides. */
int gemv_rows_per_tile(uint32_t nb, bool q5, uint32_t total_rows) {
    (void)total_rows;
    if (g_forced_rt) return g_forced_rt;
    const uint32_t cover = (q5 ? 512u : 256u) / nb;
    /* Q8 rows of 129-256 blocks: 4 rows of chunks of 64 blocks, not 1 row in one chunk (the Qwen2.5-0.5B
     * down projection, nb 152, in the decode step: fewer, fuller workgroups whose lane chains share no SIMD
     * with other workgroups' products; 1,161 -> 1,170 tok/s, measured) */
    if (!q5 && cover == 1) return 4;
    int rt = q5 ? 2 : 1;
    while (rt < 8 && (uint32_t)(rt * 2) <= cover) rt *= 2;
    return rt;
}

bool set_gemv_rows(int rt) {
    if (rt != 0 && rt != 1 && rt != 2 && rt != 4 && rt != 8 && rt != 16) return false;
    g_forced_rt = rt;
    return true;
}

bool set_exact_gemm(int mode) {
    if (mode < 0 || mode > 4) return false;
    g_exact_mode = mode;
    return true;
}

void set_att_grouped(bool on) { g_att_grouped = on; }

bool mfma_layout_ok(const MatArgs &a, bool q5) {
    if (a.nb == 0) return false;
    if (((uintptr_t)a.xq | (uintptr_t)a.xd) & 3u) return false;
    if (q5 && (a.nb & 1u)) return false;
    for (uint32_t i = 0; i < a.nitems; ++i)
        if ((((uintptr_t)a.item[i].w) | a.item[i].row_bytes) & 3u) return false;
    return true;
}

hipError_t launch_matmul_mfma(const MatArgs &a, bool q5, int32_t *sums, float *ws, size_t ws_bytes, hipStream_t s) {
    if (sums)
        return q5 ? launch_mfma_typed<true, true>(a, sums, nullptr, 0, s)
                  : launch_mfma_typed<false, true>(a, sums, nullptr, 0, s);
    return q5 ? launch_mfma_typed<true, false>(a, nullptr, ws, ws_bytes, s)
              : launch_mfma_typed<false, false>(a, nullptr, ws, ws_bytes, s);
}

hipError_t launch_glu(float *h, const float *gate, uint32_t n, int act, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_glu, dim3((n + WG - 1) / WG), dim3(WG), 0, s, h, gate, n, act);
    return hipGetLastError();
}

hipError_t launch_matmul(const MatArgs &a, bool q5, bool fast, hipStream_t s) {
    if (q5) return fast ? launch_typed<true, true>(a, s) : launch_typed<true, false>(a, s);
    return fast ? launch_typed<false, true>(a, s) : launch_typed<false, false>(a, s);
}

hipError_t launch_quantize_q8(const float *x, uint32_t rows, uint32_t n, float *d, int8_t *q, int *flag,
                              hipStream_t s) {
    const uint32_t nb = (n + QK - 1) / QK;
    const uint64_t threads = (uint64_t)rows * nb * QK;
    if (!threads) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8, dim3((uint32_t)((threads + WG - 1) / WG)), dim3(WG), 0, s, x, rows, n, nb, d,
                       q, flag);
    return hipGetLastError();
}

hipError_t launch_row_quantize(const float *src, const float *norm, float eps, const float *gate, int act,
                               uint32_t rows, uint32_t n, float *y, float *d, int8_t *q, int *flag, hipStream_t s) {
    if (!rows || !n) return hipSuccess;
    if (n > (uint32_t)(RW_WG * RW_EPT)) return hipErrorInvalidValue;
    const size_t lds = norm ? (size_t)((n + 3) & ~3u) * sizeof(float) : 0; /* the squares' whole float4s */
    const dim3 grid(rows);
    const int nt = n <= (uint32_t)(RW_NARROW * RW_EPT) ? RW_NARROW : RW_WG;
#define SMQ_RQ(NORM, ACT)                                                                                      \
    do {                                                                                                       \
        if (nt == RW_NARROW)                                                                                   \
            hipLaunchKernelGGL((k_row_quantize<NORM, ACT, RW_NARROW>), grid, dim3(RW_NARROW), lds, s, src, norm, \
                               eps, gate, n, y, d, q, flag);                                                   \
        else                                                                                                   \
            hipLaunchKernelGGL((k_row_quantize<NORM, ACT, RW_WG>), grid, dim3(RW_WG), lds, s, src, norm, eps,    \
                               gate, n, y, d, q, flag);                                                        \
    } while (0)
    if (norm) {
        if (act == 1) SMQ_RQ(true, 1);
        else if (act == 2) SMQ_RQ(true, 2);
        else SMQ_RQ(true, 0);
    } else {
        if (act == 1) SMQ_RQ(false, 1);
        else if (act == 2) SMQ_RQ(false, 2);
        else SMQ_RQ(false, 0);
    }
#undef SMQ_RQ
    return hipGetLastError();
}

bool group_layout_ok(const GroupArgs &g, bool q5) {
    if (!g.nb || g.nb > MAX_FAST_NB || (q5 && (g.nb & 1u))) return false;
    for (uint32_t i = 0; i < g.nitems; ++i)
        if ((((uintptr_t)g.item[i].w) | g.item[i].row_bytes | (uintptr_t)g.item[i].xq) & 3u ||
            g.item[i].row_bytes > PIN_MAX_ROW_BYTES)
            return false;
    return true;
}

hipError_t launch_gemv_grouped(GroupArgs &g, bool q5, bool fast, hipStream_t s) {
    if (!g.nitems) return hipSuccess;
    if (!group_layout_ok(g, q5)) return hipErrorInvalidValue;
    if (q5) return fast ? launch_gemv_pin<true, true>(g, s) : launch_gemv_pin<true, false>(g, s);
    return fast ? launch_gemv_pin<false, true>(g, s) : launch_gemv_pin<false, false>(g, s);
}

hipError_t launch_rope_kv(float *q, float *k, const float *v, uint32_t ntok, const AttnShape &sh, const float *cs,
                          const float *sn, float *kcache, float *vcache, uint32_t pos0, const int32_t *pos_dev,
                          int *flag, hipStream_t s) {
    if (!ntok) return hipSuccess;
    hipLaunchKernelGGL(k_rope_kv, dim3(ntok), dim3(256), 0, s, q, k, v, sh, cs, sn, kcache, vcache, pos0, pos_dev,
                       flag);
    return hipGetLastError();
}


bool attention_rows_ok(const AttnShape &sh, const void *q, const void *kcache, const void *vcache) {
    return sh.head_dim == AR_HD && ((uintptr_t)q & 15) == 0 && ((uintptr_t)kcache & 15) == 0 &&
           ((uintptr_t)vcache & 15) == 0;
}

hipError_t launch_attention(const float *q, const float *kcache, const float *vcache, float *att, uint32_t ntok,
                            const AttnShape &sh, uint32_t pos0, const int32_t *pos_dev, int *flag, float *xd,
                            int8_t *xq, hipStream_t s, float *scores) {
    if (!ntok) return hipSuccess;
    if (sh.context > MAX_ATT_POSITIONS || sh.head_dim > MAX_HEAD_DIM || sh.head_dim < 1 ||
        (xd && sh.head_dim % QK))
        return hipErrorInvalidValue;
    const uint32_t groups = (sh.head_dim + ATT_JW - 1) / ATT_JW;
    if (ntok == 1 && scores && attention_rows_ok(sh, q, kcache, vcache) &&
        (size_t)sh.heads * sh.context <= MAX_SCORE_FLOATS && sh.heads / sh.kv_heads <= AS_MAXG) {
        /* one decoding token whose q is rotated and whose k and v rows are in the caches already:
         * the scores spread over workgroups of positions, then the values */
        const size_t lds = (((size_t)sh.context + 3) / 4 * 4 + (size_t)AR_FIXED) * sizeof(float);
        const RopeRows none = {nullptr, nullptr, nullptr, nullptr};
        const dim3 sgrid((sh.context + AS_SP - 1) / AS_SP, sh.kv_heads);
        hipLaunchKernelGGL(k_attend_scores<false>, sgrid, dim3(AS_WG), 0, s, q, (float *)kcache, (float *)vcache, sh,
                           pos0, pos_dev, flag, none, scores);
        hipLaunchKernelGGL(k_attend_values<false>, dim3(sh.heads * groups), dim3(AR_WG), lds, s, vcache, att, sh, pos0,
                           pos_dev, xd, xq, nullptr, scores, flag);
        return hipGetLastError();
    }
    if (ntok > 1 && attention_rows_ok(sh, q, kcache, vcache) && sh.context <= AG_MAXP &&
        sh.heads % sh.kv_heads == 0 && sh.heads / sh.kv_heads <= AG_MAXG && g_att_grouped) {
        hipLaunchKernelGGL(k_attend_group, dim3(ntok * sh.kv_heads), dim3(AG_WG), 0, s, q, kcache, vcache, att, sh, pos0,
                           pos_dev, flag, xd, xq);
        return hipGetLastError();
    }
    if (attention_rows_ok(sh, q, kcache, vcache)) {
        const size_t lds = (((size_t)sh.context + 3) / 4 * 4 + (size_t)AR_FIXED) * sizeof(float);
        RopeRows none = {nullptr, nullptr, nullptr, nullptr};
        hipLaunchKernelGGL(k_attend_rows<false>, dim3(ntok * sh.heads * groups), dim3(AR_WG), lds, s, q,
                           (float *)kcache, (float *)vcache, att, sh, pos0, pos_dev, flag, xd, xq, none);
        return hipGetLastError();
    }
    const size_t lds = (((size_t)sh.context + 3) / 4 * 4 + (size_t)ATT_SHARED) * sizeof(float);
    hipLaunchKernelGGL(k_attend, dim3(ntok * sh.heads * groups), dim3(ATT_WG), lds, s, q, kcache, vcache, att, sh, pos0,
                       pos_dev, flag, xd, xq);
    return hipGetLastError();
}

/* Dynamic LDS beyond the 64 KiB default (a score per position, up to
 * MAX_ATT_POSITIONS): raised once at smq_init, before any capture, so no
 * kernel's attributes change while a captured graph holds it. */
hipError_t prepare_attention_attributes() {
    const int rows = (int)(((size_t)MAX_ATT_POSITIONS + AR_FIXED) * sizeof(float));
    const int tiled = (int)(((size_t)MAX_ATT_POSITIONS + ATT_SHARED) * sizeof(float));
    const hipError_t es[] = {
        hipFuncSetAttribute((const void *)k_attend_rows<false>, hipFuncAttributeMaxDynamicSharedMemorySize, rows),
        hipFuncSetAttribute((const void *)k_attend_rows<true>, hipFuncAttributeMaxDynamicSharedMemorySize, rows),
        hipFuncSetAttribute((const void *)k_attend_values<true>, hipFuncAttributeMaxDynamicSharedMemorySize, rows),
        hipFuncSetAttribute((const void *)k_attend_values<false>, hipFuncAttributeMaxDynamicSharedMemorySize, rows),
        hipFuncSetAttribute((const void *)k_attend, hipFuncAttributeMaxDynamicSharedMemorySize, tiled)};
    for (hipError_t e : es)
        if (e != hipSuccess) return e;
    return hipSuccess;
}

hipError_t launch_attention_rope(const float *q, const float *k, const float *v, const float *cs, const float *sn,
                                 float *kcache, float *vcache, float *att, const AttnShape &sh, uint32_t pos0,
                                 const int32_t *pos_dev, int *flag, float *xd, int8_t *xq, float *scores,
                                 hipStream_t s) {
    if (sh.context > MAX_ATT_POSITIONS || !attention_rows_ok(sh, q, kcache, vcache) ||
        ((uintptr_t)k & 15) || ((uintptr_t)v & 15))
        return hipErrorInvalidValue;
    const uint32_t groups = (sh.head_dim + ATT_JW - 1) / ATT_JW;
    const size_t lds = (((size_t)sh.context + 3) / 4 * 4 + (size_t)AR_FIXED) * sizeof(float);
    RopeRows rr = {k, v, cs, sn};
    if (scores && (size_t)sh.heads * sh.context <= MAX_SCORE_FLOATS && sh.heads / sh.kv_heads <= AS_MAXG) {
        const dim3 sgrid((sh.context + AS_SP - 1) / AS_SP, sh.kv_heads);
        hipLaunchKernelGGL(k_attend_scores<true>, sgrid, dim3(AS_WG), 0, s, q, kcache, vcache, sh, pos0, pos_dev, flag,
                           rr, scores);
        hipLaunchKernelGGL(k_attend_values<true>, dim3(sh.heads * groups), dim3(AR_WG), lds, s, vcache, att, sh, pos0,
                           pos_dev, xd, xq, v, scores, flag);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_attend_rows<true>, dim3(sh.heads * groups), dim3(AR_WG), lds, s, q, kcache, vcache, att, sh,
                       pos0, pos_dev, flag, xd, xq, rr);
    return hipGetLastError();
}

/* The allocation-free argmax's partials (smq_argmax_noalloc): a file-scope
 * device array of MAX_ARGMAX_PARTS partials (12 KiB), which every GPU the
 * library runs on holds until the process ends. Host code never passes the
 * symbol itself (on the host it is a stand-in, not a device address): at
 * smq_init, with the device current, bind_noalloc_scratch takes its device
 * address once per device, and launches use that address. */
static __device__ __align__(256) ArgBest scratch[MAX_ARGMAX_PARTS];
static_assert(NOALLOC_MAX_VOCAB == MAX_ARGMAX_PARTS * AM_SPAN, "one AM_SPAN of ids per partial");
constexpr int MAX_BOUND_DEVICES = 64;
void *g_scratch_dev[MAX_BOUND_DEVICES] = {};

hipError_t bind_noalloc_scratch(int device) {
    if (device < 0 || device >= MAX_BOUND_DEVICES) return hipErrorInvalidDevice;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_dev[device] = p;
    return hipSuccess;
}

void *noalloc_scratch(int device) {
    return device >= 0 && device < MAX_BOUND_DEVICES ? g_scratch_dev[device] : nullptr;
}

hipError_t launch_argmax(const float *logits, uint32_t n, const unsigned char *banned, uint32_t *out, void *parts,
                         int32_t *pos, uint32_t *count, uint32_t *history, uint32_t capacity, hipStream_t s,
                         const EmbedArgs *embed) {
    /* span: a multiple of AM_SPAN, large enough for at most MAX_ARGMAX_PARTS workgroups */
    const uint32_t span = ((n + MAX_ARGMAX_PARTS - 1) / MAX_ARGMAX_PARTS + AM_SPAN - 1) / AM_SPAN * AM_SPAN;
    const uint32_t np = (n + span - 1) / span;
    ArgEmbed emb = {nullptr, 0, 0, 0, 0, nullptr, nullptr};
    if (embed) emb = {embed->w, embed->row_bytes, embed->vocab, embed->cols, embed->q5 ? 1u : 0u, embed->out, embed->flag};
    hipLaunchKernelGGL(k_argmax_part, dim3(np), dim3(AM_WG), 0, s, logits, n, span, banned, (ArgBest *)parts);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(AM_FINAL_WG), 0, s, logits, (const ArgBest *)parts, np, out, pos,
                       count, history, capacity, emb);
    return hipGetLastError();
}

hipError_t launch_embed(const unsigned char *w, size_t row_bytes, bool q5, uint32_t vocab, const uint32_t *tokens,
                        uint32_t ntok, uint32_t cols, float *out, int *flag, hipStream_t s) {
    if (!ntok) return hipSuccess;
    if (q5) hipLaunchKernelGGL(k_embed<true>, dim3(ntok), dim3(256), 0, s, w, row_bytes, vocab, tokens, cols, out, flag);
    else hipLaunchKernelGGL(k_embed<false>, dim3(ntok), dim3(256), 0, s, w, row_bytes, vocab, tokens, cols, out, flag);
    return hipGetLastError();
}

hipError_t launch_decode_advance(int32_t *pos, uint32_t *count, const uint32_t *token, uint32_t *history,
                                 uint32_t capacity, hipStream_t s) {
    hipLaunchKernelGGL(k_decode_advance, dim3(1), dim3(64), 0, s, pos, count, token, history, capacity);
    return hipGetLastError();
}

hipError_t launch_dequantize_row(const unsigned char *w, uint32_t cols, float *out, bool q5, hipStream_t s) {
    if (!cols) return hipSuccess;
    const dim3 grid((cols + WG - 1) / WG);
    if (q5) hipLaunchKernelGGL(k_dequantize_row<true>, grid, dim3(WG), 0, s, w, cols, out);
    else hipLaunchKernelGGL(k_dequantize_row<false>, grid, dim3(WG), 0, s, w, cols, out);
    return hipGetLastError();
}

}  // namespace smq
