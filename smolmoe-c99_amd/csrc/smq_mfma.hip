/* Prefill GEMM of Q8 rows on int8 MFMA (relaxed block order), for batches
 * of tokens: out[t][r] = sum over blocks b of wscale[r][b] * xscale[t][b] *
 * S[r][t][b] (+ bias, + prior), where S is the exact int32 block sum (the
 * reference's eight lane sums of one block added together, kernels.c:36-79).
 * One v_mfma_i32_16x16x32_i8 gives S for a 16-row x 16-token tile of one
 * block; the scales are applied per block, acc = fma(ws * xs, float(S), acc),
 * blocks in order: the per-block integer sums are exact, the f32 result
 * differs from the eight-lane contract only in rounding.
 *
 * Layout. Workgroup tile: 64 rows x 64 tokens, four waves of 32 x 32 (2 x 2
 * MFMA tiles each). K advances in chunks of 7 blocks (252 bytes of a row, 63
 * dwords): wave w stages rows w, w+4, ... and tokens w, w+4, ..., one row (or
 * token) per load instruction, lane k loading dword k (field k % 9 of block
 * k / 9; a token's 56 int8 dwords and its 7 scales), so every load is one
 * coalesced run. Each lane knows once where its dword goes in LDS: MFMA
 * operand order A[block][k8][row] (8 bytes per lane read, planes padded to
 * 130 dwords so the staging writes spread over the banks) or the scale
 * planes [block][row] (pitch 68: 16-byte reads of four rows). Two LDS buffers
 * alternate: the next chunk's loads are in flight while this one is
 * computed, one barrier per chunk. Long K with few tiles (e.g. 896 rows x 152
 * blocks) is split over S slices of the chunks: each slice writes its partial
 * sums, and a second launch adds the slices in order and applies bias,
 * finiteness and the residual add.
 */
#include <float.h>
#include <stddef.h>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t MQ_NT = 256;                 /* four waves */
constexpr uint32_t MQ_R = 64, MQ_T = 64;        /* rows and tokens per workgroup tile */
constexpr uint32_t MQ_KC = 7;                   /* blocks per K chunk: 63 dwords of a row */
constexpr uint32_t MQ_PL = 2 * MQ_R + 2;        /* dwords per (block, k8) operand plane (64 x 8 bytes + pad) */
constexpr uint32_t MQ_SP = MQ_R + 4;            /* scale plane pitch */
constexpr uint32_t MQ_A = 0;                    /* dword offsets inside one buffer */
constexpr uint32_t MQ_B = MQ_A + MQ_KC * 4 * MQ_PL;
constexpr uint32_t MQ_WS = MQ_B + MQ_KC * 4 * MQ_PL;
constexpr uint32_t MQ_XS = MQ_WS + MQ_KC * MQ_SP;
constexpr uint32_t MQ_SINK = MQ_XS + MQ_KC * MQ_SP; /* lane 63's writes (it holds no dword of a row) */
constexpr uint32_t MQ_BUF = MQ_SINK + 4;          /* 8236 dwords = 32.9 KB */
constexpr uint32_t MQ_LD = MQ_R / 4;            /* rows (and tokens) each wave stages per chunk */
static_assert(MQ_T == MQ_R && MQ_BUF % 4 == 0 && MQ_WS % 4 == 0 && MQ_XS % 4 == 0, "16-byte aligned planes");
static_assert(MQ_PL % 32 == 2 && MQ_SP % 32 == 4, "bank spread of the staging writes");

typedef int v4i __attribute__((ext_vector_type(4)));

/* The item whose tiles hold `tile` (items are laid out tile after tile). */
__device__ __forceinline__ uint32_t mq_item(const MatArgs &a, uint32_t tile) {
    uint32_t it = 0;
    if (a.nitems > 1 && tile >= a.item[1].tile_begin) it = 1;
    if (a.nitems > 2 && tile >= a.item[2].tile_begin) it = 2;
    if (a.nitems > 3 && tile >= a.item[3].tile_begin) it = 3;
    return it;
}

struct MqArgs {
    MatArgs m;
    uint32_t tok_tiles, row_tiles, slices, cps; /* chunks per slice */
    float *part;                                /* slices > 1: [slice][ntok][total rows] partial sums */
    uint32_t total_rows;
};

constexpr size_t MQ_LDS_BYTES = 2 * MQ_BUF * sizeof(uint32_t); /* two buffers: 65,856 bytes (dynamic) */

__global__ __launch_bounds__(MQ_NT, 2) void k_gemm_mq8(MqArgs q) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const MatArgs &a = q.m;
    const uint32_t tid = threadIdx.x, l = tid % 64, w = tid / 64, nb = a.nb;

    /* workgroup -> (slice, row tile, token tile), consecutive tiles of an XCD's share together */
    const uint32_t G = gridDim.x, xcd = blockIdx.x % 8u, kk = blockIdx.x / 8u;
    const uint32_t per = G / 8u, extra = G % 8u;
    const uint32_t L = xcd * per + (xcd < extra ? xcd : extra) + kk;
    const uint32_t tiles = q.row_tiles * q.tok_tiles;
    const uint32_t slice = L / tiles, rem = L % tiles, row_tile = rem / q.tok_tiles, tok_tile = rem % q.tok_tiles;
    const uint32_t it = mq_item(a, row_tile);
    const Item &I = a.item[it];
    const uint32_t r0 = (row_tile - I.tile_begin) * MQ_R, t0 = tok_tile * MQ_T;
    const uint32_t nchunks = (nb + MQ_KC - 1) / MQ_KC;
    const uint32_t c_begin = slice * q.cps, c_end = c_begin + q.cps < nchunks ? c_begin + q.cps : nchunks;

    /* this lane's dword of a staged row / token: field k % 9 of block k / 9 (rows), or int8 dword k
     * (k < 56) / scale k - 56 (tokens) */
    const uint32_t kb = l / 9, kf = l % 9;
    const bool wlane = l < 63;
    const uint32_t wdst = !wlane ? MQ_SINK : kf == 0 ? MQ_WS + kb * MQ_SP : MQ_A + (kb * 4 + (kf - 1) / 2) * MQ_PL + (kf - 1) % 2;
    const uint32_t wstep = !wlane ? 0u : kf == 0 ? 1u : 2u; /* per row */
    const uint32_t xb = l < 56 ? l / 8 : l - 56, xk = (l % 8) / 2, xh = l % 2;
    const uint32_t xdst = !wlane ? MQ_SINK + 1 : l < 56 ? MQ_B + (xb * 4 + xk) * MQ_PL + xh : MQ_XS + xb * MQ_SP;
    const uint32_t xstep = !wlane ? 0u : l < 56 ? 2u : 1u;

    /* buffer resources over this tile's rows and tokens: a load past the matrix (or past the batch)
     * returns 0, and a lane with no dword to load passes an offset past every record (2^31 plus at
     * most 60 rows), so the loads need no branch and no clamp; the per-load row step is part of the
     * range-checked vector offset */
    const uint32_t rows = I.rows, ntok = a.ntok, xs = a.xstride;
    const size_t rbytes = I.row_bytes;
    const __amdgpu_buffer_rsrc_t wsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(I.w + (size_t)r0 * rbytes), (short)0, (int)((rows - r0) * rbytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t qsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.xq + (size_t)t0 * xs * QK), (short)0, (int)((size_t)(ntok - t0) * xs * QK), 0x00020000);
    const __amdgpu_buffer_rsrc_t dsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.xd + (size_t)t0 * xs), (short)0, (int)((size_t)(ntok - t0) * xs * 4), 0x00020000);
    constexpr uint32_t OOB = 0x80000000u;
    uint32_t wv[MQ_LD], qv[MQ_LD], dv[MQ_LD];
    uint32_t wo = OOB, qo = OOB, dof = OOB;
    /* chunk c's offsets, then its loads i0..i1 */
    auto fetch_setup = [&](uint32_t c) __attribute__((always_inline)) {
        const uint32_t b0 = c * MQ_KC, nbc = nb - b0 < MQ_KC ? nb - b0 : MQ_KC; /* blocks in this chunk */
        wo = wlane && kb < nbc ? w * (uint32_t)rbytes + b0 * Q8_BYTES + 4 * l : OOB;
        qo = l < 56 && xb < nbc ? (w * xs + b0) * QK + 4 * l : OOB;
        dof = l >= 56 && wlane && xb < nbc ? (w * xs + b0 + xb) * 4 : OOB;
    };
    auto fetch_part = [&](uint32_t i0, uint32_t i1) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = i0; i < i1; ++i) {
            wv[i] = __builtin_amdgcn_raw_buffer_load_b32(wsrc, wo + 4 * i * (uint32_t)rbytes, 0, 0);
            qv[i] = __builtin_amdgcn_raw_buffer_load_b32(qsrc, qo + 4 * i * xs * QK, 0, 0);
            dv[i] = __builtin_amdgcn_raw_buffer_load_b32(dsrc, dof + 4 * i * xs * 4, 0, 0);
        }
    };
    auto stage = [&](uint32_t buf) __attribute__((always_inline)) {
        uint32_t *B = lds + buf * MQ_BUF;
#pragma unroll
        for (uint32_t i = 0; i < MQ_LD; ++i) { /* no branch: lane 63 writes the sink */
            const uint32_t rr = w + 4 * i;
            B[wdst + rr * wstep] = wv[i];
            B[xdst + rr * xstep] = qv[i] | dv[i]; /* at most one of them is a record; merged here, not
                                                   * at the loads, so no wait follows the loads */
        }
    };

    const uint32_t wr = w / 2, wt = w % 2, g4 = l / 16, c16 = l % 16;
    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.0f;
    const v4i zero = {0, 0, 0, 0};

    if (c_begin < c_end) {
        fetch_setup(c_begin);
        fetch_part(0, MQ_LD);
        __builtin_amdgcn_sched_barrier(0); /* every load issued before the first wait */
        stage(0);
    }
    __syncthreads();
    for (uint32_t c = c_begin; c < c_end; ++c) {
        const uint32_t buf = (c - c_begin) & 1u;
        const bool more = c + 1 < c_end; /* uniform */
        if (more) { /* the next chunk's loads, in flight during this one (spreading them over the blocks
                     * measured slower) */
            fetch_setup(c + 1);
            fetch_part(0, MQ_LD);
        }
        const uint32_t *B = lds + buf * MQ_BUF;
        const uint32_t nbc = nb - c * MQ_KC < MQ_KC ? nb - c * MQ_KC : MQ_KC;
        /* a block in two parts, so the next block's operand reads and MFMAs are in flight while this
         * block's scales are applied: issue = A/B operand reads and the four MFMAs, finish = the
         * scale reads and acc = fma(ws * xs, float(S), acc) */
        auto issue = [&](uint32_t bb, v4i (&S)[2][2]) __attribute__((always_inline)) {
            long av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint2 x = *(const uint2 *)&B[MQ_A + (bb * 4 + g4) * MQ_PL + 2 * (32 * wr + 16 * i + c16)];
                av[i] = (long)(((unsigned long)x.y << 32) | x.x);
                const uint2 y = *(const uint2 *)&B[MQ_B + (bb * 4 + g4) * MQ_PL + 2 * (32 * wt + 16 * i + c16)];
                bv[i] = (long)(((unsigned long)y.y << 32) | y.x);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) S[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bv[j], zero, 0, 0, 0);
        };
        auto finish = [&](uint32_t bb, const v4i (&S)[2][2]) __attribute__((always_inline)) {
            float4 ws[2];
            float xs[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) ws[i] = *(const float4 *)&B[MQ_WS + bb * MQ_SP + 32 * wr + 16 * i + 4 * g4];
#pragma unroll
            for (int j = 0; j < 2; ++j) xs[j] = __uint_as_float(B[MQ_XS + bb * MQ_SP + 32 * wt + 16 * j + c16]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j][0] = __builtin_fmaf(ws[i].x * xs[j], (float)S[i][j][0], acc[i][j][0]);
                    acc[i][j][1] = __builtin_fmaf(ws[i].y * xs[j], (float)S[i][j][1], acc[i][j][1]);
                    acc[i][j][2] = __builtin_fmaf(ws[i].z * xs[j], (float)S[i][j][2], acc[i][j][2]);
                    acc[i][j][3] = __builtin_fmaf(ws[i].w * xs[j], (float)S[i][j][3], acc[i][j][3]);
                }
        };
        v4i S0[2][2], S1[2][2];
        if (nbc == MQ_KC) {
            issue(0, S0);
#pragma unroll
            for (uint32_t bb = 0; bb < MQ_KC; ++bb) {
                if (bb + 1 < MQ_KC) issue(bb + 1, (bb & 1u) ? S0 : S1);
                finish(bb, (bb & 1u) ? S1 : S0);
            }
        } else {
            for (uint32_t bb = 0; bb < nbc; ++bb) {
                issue(bb, S0);
                finish(bb, S0);
            }
        }
        if (more) stage(buf ^ 1u); /* the other buffer was last read before the previous barrier */
        __syncthreads();
    }

    /* outputs: lane holds rows 4*g4 + v of each row tile i, token c16 of each token tile j */
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t r = r0 + 32 * wr + 16 * i + 4 * g4 + v, t = t0 + 32 * wt + 16 * j + c16;
                if (r < I.rows && t < a.ntok) {
                    if (q.slices > 1)
                        q.part[((size_t)slice * a.ntok + t) * q.total_rows + I.tile_begin * MQ_R + r] = acc[i][j][v];
                    else
                        store_out(I, a.flag, t, r, acc[i][j][v]);
                }
            }
}

/* The slices' partial sums added in slice order, then bias, finiteness and the residual add. */
__global__ __launch_bounds__(256) void k_mq8_reduce(MqArgs q) {
    const MatArgs &a = q.m;
    const uint64_t gi = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= (uint64_t)a.ntok * q.total_rows) return;
    const uint32_t t = (uint32_t)(gi / q.total_rows), rr = (uint32_t)(gi % q.total_rows);
    const uint32_t it = mq_item(a, rr / MQ_R); /* tile_begin counts 64-row tiles: items start on tile edges */
    const Item &I = a.item[it];
    const uint32_t r = rr - I.tile_begin * MQ_R;
    if (r >= I.rows) return;
    float s = q.part[(size_t)t * q.total_rows + rr];
    for (uint32_t k = 1; k < q.slices; ++k) s = s + q.part[((size_t)k * a.ntok + t) * q.total_rows + rr];
    store_out(I, a.flag, t, r, s);
}

/* ------------------------------------------------------------------------
 * Prefill GEMM on f16 MFMA with the activation held in registers (Q8 rows of
 * MH_NB blocks: the 896-wide projections and the LM head). Same contract as
 * the int8 kernels: out[t][r] = the blocks in order of
 * acc = fma(wscale * xscale, S, acc), S the exact block sum. The quants are
 * exact in f16, and v_mfma_f32_16x16x32_f16 adds 32 products of at most
 * 127^2 in f32: every partial sum is an integer below 2^24, so S is exact
 * whatever the order of the additions, and the outputs equal the int8
 * kernel's bit for bit with no convert in the epilogue (a multiply and a
 * fused add per output and block).
 *
 * Layout. Wave w holds the B operands of 16 tokens (t0 + 16w + l%16, K group
 * l/16) for every block, converted to f16 once (MH_NB x 4 registers), and
 * their scales. The tokens and their scales arrive by 16-byte loads of
 * whole rows (14 + 2 per lane) and pass through the wave's own LDS rows to
 * reach operand order; the weight buffers later take the same bytes. The weights stream through LDS in 16-row subtiles: thread
 * (row, block) loads its 36-byte block (consecutive threads take consecutive
 * blocks of a row, one coalesced run) and writes the scale to Wb[block][row]
 * and the quants as f16 into the operand planes Ab[block][k group][row] (a
 * lane's A operand is one 16-byte read; the planes are padded by 16 bytes so
 * the staging writes spread over the banks). Persistent workgroups: each
 * takes one token tile and a contiguous range of subtiles; while subtile i is
 * computed, subtile i+1's loads have landed in registers and i+2's are in
 * flight (two LDS buffers, one barrier per subtile). The reads of the
 * outputs' bias and prior travel with the subtile's weight loads.
 * ---------------------------------------------------------------------- */
constexpr uint32_t MH_NB = 28;             /* blocks per row (896 columns) */
constexpr uint32_t MH_R = 16;              /* rows per subtile */
constexpr uint32_t MH_PLANE = 4 * MH_R + 1; /* 16-byte operand entries per block, one of them padding */
constexpr uint32_t MH_WP = 20;             /* scale plane pitch (floats) */
constexpr uint32_t MH_TP = MH_NB * QK + 16; /* a staged token's pitch in bytes (padded: the operand reads spread) */
constexpr uint32_t MH_BUF_BYTES = 2 * MH_NB * (MH_PLANE * 16 + MH_WP * 4); /* the two weight buffers */
/* dynamic LDS: the weight buffers, or (before them, in the same bytes) the waves' token staging */
constexpr uint32_t MH_WAVE_STAGE = 16 * MH_TP + 16 * MH_NB * 4; /* a wave's token rows, then their scales */
constexpr size_t mh_lds_bytes(uint32_t nw) {
    return (size_t)nw * MH_WAVE_STAGE > MH_BUF_BYTES ? (size_t)nw * MH_WAVE_STAGE : (size_t)MH_BUF_BYTES;
}

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

/* Four int8 (one dword) as four exact f16 (two dwords): byte b becomes the half
 * 0x6400 | (b ^ 0x80) = 1024 + (b + 128), then 1152 is taken off. */
__device__ __forceinline__ uint2 i8x4_f16(uint32_t q) {
    const uint32_t u = q ^ 0x80808080u;
    const h2v m = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2v lo = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - m;
    const h2v hi = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - m;
    return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

/* Lane V of each quad of lanes, to every lane of the quad (DPP quad_perm [V,V,V,V]). */
template <int V>
__device__ __forceinline__ float quad_lane(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), V * 0x55, 0xf, 0xf, false));
}

struct MhArgs {
    MatArgs m;
    uint32_t subtiles, tok_tiles, per; /* per: workgroups per token tile */
};

/* PRE: some item has a bias or adds to its output (their reads travel with the weight loads) */
template <uint32_t NW, bool PRE>
__global__ __launch_bounds__(64 * NW, 8 / NW) void k_gemm_mh(MhArgs q) {
    constexpr uint32_t NB = MH_NB, T = 64 * NW, TASKS = MH_R * NB, TPT = (TASKS + T - 1) / T;
    constexpr uint32_t RB = NB * Q8_BYTES, OOB = 0x80000000u;
    constexpr uint32_t MH_AHEAD = NW == 8 ? 8 : 4; /* operand reads ahead in the product loop (within the registers) */
    extern __shared__ __attribute__((aligned(16))) uint4 mh_lds[];
    uint4 *const Ab = mh_lds;                                  /* [2][NB * MH_PLANE] */
    float *const Wb = (float *)(mh_lds + 2 * NB * MH_PLANE);  /* [2][NB * MH_WP] */
    const MatArgs &a = q.m;
    const uint32_t tid = threadIdx.x, l = tid % 64, w = tid / 64, g = l / 16, c16 = l % 16;

    /* workgroup -> (token tile, range of subtiles): an XCD's workgroups take neighbouring ranges */
    const uint32_t G = gridDim.x, xcd = blockIdx.x % 8u, kk = blockIdx.x / 8u;
    const uint32_t per8 = G / 8u, extra = G % 8u;
    const uint32_t L = xcd * per8 + (xcd < extra ? xcd : extra) + kk;
    const uint32_t tt = L % q.tok_tiles, p = L / q.tok_tiles;
    const uint32_t s_begin = (uint32_t)((uint64_t)q.subtiles * p / q.per);
    const uint32_t n = (uint32_t)((uint64_t)q.subtiles * (p + 1) / q.per) - s_begin;
    const uint32_t ntok = a.ntok, t0 = tt * 16 * NW, tok = t0 + 16 * w + c16;
    const bool live = t0 + 16 * w < ntok; /* this wave holds at least one token (uniform) */

    /* staging role: (row, block) tasks of a subtile, blocks of a row on consecutive threads */
    uint32_t trow[TPT], tblk[TPT];
    bool tuse[TPT];
#pragma unroll
    for (uint32_t j = 0; j < TPT; ++j) {
        const uint32_t k = tid + T * j;
        tuse[j] = k < TASKS;
        trow[j] = k / NB;
        tblk[j] = k % NB;
    }

    /* Every step issues the same vector memory operations whatever the data (loads of a subtile past
     * the range and of rows past an item read 0 from an empty or ending range; stores past the batch
     * or the rows are dropped by the range check): the compiler's waits for a slot's loads then count
     * only what was issued after them, and the next subtiles' loads stay in flight. */
    u4a wa[2][TPT], wb[2][TPT];
    uint32_t wc[2][TPT];
    OutPre cur[4];
    const uint32_t s_end = s_begin + n;
    /* subtile s's weight loads into a slot (rows past the item read 0: the range ends at its last
     * row) */
    auto issue = [&](uint32_t s, u4a (&xa)[TPT], u4a (&xb)[TPT], uint32_t (&xc)[TPT])
        __attribute__((always_inline)) {
        const bool has = s < s_end; /* uniform */
        const uint32_t sv = has ? s : s_begin;
        const Item I = pick_item(a, sv);
        const uint32_t r_sub = (sv - I.tile_begin) * MH_R;
        const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(I.w + (size_t)r_sub * RB), (short)0, has ? (int)((I.rows - r_sub) * RB) : 0, 0x00020000);
#pragma unroll
        for (uint32_t j = 0; j < TPT; ++j) {
            const uint32_t off = tuse[j] ? trow[j] * RB + tblk[j] * Q8_BYTES : OOB;
            xa[j] = __builtin_amdgcn_raw_buffer_load_b128(src, off, 0, 0);
            xb[j] = __builtin_amdgcn_raw_buffer_load_b128(src, off + 16, 0, 0);
            xc[j] = __builtin_amdgcn_raw_buffer_load_b32(src, off + 32, 0, 0);
        }
    };
    /* the bias and prior of subtile s's outputs, one step before they are stored */
    auto load_pre = [&](uint32_t s, OutPre (&o)[4]) __attribute__((always_inline)) {
        if constexpr (PRE) {
            const bool has = s < s_end; /* uniform */
            const uint32_t sv = has ? s : s_begin;
            const Item I = pick_item(a, sv);
            const uint32_t r_sub = (sv - I.tile_begin) * MH_R;
            const __amdgpu_buffer_rsrc_t bsrc = __builtin_amdgcn_make_buffer_rsrc(
                (void *)I.bias, (short)0, I.bias ? (int)(I.rows * 4) : 0, 0x00020000);
            const __amdgpu_buffer_rsrc_t ysrc = __builtin_amdgcn_make_buffer_rsrc(
                (void *)I.y, (short)0, I.accumulate ? (int)((size_t)ntok * I.y_stride * 4) : 0, 0x00020000);
#pragma unroll
            for (uint32_t v = 0; v < 4; ++v) {
                const uint32_t r = r_sub + 4 * g + v;
                const bool ok = has && tok < ntok && r < I.rows;
                o[v].bias = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(bsrc, ok ? r * 4 : OOB, 0, 0));
                o[v].cell = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    ysrc, ok ? (uint32_t)((tok * I.y_stride + r) * 4) : OOB, 0, 0));
            }
        }
    };
    /* slot -> LDS buffer: the scale, and the quants as f16 in operand order */
    auto stage = [&](const u4a (&xa)[TPT], const u4a (&xb)[TPT], const uint32_t (&xc)[TPT], uint32_t buf)
        __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t j = 0; j < TPT; ++j)
            if (tuse[j]) {
                Wb[buf * NB * MH_WP + tblk[j] * MH_WP + trow[j]] = __uint_as_float(xa[j].x);
                const uint32_t qd[8] = {xa[j].y, xa[j].z, xa[j].w, xb[j].x, xb[j].y, xb[j].z, xb[j].w, xc[j]};
                uint4 *e = &Ab[buf * NB * MH_PLANE + tblk[j] * MH_PLANE + trow[j]];
#pragma unroll
                for (uint32_t gi = 0; gi < 4; ++gi) {
                    const uint2 lo = i8x4_f16(qd[2 * gi]), hi = i8x4_f16(qd[2 * gi + 1]);
                    e[gi * MH_R] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                }
            }
    };

    const uint32_t n_ = n; /* subtiles of this workgroup */
    issue(s_begin, wa[0], wb[0], wc[0]);

    /* this wave's tokens: K group g of token `tok` for every block, as f16, and their scales (a token
     * past the batch reads 0) */
    h8v Bq[NB];
    float xsc[NB];
    {
        const uint32_t xs = a.xstride;
        const __amdgpu_buffer_rsrc_t qsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)a.xq, (short)0, (int)((size_t)ntok * xs * QK), 0x00020000);
        const __amdgpu_buffer_rsrc_t dsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)a.xd, (short)0, (int)((size_t)ntok * xs * 4), 0x00020000);
        /* the wave's 16 token rows in 16-byte pieces, consecutive lanes on consecutive pieces */
        constexpr uint32_t PR = NB * QK / 16, NPC = 16 * PR / 64; /* pieces per row, per lane */
        static_assert(16 * PR % 64 == 0, "whole pieces per lane");
        u4a pc[NPC];
#pragma unroll
        for (uint32_t j = 0; j < NPC; ++j) {
            const uint32_t P = 64 * j + l, tp = P / PR, t = t0 + 16 * w + tp;
            pc[j] = __builtin_amdgcn_raw_buffer_load_b128(qsrc, t < ntok ? t * xs * QK + 16 * (P % PR) : OOB, 0, 0);
        }
        /* the 16 tokens' scales in 16-byte pieces too (rows of NB floats, 16-byte aligned) */
        constexpr uint32_t SPR = NB / 4, NSP = (16 * SPR + 63) / 64; /* scale pieces per row, per lane */
        u4a sp[NSP];
#pragma unroll
        for (uint32_t j = 0; j < NSP; ++j) {
            const uint32_t P = 64 * j + l, t = t0 + 16 * w + P / SPR;
            sp[j] = __builtin_amdgcn_raw_buffer_load_b128(
                dsrc, P < 16 * SPR && t < ntok ? (t * xs + 4 * (P % SPR)) * 4 : OOB, 0, 0);
        }
        unsigned char *const stg = (unsigned char *)mh_lds + w * MH_WAVE_STAGE; /* this wave's rows */
        float *const stg_d = (float *)(stg + 16 * MH_TP);                      /* and their scales */
#pragma unroll
        for (uint32_t j = 0; j < NPC; ++j) {
            const uint32_t P = 64 * j + l;
            *(u4a *)(stg + (P / PR) * MH_TP + 16 * (P % PR)) = pc[j];
        }
#pragma unroll
        for (uint32_t j = 0; j < NSP; ++j) {
            const uint32_t P = 64 * j + l;
            if (P < 16 * SPR) *(u4a *)(stg_d + 4 * P) = sp[j];
        }
        /* the wave's own rows: its writes are complete before its reads */
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (uint32_t b = 0; b < NB; ++b) {
            const uint2 v = *(const uint2 *)(stg + c16 * MH_TP + b * QK + 8 * g);
            const uint2 lo = i8x4_f16(v.x), hi = i8x4_f16(v.y);
            Bq[b] = __builtin_bit_cast(h8v, make_uint4(lo.x, lo.y, hi.x, hi.y));
        }
#pragma unroll
        for (uint32_t j = 0; j < NB / 4; ++j) {
            const float4 v = *(const float4 *)(stg_d + c16 * NB + 4 * j);
            xsc[4 * j] = v.x;
            xsc[4 * j + 1] = v.y;
            xsc[4 * j + 2] = v.z;
            xsc[4 * j + 3] = v.w;
        }
    }
    /* the scales in hand here, so no wait inside the subtile loop is for them */
#pragma unroll
    for (uint32_t b = 0; b < NB; ++b) asm volatile("" : : "v"(xsc[b]));
    issue(s_begin + 1, wa[1], wb[1], wc[1]); /* (here: the rows' registers are free) */
    __syncthreads(); /* every wave is done with its rows before the weights take those bytes */
    if (n_ > 0) stage(wa[0], wb[0], wc[0], 0);
    load_pre(s_begin, cur);
    {   /* four stores that the range check drops, where a step stores its outputs: the loop is entered
         * with the operations in flight that each of its steps leaves (so its waits are the steady ones) */
        const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc((void *)a.item[0].y, (short)0, 0, 0x00020000);
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v) __builtin_amdgcn_raw_buffer_store_b32(0u, none, OOB, 0, 0);
    }
    issue(s_begin + 2, wa[0], wb[0], wc[0]);
    __syncthreads();
    bool bad = false; /* a non-finite output of this lane */

    /* subtile i from buffer P; then subtile i+1 (slot P^1) staged into the other buffer, and i+3's loads
     * into the slot it leaves */
    auto step = [&](uint32_t i, uint32_t P) __attribute__((always_inline)) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
            const uint4 *A = Ab + P * NB * MH_PLANE;
            const float *W = Wb + P * NB * MH_WP;
            const f4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
            /* operand reads MH_AHEAD blocks ahead; the empty asm after each block keeps the products
             * and their scale chain in block order (left free, the compiler issues every block's
             * product first and holds all the sums: the registers spill) */
            /* a lane reads one row scale, row 4g + c16 % 4: each quad of lanes holds its four rows'
             * scales, and the multiplies take them by a quad broadcast of their first operand */
            h8v av[MH_AHEAD];
            float wv[MH_AHEAD];
            const uint32_t wrow = 4 * g + (c16 & 3u);
#pragma unroll
            for (uint32_t b = 0; b < MH_AHEAD; ++b) {
                av[b] = __builtin_bit_cast(h8v, A[b * MH_PLANE + g * MH_R + c16]);
                wv[b] = W[b * MH_WP + wrow];
            }
            /* block b+1's product is issued before block b's scale chain reads its sums */
            f4v S = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[0], Bq[0], zero, 0, 0, 0);
#pragma unroll
            for (uint32_t b = 0; b < NB; ++b) {
                const uint32_t k = b % MH_AHEAD;
                f4v Sn = zero;
                if (b + 1 < NB) Sn = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[(b + 1) % MH_AHEAD], Bq[b + 1], zero, 0, 0, 0);
                acc[0] = __builtin_fmaf(quad_lane<0>(wv[k]) * xsc[b], S[0], acc[0]);
                acc[1] = __builtin_fmaf(quad_lane<1>(wv[k]) * xsc[b], S[1], acc[1]);
                acc[2] = __builtin_fmaf(quad_lane<2>(wv[k]) * xsc[b], S[2], acc[2]);
                acc[3] = __builtin_fmaf(quad_lane<3>(wv[k]) * xsc[b], S[3], acc[3]);
                S = Sn;
                asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]) : : "memory");
                if (b + MH_AHEAD < NB) {
                    av[k] = __builtin_bit_cast(h8v, A[(b + MH_AHEAD) * MH_PLANE + g * MH_R + c16]);
                    wv[k] = W[(b + MH_AHEAD) * MH_WP + wrow];
                }
            }
        }
        {   /* the outputs (model.c:259-262 bias, then the finiteness check, then the residual add of
             * model.c:452-455), stored by every lane: one past the batch or the rows is dropped */
            const Item I = pick_item(a, s_begin + i);
            const uint32_t r_sub = (s_begin + i - I.tile_begin) * MH_R;
            const __amdgpu_buffer_rsrc_t ydst = __builtin_amdgcn_make_buffer_rsrc(
                (void *)I.y, (short)0, (int)((size_t)ntok * I.y_stride * 4), 0x00020000);
#pragma unroll
            for (uint32_t v = 0; v < 4; ++v) {
                const uint32_t r = r_sub + 4 * g + v;
                const bool ok = tok < ntok && r < I.rows;
                float val = acc[v];
                if (PRE && I.bias) val = val + cur[v].bias;
                bad = bad || (ok && !(fabsf(val) <= FLT_MAX));
                if (PRE && I.accumulate) val = cur[v].cell + val;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), ydst,
                                                      ok ? (uint32_t)((tok * I.y_stride + r) * 4) : OOB, 0, 0);
            }
        }
        const uint32_t Q = P ^ 1u;
        if (i + 1 < n_) stage(wa[Q], wb[Q], wc[Q], Q);
        load_pre(s_begin + i + 1, cur);
        issue(s_begin + i + 3, wa[Q], wb[Q], wc[Q]);
        __syncthreads();
    };
    /* pairs of steps, then an odd last one: every way round the loop issues the same operations */
    uint32_t i = 0;
    for (; i + 1 < n_; i += 2) {
        step(i, 0);
        step(i + 1, 1);
    }
    if (i < n_) step(i, 0);
    if (a.flag && __ballot(bad) && l == 0) *a.flag = 1;
}

/* ------------------------------------------------------------------------
 * Exact prefill GEMM with the lane sums on f16 MFMA (k_gemm_xm): the results
 * of k_gemm_exact, bit for bit, with the eight lane sums of each (row, token,
 * block) formed by the matrix cores instead of v_dot4.
 * v_mfma_f32_16x16x4_4b_f16 computes four independent 16 x 16 products of
 * K = 4. Instruction h (0, 1) gives its block m lane 4h + m of a Q8 block:
 * A = weight word 4h + m of 16 rows, B = activation word 4h + m of 16
 * tokens, so it returns four of the eight lane sums s_l (kernels.c:36-50) of
 * a 16 x 16 tile. They are exact: int8 values (and Q5 codes - 16) are exact
 * in f16, their products exact in f32, and a sum of four is an integer below
 * 2^24; with C = +0 a zero sum is +0, as v_dot4's convert gives. The VALU
 * keeps the contract's own arithmetic: per lane sum acc_l = acc_l + d * s_l
 * (FAST: fmaf), per output and block one d = wscale * xscale, blocks in
 * order, then the fixed lane tree.
 * Operand layout (checked on MI355X): lane L supplies A[m = L/16][i = L%16][0..3]
 * and B[m][0..3][j = L%16] and receives D[m][4 (L/16) + v][L%16] in register
 * 4m + v, so a lane ends with rows 4 (L/16) + v (v = 0..3) of token L%16 and
 * all eight lane sums of each.
 * Workgroup tile 32 rows x 32 tokens; wave w takes rows 16 (w%2) .. and tokens
 * 16 (w/2) ... K advances in chunks of XM_CB blocks (2 XM_CB for the 16 x 16
 * tiles of the four-wave split, 38 KB of LDS: half the barriers per block,
 * 896x4864 at 128 tokens 35.1 -> 30.9 us): each thread loads one
 * block of a row (Q5: the pair holding it) and one block of a token, turns
 * their eight words into f16 and writes them in MFMA operand order (a wave's
 * operand read is one contiguous 512-byte run); the next chunk's loads are
 * issued before the current chunk is computed.
 * ---------------------------------------------------------------------- */
constexpr uint32_t XM_CB = 8;          /* blocks per K chunk */
constexpr uint32_t XM_PS = 4 * 64 + 4; /* uint2 per block: [group][half][lane] and 32 bytes, so that a staging write
                                        * (8 blocks x 4 rows per 32 lanes) meets 64 distinct banks */
constexpr uint32_t XM_SP = 36;         /* scale plane pitch: 16-byte reads, the 8 x 4 staging writes conflict-free */
static_assert(XM_PS % 32 == 4 && XM_SP % 4 == 0 && XM_SP % 64 == 36, "bank spread of the staging writes");
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));

/* Four bytes of 5-bit codes q as the four exact f16 q - 16: the half 0x6400 | q is 1024 + q. */
__device__ __forceinline__ uint2 q5x4_f16(uint32_t codes) {
    const h2v m = {(_Float16)1040.0f, (_Float16)1040.0f};
    const h2v lo = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, codes, 0x04010400u)) - m;
    const h2v hi = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, codes, 0x04030402u)) - m;
    return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

template <bool FAST>
__device__ __forceinline__ float lane_step_f(float acc, float d, float s) {
    if (FAST) return __builtin_fmaf(d, s, acc);
    const float p = d * s;
    return acc + p;
}

template <bool Q5, bool FAST, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gemm_xm(MatArgs a,
                                                                                           uint32_t tok_tiles) {
    /* S waves share each 16 x 16 tile's eight lane sums: S = 1, 32 x 32 workgroup tiles, a wave all eight
     * lane sums of its tile; S = 2, 16-row x 32-token tiles, wave w tokens 16 (w/2) .. and lane sums
     * 4 (w%2) .. 4 (w%2) + 3; S = 4, one 16 x 16 tile, wave w lane sums 2w, 2w + 1. The parts are joined
     * in the lane tree at the end (S times the workgroups of a shape, 1/S of the chain per wave). */
    static_assert(S == 1 || S == 2 || S == 4, "lane-sum split");
    constexpr uint32_t TR = S == 1 ? 32 : 16, TT = S == 4 ? 16 : 32;
    constexpr uint32_t APS = S == 1 ? XM_PS : 2 * 64 + 4, BPS = S == 4 ? 2 * 64 + 4 : XM_PS;
    constexpr uint32_t CB = S == 4 ? 2 * XM_CB : XM_CB; /* blocks per K chunk: S = 4 stages 16 rows and 16
                                                         * tokens, so a thread per (row, block) takes 16 */
    static_assert(APS % 32 == 4 && BPS % 32 == 4, "bank spread of the staging writes");
    __shared__ __attribute__((aligned(16))) uint2 opa[CB * APS];
    __shared__ __attribute__((aligned(16))) uint2 opb[CB * BPS];
    __shared__ __attribute__((aligned(16))) float wsc[CB][XM_SP];
    __shared__ __attribute__((aligned(16))) float xsc[CB][XM_SP];

    const uint32_t tid = threadIdx.x, nb = a.nb;
    /* XCD-aware order: workgroup i runs on XCD i % 8; each XCD takes a contiguous range of tiles, so
     * the token tiles of one row tile share an L2 */
    const uint32_t G = gridDim.x, xcd = blockIdx.x % 8u, k = blockIdx.x / 8u;
    const uint32_t per = G / 8u, extra = G % 8u;
    const uint32_t L = xcd * per + (xcd < extra ? xcd : extra) + k;
    const uint32_t row_tile = L / tok_tiles, tok_tile = L % tok_tiles;
    const Item I = pick_item(a, row_tile);
    const uint32_t r0 = (row_tile - I.tile_begin) * TR, t0 = tok_tile * TT;

    /* staging: thread (row or token tid/CB, block tid%CB of the chunk); 16-row (16-token) tiles of 8-block
     * chunks: threads below 128 */
    const uint32_t srow = tid / CB, sblk = tid % CB;
    const bool wstage = srow < TR, xstage = srow < TT;
    const bool srow_ok = wstage && r0 + srow < I.rows, stok_ok = xstage && t0 + srow < a.ntok;
    const unsigned char *wrow = I.w + (size_t)(srow_ok ? r0 + srow : 0) * I.row_bytes;
    const size_t tok_base = (size_t)(stok_ok ? t0 + srow : 0) * a.xstride;
    uint32_t wr[Q5 ? 11 : 9] = {};
    uint32_t xr[8] = {};
    float xs = 0.0f;
    auto fetch = [&](uint32_t c) __attribute__((always_inline)) {
        if (Q5) {
            const uint32_t b = c * CB + (sblk & ~1u); /* the pair holding the block (nb even) */
            if (srow_ok && b < nb) {
                const unsigned char *p = wrow + (size_t)b * Q5_BYTES;
                const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                const u3a v2 = *(const u3a *)(p + 32);
                wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
                wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
                wr[8] = v2.x; wr[9] = v2.y; wr[10] = v2.z;
            }
        } else {
            const uint32_t b = c * CB + sblk;
            if (srow_ok && b < nb) {
                const unsigned char *p = wrow + (size_t)b * Q8_BYTES;
                const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
                wr[0] = v0.x; wr[1] = v0.y; wr[2] = v0.z; wr[3] = v0.w;
                wr[4] = v1.x; wr[5] = v1.y; wr[6] = v1.z; wr[7] = v1.w;
                wr[8] = *(const uint32_t *)(p + 32);
            }
        }
        const uint32_t bx = c * CB + sblk;
        if (stok_ok && bx < nb) {
            const int8_t *p = a.xq + (tok_base + bx) * QK;
            const u4a v0 = *(const u4a *)p, v1 = *(const u4a *)(p + 16);
            xr[0] = v0.x; xr[1] = v0.y; xr[2] = v0.z; xr[3] = v0.w;
            xr[4] = v1.x; xr[5] = v1.y; xr[6] = v1.z; xr[7] = v1.w;
            xs = a.xd[tok_base + bx];
        }
    };
    /* no select on the staged words: a row past the matrix or a token past the batch stages whatever its
     * registers hold (zeros, or an earlier chunk's words) and is never stored, since each output takes only
     * its own row's and token's operands; a block past the row is skipped by the block loop (34 fewer VALU
     * per thread and chunk) */
    auto stage = [&]() __attribute__((always_inline)) {
        /* lane word l = 4h + m of row (token) s goes to [block][s / 16][h][s % 16 + 16 m] */
        uint2 *wd = opa + sblk * APS + (srow / 16) * 128 + srow % 16;
        uint2 *xd = opb + sblk * BPS + (srow / 16) * 128 + srow % 16;
        float sc = 0.0f;
        if (!wstage) {
        } else if (Q5) {
            Q5Fields f[2];
            q5_parse_pair(wr, f[0], f[1]);
            const bool second = sblk & 1u;
            Q5Fields q;
            q.scale = second ? f[1].scale : f[0].scale;
            q.high = second ? f[1].high : f[0].high;
#pragma unroll
            for (int j = 0; j < 4; ++j) q.nib[j] = second ? f[1].nib[j] : f[0].nib[j];
            q.even = second ? f[1].even : f[0].even;
            q.odd = second ? f[1].odd : f[0].odd;
#pragma unroll
            for (int l = 0; l < 8; ++l) wd[(l / 4) * 64 + (l % 4) * 16] = q5x4_f16(q5_codes(q, l));
            sc = q.scale;
        } else {
#pragma unroll
            for (int l = 0; l < 8; ++l) wd[(l / 4) * 64 + (l % 4) * 16] = i8x4_f16(wr[1 + l]);
            sc = __uint_as_float(wr[0]);
        }
        if (wstage) wsc[sblk][srow] = sc;
        if (xstage) {
#pragma unroll
            for (int l = 0; l < 8; ++l) xd[(l / 4) * 64 + (l % 4) * 16] = i8x4_f16(xr[l]);
            xsc[sblk][srow] = xs;
        }
    };

    /* this wave's row group rg, token group tg, and (S > 1) the MFMA instruction hs (lane sums 4hs .. 4hs+3)
     * and its first MFMA block mb */
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t rg = S == 1 ? w & 1u : 0u, tg = S == 4 ? 0u : w >> 1;
    const uint32_t hs = S == 2 ? w & 1u : (S == 4 ? w >> 1 : 0u), mb = S == 4 ? 2 * (w & 1u) : 0u;
    constexpr int NL = 8 / S; /* lane sums per output held by this wave */
    float acc[NL][4];
#pragma unroll
    for (int l = 0; l < NL; ++l)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[l][v] = 0.0f;

    const uint32_t nchunks = (nb + CB - 1) / CB;
    fetch(0);
    for (uint32_t c = 0; c < nchunks; ++c) {
        stage();
        __syncthreads();
        if (c + 1 < nchunks) fetch(c + 1);
        const uint32_t count = nb - c * CB < CB ? nb - c * CB : CB;
        auto block = [&](uint32_t bb) __attribute__((always_inline)) {
            if constexpr (S > 1) {
                /* S = 4: a wave whose lane sums are the instruction's blocks 2 and 3 reads the operands of lane
                 * L ^ 32, so that they arrive in blocks 0 and 1 (the result registers are then indexed by
                 * constants; indexing them by the wave's half made the compiler select every element) */
                const uint32_t ol = S == 4 ? lane ^ (mb * 16u) : lane;
                const uint2 *pa = opa + bb * APS + hs * 64 + ol, *pb = opb + bb * BPS + tg * 128 + hs * 64 + ol;
                const h4v a0 = __builtin_bit_cast(h4v, pa[0]), b0 = __builtin_bit_cast(h4v, pb[0]);
                const f16x z = {};
                const f16x s0 = __builtin_amdgcn_mfma_f32_16x16x4f16(a0, b0, z, 0, 0, 0); /* lanes 4hs + mb .. */
                const float4 dw = *(const float4 *)&wsc[bb][4 * (lane >> 4)];
                const float dx = xsc[bb][tg * 16 + (lane & 15u)];
                const float d[4] = {dw.x * dx, dw.y * dx, dw.z * dx, dw.w * dx};
#pragma unroll
                for (int m = 0; m < NL; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[m][v] = lane_step_f<FAST>(acc[m][v], d[v], s0[4 * m + v]);
                return;
            }
            const uint2 *pa = opa + bb * XM_PS + rg * 128 + lane, *pb = opb + bb * XM_PS + tg * 128 + lane;
            const h4v a0 = __builtin_bit_cast(h4v, pa[0]), a1 = __builtin_bit_cast(h4v, pa[64]);
            const h4v b0 = __builtin_bit_cast(h4v, pb[0]), b1 = __builtin_bit_cast(h4v, pb[64]);
            const f16x z = {};
            const f16x s0 = __builtin_amdgcn_mfma_f32_16x16x4f16(a0, b0, z, 0, 0, 0); /* lanes 0-3 */
            const f16x s1 = __builtin_amdgcn_mfma_f32_16x16x4f16(a1, b1, z, 0, 0, 0); /* lanes 4-7 */
            const float4 dw = *(const float4 *)&wsc[bb][rg * 16 + 4 * (lane >> 4)];
            const float dx = xsc[bb][tg * 16 + (lane & 15u)];
            const float d[4] = {dw.x * dx, dw.y * dx, dw.z * dx, dw.w * dx};
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[m][v] = lane_step_f<FAST>(acc[m][v], d[v], s0[4 * m + v]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[(4 + m) % NL][v] = lane_step_f<FAST>(acc[(4 + m) % NL][v], d[v], s1[4 * m + v]);
        };
        /* unrolled with uniform guards: fixed LDS offsets per block, 103-106 registers (four waves per SIMD) */
#pragma unroll
        for (uint32_t bb = 0; bb < CB; ++bb)
            if (bb < count) block(bb);
        __syncthreads();
    }

    float a8[8][4]; /* the eight lane sums of each of this lane's four outputs */
    if constexpr (S == 1) {
#pragma unroll
        for (int l = 0; l < 8; ++l)
#pragma unroll
            for (int v = 0; v < 4; ++v) a8[l][v] = acc[l][v];
    } else { /* the other waves' lane sums through LDS (opa: every read of it ended at the last barrier);
              * the wave holding lane sum 0 of a tile forms the tree */
        constexpr uint32_t XS = S == 2 ? 128 : 64; /* exchange row: a slot per (token group, lane) */
        float *xch = (float *)opa;
        static_assert((8 - NL) * 4 * XS * sizeof(float) <= sizeof(opa), "exchange buffer");
        const uint32_t part = S == 2 ? hs : w, slot = S == 2 ? tg * 64 + lane : lane; /* part: lane sums NL*part.. */
        if (part != 0) {
#pragma unroll
            for (int m = 0; m < NL; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) xch[((part - 1) * NL * 4 + 4 * m + v) * XS + slot] = acc[m][v];
        }
        __syncthreads();
        if (part != 0) return; /* whole waves */
#pragma unroll
        for (int l = 0; l < 8; ++l)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                a8[l][v] = l < NL ? acc[l % NL][v] : xch[((l / NL - 1) * NL * 4 + 4 * (l % NL) + v) * XS + slot];
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) { /* the lane tree of reduce8: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
        const float o = ((a8[0][v] + a8[4][v]) + (a8[2][v] + a8[6][v])) + ((a8[1][v] + a8[5][v]) + (a8[3][v] + a8[7][v]));
        const uint32_t r = r0 + rg * 16 + 4 * (lane >> 4) + v, t = t0 + tg * 16 + (lane & 15u);
        if (r < I.rows && t < a.ntok) store_out(I, a.flag, t, r, o);
    }
}

}  // namespace

hipError_t launch_gemm_xm(MatArgs a, bool q5, bool fast, int split, hipStream_t s) {
    if (split != 1 && split != 2 && split != 4) return hipErrorInvalidValue;
    const uint32_t tr = split == 1 ? 32 : 16, tt = split == 4 ? 16 : 32;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = tiles;
        tiles += (a.item[i].rows + tr - 1) / tr;
    }
    const uint32_t tok_tiles = (a.ntok + tt - 1) / tt;
    if (!tiles || !tok_tiles || !a.nb) return hipSuccess;
    const dim3 grid(tiles * tok_tiles), block(256);
#define SMQ_XM(Q5, FAST)                                                                                \
    do {                                                                                                \
        if (split == 4) hipLaunchKernelGGL((k_gemm_xm<Q5, FAST, 4>), grid, block, 0, s, a, tok_tiles);  \
        else if (split == 2) hipLaunchKernelGGL((k_gemm_xm<Q5, FAST, 2>), grid, block, 0, s, a, tok_tiles); \
        else hipLaunchKernelGGL((k_gemm_xm<Q5, FAST, 1>), grid, block, 0, s, a, tok_tiles);            \
    } while (0)
    if (q5) {
        if (fast) SMQ_XM(true, true);
        else SMQ_XM(true, false);
    } else {
        if (fast) SMQ_XM(false, true);
        else SMQ_XM(false, false);
    }
#undef SMQ_XM
    return hipGetLastError();
}

namespace {
bool g_mh_on = true;
}  // namespace

void set_mh_enabled(bool on) { g_mh_on = on; }
bool mh_enabled() { return g_mh_on; }

bool mh_wanted(const MatArgs &a) {
    if (a.nb != MH_NB || a.ntok < 2 || !mh_enabled() || (((uintptr_t)a.xq) & 7u) || (((uintptr_t)a.xd) & 15u) ||
        a.xstride % 4u)
        return false;
    if ((uint64_t)a.ntok * a.xstride * QK >= (1ull << 31)) return false;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        const Item &I = a.item[i];
        if (I.row_bytes != (size_t)MH_NB * Q8_BYTES || (((uintptr_t)I.w) & 3u)) return false;
        if ((uint64_t)I.rows * I.row_bytes >= (1ull << 31)) return false;
        /* buffer offsets of the outputs below 2^31 */
        if ((uint64_t)a.ntok * I.y_stride * 4 >= (1ull << 31) || I.rows * 4ull >= (1ull << 31)) return false;
    }
    return true;
}

hipError_t launch_mh(MatArgs a, hipStream_t s) {
    static int cus = 0;
    if (!cus) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cus = v;
    }
    MhArgs q;
    uint32_t subtiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = subtiles;
        subtiles += (a.item[i].rows + MH_R - 1) / MH_R;
    }
    if (!subtiles || !a.ntok) return hipSuccess;
    const bool wide = a.ntok > 64; /* eight waves of 16 tokens, else four */
    const uint32_t nw = wide ? 8u : 4u, resident = (uint32_t)cus * (wide ? 1u : 2u);
    q.m = a;
    q.subtiles = subtiles;
    q.tok_tiles = (a.ntok + 16 * nw - 1) / (16 * nw);
    uint32_t per = resident / q.tok_tiles;
    per = per < subtiles ? per : subtiles;
    q.per = per ? per : 1u;
    const dim3 grid(q.per * q.tok_tiles);
    bool pre = false;
    for (uint32_t i = 0; i < a.nitems; ++i) pre = pre || a.item[i].bias || a.item[i].accumulate;
    if (wide && pre) hipLaunchKernelGGL((k_gemm_mh<8, true>), grid, dim3(512), mh_lds_bytes(8), s, q);
    else if (wide) hipLaunchKernelGGL((k_gemm_mh<8, false>), grid, dim3(512), mh_lds_bytes(8), s, q);
    else if (pre) hipLaunchKernelGGL((k_gemm_mh<4, true>), grid, dim3(256), mh_lds_bytes(4), s, q);
    else hipLaunchKernelGGL((k_gemm_mh<4, false>), grid, dim3(256), mh_lds_bytes(4), s, q);
    return hipGetLastError();
}

bool mq8_ok(const MatArgs &a) {
    if (!a.nb || a.ntok < 2 || (((uintptr_t)a.xq | (uintptr_t)a.xd) & 3u)) return false;
    /* buffer offsets stay below 2^31 (the out-of-range offset), and so do 64 rows or tokens of them */
    if ((uint64_t)a.ntok * a.xstride * QK >= (1ull << 31) || (uint64_t)MQ_T * a.xstride * QK >= (1ull << 31))
        return false;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        if ((((uintptr_t)a.item[i].w) | a.item[i].row_bytes) & 3u) return false;
        if ((uint64_t)a.item[i].rows * a.item[i].row_bytes >= (1ull << 31) ||
            (uint64_t)MQ_R * a.item[i].row_bytes >= (1ull << 31))
            return false;
    }
    return true;
}

/* Tiles (64 x 64) below which K is split over slices. At more tiles this kernel measured no faster
 * than the 32 x 64 block-pair kernel (9728 x 896 x 128: 17.5 us against 16.6), so those shapes stay
 * there; below it the slices spread a long K over the CUs (896 x 4864 x 128: 18.5 us against 36). */
constexpr uint32_t MQ_MIN_SPLIT_TILES = 192;

bool mq8_wanted(const MatArgs &a) {
    /* counted in the 32 x 64 tiles of the block-pair kernel: where it has enough workgroups on its own
     * (e.g. 896 x 4864 at 512 tokens: 224), splitting K (a second launch, the partials' traffic) does
     * not pay */
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) tiles += (a.item[i].rows + 31) / 32;
    return mq8_ok(a) && tiles * ((a.ntok + MQ_T - 1) / MQ_T) < MQ_MIN_SPLIT_TILES && (a.nb + MQ_KC - 1) / MQ_KC >= 4;
}

hipError_t prepare_mq8_attributes() {
    hipError_t e = hipFuncSetAttribute((const void *)k_gemm_mq8, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)MQ_LDS_BYTES);
    const void *mh[4] = {(const void *)k_gemm_mh<8, false>, (const void *)k_gemm_mh<8, true>,
                         (const void *)k_gemm_mh<4, false>, (const void *)k_gemm_mh<4, true>};
    for (int i = 0; i < 4 && e == hipSuccess; ++i)
        e = hipFuncSetAttribute(mh[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)mh_lds_bytes(i < 2 ? 8 : 4));
    return e;
}

hipError_t launch_mq8(MatArgs a, float *ws, size_t ws_bytes, hipStream_t s) {
    MqArgs q;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        a.item[i].tile_begin = tiles;
        tiles += (a.item[i].rows + MQ_R - 1) / MQ_R;
    }
    q.m = a;
    q.row_tiles = tiles;
    q.tok_tiles = (a.ntok + MQ_T - 1) / MQ_T;
    q.total_rows = tiles * MQ_R;
    const uint32_t nchunks = (a.nb + MQ_KC - 1) / MQ_KC, grid1 = tiles * q.tok_tiles;
    if (!grid1 || !a.nb) return hipSuccess;
    if (grid1 >= MQ_MIN_SPLIT_TILES) return hipErrorNotSupported; /* mq8_wanted: the caller checks */
    /* K split so that about 512 workgroups run, at least two chunks each, partial sums within the
     * workspace */
    uint32_t slices = (512 + grid1 - 1) / grid1;
    const uint32_t most = nchunks / 2;
    slices = slices < most ? slices : most;
    const size_t per = (size_t)a.ntok * q.total_rows * sizeof(float);
    const uint32_t fit = per ? (uint32_t)(ws_bytes / per) : 0;
    slices = slices < fit ? slices : fit;
    if (slices < 2) slices = 1;
    q.cps = (nchunks + slices - 1) / slices;
    q.slices = (nchunks + q.cps - 1) / q.cps; /* every slice holds at least one chunk */
    q.part = q.slices > 1 ? ws : nullptr;
    hipLaunchKernelGGL(k_gemm_mq8, dim3(grid1 * q.slices), dim3(MQ_NT), MQ_LDS_BYTES, s, q);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || q.slices == 1) return e;
    const uint64_t n = (uint64_t)a.ntok * q.total_rows;
    hipLaunchKernelGGL(k_mq8_reduce, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, q);
    return hipGetLastError();
}

}  // namespace smq
