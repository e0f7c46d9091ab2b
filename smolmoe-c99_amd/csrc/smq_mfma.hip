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

}  // namespace

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
    return hipFuncSetAttribute((const void *)k_gemm_mq8, hipFuncAttributeMaxDynamicSharedMemorySize, (int)MQ_LDS_BYTES);
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
