/* Decode matmuls of one token on packed 28-block Q8 rows (the 896-wide
 * Qwen2.5-0.5B matrices), with the activation formed inside the launch and,
 * for the FFN, the gated product and its Q8 blocks formed in the store.
 *
 * Reference steps fused here (src/model.c:334-415, 496-509, 622-643;
 * vecmath.c:61-93; kernels.c:912-935):
 *  PRO_NORM  RMSNorm of x (sum of squares in element order by one lane,
 *            inv = 1/sqrtf(sum/n + eps), (x*inv)*w), then its Q8 blocks;
 *  PRO_F32   the Q8 blocks of the f32 row x;
 *  EPI_STORE each item's rows + bias, finiteness, y or y += result;
 *  EPI_GLU   gate and up rows of 32 outputs h = up*act(gate) (SwiGLU or
 *            GeGLU), their finiteness, and h's Q8 block (silu_quantize).
 * Every result is bit-identical to the unfused calls.
 *
 * Layout: a workgroup owns RT rows (STORE: a 16-row tile of one item; GLU: 32
 * gate rows and the 32 up rows of the same outputs). It requests all its
 * weight bytes at once as 16-byte pieces (one 1 KiB non-temporal load per
 * wave instruction) right after the activation's own loads, so the weights
 * arrive while the RMSNorm's serial sum runs. Then each dword of a piece
 * meets its activation word: a block's scale dword stores d = wscale*xscale,
 * a lane dword stores float(s) of its exact dot4 sum; after one barrier chain
 * thread (row, lane) adds d*float(s) in block order, and the DPP lane tree
 * gives the row (the contract of src/kernels.c:36-79).
 */
#include <float.h>
#include <stddef.h>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t DC_NT = 1024;
constexpr int DPRO_NORM = 1, DPRO_F32 = 2; /* SMQ_ACT_NORM, SMQ_ACT_F32 */

/* One launch's LDS: lane sums sf[r][l][b], block scale products d[r][b] (pitch SP floats, 4 mod
 * 32: distinct banks for one block's eight lane sums), a sink for writes past the tile, the
 * activation's Q8 blocks, the squares of the RMSNorm and the rows' results. */
template <uint32_t NB, uint32_t RT, uint32_t SP>
struct DcLds {
    float sf[RT * 8 * SP];
    float d[RT * SP];
    float sink[64];
    uint32_t act_q[NB * 8];
    float act_d[NB];
    float sq[DC_NT];
    float res[RT];
    float inv;
    int bad;
};

__device__ __forceinline__ uint32_t find_dec_item(const FusedArgs &a, uint32_t tile) {
    uint32_t it = 0;
    if (a.nitems > 1 && tile >= a.item[1].tile_begin) it = 1;
    if (a.nitems > 2 && tile >= a.item[2].tile_begin) it = 2;
    if (a.nitems > 3 && tile >= a.item[3].tile_begin) it = 3;
    return it;
}

template <bool GLU, int PRO, uint32_t NB, uint32_t RT, uint32_t CPT>
__global__ __launch_bounds__(DC_NT) void k_decode_ct(FusedArgs a) {
    static_assert(NB % 4 == 0 && NB * 32 <= DC_NT, "packed rows of whole 16-byte pieces; one element per thread");
    constexpr uint32_t C16 = 9 * NB / 4;
    constexpr uint32_t TCH = RT * C16;
    constexpr uint32_t SP = (NB + 3) / 4 * 4 + (36 - (NB + 3) / 4 * 4 % 32) % 32;
    static_assert(SP % 32 == 4 && SP >= NB, "pitch 4 mod 32");
    static_assert(TCH <= CPT * DC_NT, "each piece of the tile has a thread slot");
    static_assert(!GLU || RT == 64, "GLU: 32 gate and 32 up rows");
    using Lds = DcLds<NB, RT, SP>;
    __shared__ __attribute__((aligned(16))) Lds L;

    const uint32_t tid = threadIdx.x, n = a.n;
    /* this workgroup's rows: STORE a tile of one item, GLU the 32 outputs of h block blockIdx.x */
    uint32_t item = 0, r0 = 0;
    if constexpr (!GLU) {
        item = find_dec_item(a, blockIdx.x);
        r0 = (blockIdx.x - a.item[item].tile_begin) * RT;
    }

    /* 1. the activation's own loads first (loads complete in order) */
    const bool xel = tid < n;
    const float xv = xel ? a.src[tid] : 0.0f;
    const float wv = PRO == DPRO_NORM && xel ? a.norm[tid] : 0.0f;

    /* 2. all the workgroup's weight bytes: piece c = tid + j*DC_NT (row c / C16, 16-byte piece
     * c % C16); rows past a matrix re-read its last row (in bounds, never stored) */
    u4a W[CPT];
#pragma unroll
    for (uint32_t j = 0; j < CPT; ++j) {
        const uint32_t c = tid + j * DC_NT, cc = c < TCH ? c : 0, rr = cc / C16, pc = cc % C16;
        const unsigned char *w;
        size_t rb;
        uint32_t row, rows;
        if constexpr (GLU) {
            const Item &I = a.item[rr < 32 ? 0 : 1];
            w = I.w;
            rb = I.row_bytes;
            rows = a.rows;
            row = blockIdx.x * 32 + (rr & 31u);
        } else {
            const Item &I = a.item[item];
            w = I.w;
            rb = I.row_bytes;
            rows = I.rows;
            row = r0 + rr;
        }
        row = row < rows ? row : rows - 1;
        W[j] = __builtin_nontemporal_load((const u4a *)(w + (size_t)row * rb + 16 * pc));
    }

    /* 3. the activation's Q8 blocks into LDS (RMSNorm first) */
    if constexpr (PRO == DPRO_NORM) {
        if (xel) L.sq[tid] = xv * xv;
        __syncthreads();
        if (tid < 64) { /* the whole first wave runs the chain (faster than one lane) */
            const float ss = serial_sum_lds(L.sq, n);
            if (tid == 0) {
                const float iv = 1.0f / sqrtf(ss / (float)n + a.eps); /* model.c:338 */
                L.inv = iv;
                L.bad = !(fabsf(ss) <= FLT_MAX) || !(fabsf(iv) <= FLT_MAX);
            }
        }
        __syncthreads();
    }
    int bad = 0;
    if (tid < NB * 32) { /* whole half-waves: a block's 32 lanes */
        float v = xv;
        if constexpr (PRO == DPRO_NORM) {
            const float t = xv * L.inv;
            v = t * wv; /* model.c:340 */
        }
        stage_q8(v, xel, tid, (int8_t *)L.act_q, L.act_d, bad);
    }
    if (bad && a.flag) *a.flag = 1;
    if (PRO == DPRO_NORM && tid == 0 && L.bad && a.flag) *a.flag = 1;
    __syncthreads();

    /* 4. every dword of the tile: its lane sum as float, or for a scale d = wscale * xscale */
#pragma unroll
    for (uint32_t j = 0; j < CPT; ++j) {
        const uint32_t c = tid + j * DC_NT, cc = c < TCH ? c : 0, rr = cc / C16, pc = cc % C16;
        const uint32_t wd[4] = {W[j].x, W[j].y, W[j].z, W[j].w};
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t k = 4 * pc + q, b = k / 9, f = k % 9;
            float v;
            uint32_t at;
            if (f == 0) {
                v = __uint_as_float(wd[q]) * L.act_d[b];
                at = (uint32_t)(offsetof(Lds, d) / 4) + rr * SP + b;
            } else {
                v = (float)dot4(wd[q], L.act_q[8 * b + f - 1], 0);
                at = (uint32_t)(offsetof(Lds, sf) / 4) + (rr * 8 + f - 1) * SP + b;
            }
            ((float *)&L)[c < TCH ? at : (uint32_t)(offsetof(Lds, sink) / 4) + (tid & 63u)] = v;
        }
    }
    __syncthreads();

    /* 5. chains: thread (row r, lane l) adds d*float(s) in block order; the lane tree */
    const uint32_t cr = tid / 8, cl = tid % 8;
    float v = 0.0f;
    if (tid < RT * 8) {
        const float4 *sp = (const float4 *)&L.sf[(cr * 8 + cl) * SP];
        const float4 *dp = (const float4 *)&L.d[cr * SP];
        float acc = 0.0f;
#pragma unroll
        for (uint32_t qq = 0; qq < NB / 4; ++qq) {
            const float4 s4 = sp[qq], d4 = dp[qq];
            float p;
            p = d4.x * s4.x; acc = acc + p;
            p = d4.y * s4.y; acc = acc + p;
            p = d4.z * s4.z; acc = acc + p;
            p = d4.w * s4.w; acc = acc + p;
        }
        v = reduce8_to_lane7(acc);
    }

    if constexpr (!GLU) {
        const Item &I = a.item[item];
        const uint32_t row = r0 + cr;
        if (tid < RT * 8 && cl == 7 && row < I.rows) store_out(I, a.flag, 0, row, v);
        return;
    } else {
        /* 6. h = up * act(gate) for the 32 outputs, then their Q8 block (vecmath.c:78-93, model.c:409-415) */
        if (tid < RT * 8 && cl == 7) L.res[cr] = v;
        __syncthreads();
        if (tid < 32) {
            const uint32_t row = blockIdx.x * 32 + tid;
            const bool valid = row < a.rows;
            const float gv = L.res[tid], u = L.res[32 + tid];
            int hbad = valid && (!(fabsf(gv) <= FLT_MAX) || !(fabsf(u) <= FLT_MAX)); /* model.c:309 */
            float hv = 0.0f;
            if (valid) {
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
                hv = u * sg;
                if (a.h) a.h[row] = hv;
            }
            const float av = fabsf(hv);
            hbad |= valid && !(av <= FLT_MAX);
            const float m = max32(valid ? av : 0.0f);
            const float scale = m / 127.0f;
            const float inv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
            int qv = 0;
            if (valid) {
                const float pq = hv * inv;
                qv = (int)__builtin_rintf(pq);
                qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
            }
            a.hq[(size_t)blockIdx.x * QK + tid] = (int8_t)qv;
            if (tid == 0) a.hd[blockIdx.x] = scale;
            if (__ballot(hbad) && tid == 0 && a.flag) *a.flag = 1;
        }
    }
}

template <bool GLU, int PRO>
hipError_t launch_dec(FusedArgs a, hipStream_t s) {
    constexpr uint32_t RT = GLU ? 64 : 16;
    constexpr uint32_t CPT = (RT * 63 + DC_NT - 1) / DC_NT;
    uint32_t blocks = 0;
    if (GLU) {
        blocks = (a.rows + 31) / 32;
    } else {
        for (uint32_t i = 0; i < a.nitems; ++i) {
            a.item[i].tile_begin = blocks;
            blocks += (a.item[i].rows + RT - 1) / RT;
        }
    }
    if (!blocks) return hipSuccess;
    hipLaunchKernelGGL((k_decode_ct<GLU, PRO, 28, RT, CPT>), dim3(blocks), dim3(DC_NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool decode_ct_ok(const FusedArgs &a, bool q5, int pro, bool glu) {
    if (q5 || a.nb != 28 || a.n > 28 * QK || a.n + QK <= 28 * QK || (pro != DPRO_NORM && pro != DPRO_F32)) return false;
    if (glu && (!a.hd || !a.hq || a.nitems != 2 || ((uintptr_t)a.hd & 3u))) return false;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        const Item &it = a.item[i];
        if ((((uintptr_t)it.w) & 15u) || it.row_bytes != 28 * Q8_BYTES || !it.rows) return false;
    }
    return true;
}

hipError_t launch_decode_ct(const FusedArgs &a, int pro, bool glu, hipStream_t s) {
    if (glu) return pro == DPRO_NORM ? launch_dec<true, DPRO_NORM>(a, s) : launch_dec<true, DPRO_F32>(a, s);
    return pro == DPRO_NORM ? launch_dec<false, DPRO_NORM>(a, s) : launch_dec<false, DPRO_F32>(a, s);
}

}  // namespace smq
