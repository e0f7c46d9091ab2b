/* Decode matmuls of one token on packed 28-block Q8 rows (the 896-wide
 * Qwen2.5-0.5B matrices), with the activation formed inside the launch and,
 * for the FFN, the gated product and its Q8 blocks formed in the store.
 *
 * Reference steps fused here (src/model.c:334-415, 496-509, 622-643;
 * vecmath.c:61-93; kernels.c:912-935):
 *  PRO_NORM  RMSNorm of x (sum of squares in element order by one wave,
 *            the running sum moving lane to lane over squares held in
 *            registers, inv = 1/sqrtf(sum/n + eps), (x*inv)*w), then its Q8
 *            blocks;
 *  PRO_F32   the Q8 blocks of the f32 row x;
 *  EPI_STORE each item's rows + bias, finiteness, y or y += result;
 *  EPI_GLU   gate and up rows of 32 outputs h = up*act(gate) (SwiGLU or
 *            GeGLU), their finiteness, and h's Q8 block (silu_quantize);
 *  ROPE      (STORE, items q, k, v of one token) after bias and finiteness,
 *            q and k rows rotated by the position's table row (model.c:442-450;
 *            a row meets its pair partner, the next chain group's row, by a
 *            lane exchange), and k and v also stored into the caches at the
 *            position (model.c:511-526).
 * Every result is bit-identical to the unfused calls.
 *
 * Layout: a workgroup owns RT rows (STORE: a 16-row tile of one item; GLU: 32
 * gate rows and the 32 up rows of the same outputs). Thread t owns the
 * 16-byte piece t % 63 of rows t / 63 + 16 j (one 1 KiB non-temporal load of
 * consecutive bytes per wave instruction), so which block and field each of
 * its dwords holds and where its result goes are fixed for the thread, and
 * work out while the activation loads. The activation's Q8 blocks are kept in
 * the rows' own 36-byte layout, so dword k of a row meets dword k of the
 * activation: one 16-byte LDS read serves all the thread's rows. Eight
 * threads form a block's Q8 (four elements each). The weight bytes are
 * requested once every thread's activation
 * element is in (so no wave's activation load queues behind other waves'
 * weights), and arrive while the RMSNorm's serial sum runs. A block's scale
 * dword stores d = wscale*xscale, a lane dword float(s) of its exact dot4
 * sum; after one barrier chain thread (row, lane) adds d*float(s) in block
 * order, and the DPP lane tree gives the row (the contract of
 * src/kernels.c:36-79).
 */
#include <float.h>
#include <stddef.h>

#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t DC_NT = 1024;
constexpr int DPRO_NORM = 1, DPRO_F32 = 2; /* SMQ_ACT_NORM, SMQ_ACT_F32 */

/* One launch's LDS: per row nine fields of NB floats, f[r][0][b] = the block scale products d
 * and f[r][1 + l][b] = lane l's sums (pitch SP floats, 4 mod 32: distinct banks for one block's
 * eight lane sums), the activation's Q8 blocks laid out as a row (dword 9b = block b's scale,
 * 9b + 1.. its 32 int8), the squares of the RMSNorm, exp_det's table and the rows' results. */
template <uint32_t NB, uint32_t RT, uint32_t SP>
struct DcLds {
    float f[RT * 9 * SP];
    uint32_t act[NB * 9];
    float sq[NB * 32];
    uint64_t etab[32];
    float res[RT];
    float inv;
    int bad;
};

template <bool GLU, int PRO, uint32_t NB, uint32_t RT, uint32_t CPT, bool ROPE = false>
__global__ __launch_bounds__(DC_NT) void k_decode_ct(FusedArgs a) {
    static_assert(NB % 4 == 0 && NB * 8 <= DC_NT, "packed rows of whole 16-byte pieces; four elements per thread");
    constexpr uint32_t NQ = NB * 8;        /* threads holding four activation elements */
    constexpr uint32_t C16 = 9 * NB / 4;   /* pieces per row */
    constexpr uint32_t RG = DC_NT / C16;   /* rows per slab of the tile */
    constexpr uint32_t SP = (NB + 3) / 4 * 4 + (36 - (NB + 3) / 4 * 4 % 32) % 32;
    constexpr uint32_t SLAB = RG * 9 * SP; /* LDS floats between a thread's rows */
    static_assert(SP % 32 == 4 && SP >= NB, "pitch 4 mod 32");
    static_assert((RT * 9 * SP) % 4 == 0, "the activation row starts 16-byte aligned");
    static_assert(RT == CPT * RG, "the tile is CPT slabs of RG rows");
    static_assert(!GLU || (RT == 64 && 32 % RG == 0), "GLU: 32 gate and 32 up rows, a slab in one of them");
    static_assert(!(ROPE && GLU) && RT % 2 == 0, "ROPE: a STORE tile holds whole pairs of rows");
    using Lds = DcLds<NB, RT, SP>;
    __shared__ __attribute__((aligned(16))) Lds L;

    const uint32_t tid = threadIdx.x, n = a.n;
    /* this workgroup's rows: STORE a tile of one item, GLU the 32 outputs of h block blockIdx.x */
    const Item It = GLU ? a.item[0] : pick_item(a, blockIdx.x); /* STORE: this tile's item */
    const uint32_t r0 = GLU ? 0u : (blockIdx.x - It.tile_begin) * RT;

    /* 1. the activation's own loads first: thread t < NQ holds elements 4t..4t+3 (n % 4 == 0 and
     * 16-byte aligned rows: one in-bounds 16-byte load each, zeros past n) */
    float xv[4], wv[4];
    {
        const bool ok = 4 * tid < n;
        const uint32_t e = ok ? 4 * tid : 0;
        const float4 xl = *(const float4 *)(a.src + e);
        xv[0] = ok ? xl.x : 0.0f;
        xv[1] = ok ? xl.y : 0.0f;
        xv[2] = ok ? xl.z : 0.0f;
        xv[3] = ok ? xl.w : 0.0f;
        if constexpr (PRO == DPRO_NORM) {
            const float4 wl = *(const float4 *)(a.norm + e);
            wv[0] = ok ? wl.x : 0.0f;
            wv[1] = ok ? wl.y : 0.0f;
            wv[2] = ok ? wl.z : 0.0f;
            wv[3] = ok ? wl.w : 0.0f;
        } else {
            wv[0] = wv[1] = wv[2] = wv[3] = 0.0f;
        }
    }

    /* 2. the thread's weight pieces: piece pc of rows rg + RG*j (threads past the RG slab rows,
     * and rows past a matrix, re-read an in-bounds row that is never stored); dword k = 4*pc + q
     * of a row is field k % 9 of block k / 9, and its result goes to at[q] + j*SLAB */
    const uint32_t pc = tid % C16, rg = tid / C16;
    const bool owner = rg < RG;
    const u4a *wp[CPT];
#pragma unroll
    for (uint32_t j = 0; j < CPT; ++j) {
        const uint32_t rr = (owner ? rg : 0) + RG * j;
        const unsigned char *w;
        size_t rb;
        uint32_t row, rows;
        if constexpr (GLU) {
            const Item &I = a.item[j < 32 / RG ? 0 : 1]; /* slabs of the gate rows, then the up rows */
            w = I.w;
            rb = I.row_bytes;
            rows = a.rows;
            row = blockIdx.x * 32 + (rr & 31u);
        } else {
            w = It.w;
            rb = It.row_bytes;
            rows = It.rows;
            row = r0 + rr;
        }
        row = row < rows ? row : rows - 1;
        wp[j] = (const u4a *)(w + (size_t)row * rb + 16 * pc);
    }
    uint32_t at[4];
    bool isd[4];
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t k = 4 * pc + q, b = k / 9, f = k % 9;
        isd[q] = f == 0;
        at[q] = (rg * 9 + f) * SP + b;
    }
    /* the epilogue's own loads: exp_det's table (GLU), or the bias and accumulated cell of the
     * thread's output row (STORE), so the stores wait on no memory round trip */
    const uint32_t cr = tid / 8, cl = tid % 8;
    uint64_t ev = 0;
    OutPre pre = {0.0f, 0.0f};
    if constexpr (GLU) {
        if (tid < 32) ev = EXP2_TABLE[tid];
    } else {
        if (tid < RT * 8 && cl == 7 && r0 + cr < It.rows) pre = load_out(It, 0, r0 + cr);
    }
    /* ROPE: the item's role (0 q, 1 k, 2 v), the position, this row's table entries */
    uint32_t role = 0, rpos = 0;
    bool rok = false;
    float rc = 0.0f, rs = 0.0f;
    if constexpr (ROPE) {
        role = blockIdx.x >= a.item[2].tile_begin ? 2u : (blockIdx.x >= a.item[1].tile_begin ? 1u : 0u);
        rpos = a.rope.pos_dev ? (uint32_t)*a.rope.pos_dev : a.rope.pos0;
        rok = rpos < a.rope.context;
        const uint32_t pr = ((r0 + cr) % a.rope.head_dim) / 2;
        if (role < 2 && tid < RT * 8 && cl == 7 && pr < a.rope.pairs) {
            const size_t at = (size_t)(rok ? rpos : 0) * a.rope.pairs + pr;
            rc = a.rope.cs[at];
            rs = a.rope.sn[at];
        }
    }
    u4a W[CPT];
    auto fetch = [&]() {
#pragma unroll
        for (uint32_t j = 0; j < CPT; ++j) W[j] = __builtin_nontemporal_load(wp[j]);
    };
    if constexpr (PRO != DPRO_NORM) fetch(); /* no serial sum to hide them behind */

    /* 3. the activation's Q8 blocks into LDS in the rows' own layout (RMSNorm first) */
    if constexpr (PRO == DPRO_NORM) {
        if (tid < NQ) *(float4 *)&L.sq[4 * tid] = make_float4(xv[0] * xv[0], xv[1] * xv[1], xv[2] * xv[2], xv[3] * xv[3]);
        __syncthreads(); /* every activation element is in */
        fetch();
        if (tid < 64) { /* the first wave runs the chain, NB / 2 squares per lane in registers */
            constexpr int KT = NB * 32 / 64;
            float t[KT];
#pragma unroll
            for (int k = 0; k < KT; ++k) t[k] = L.sq[KT * tid + k]; /* +0.0 past n */
            const float ss = wave_chain<KT>(t);
            if (tid == 63) {
                const float iv = 1.0f / sqrtf(ss / (float)n + a.eps); /* model.c:338 */
                L.inv = iv;
                L.bad = !(fabsf(ss) <= FLT_MAX) || !(fabsf(iv) <= FLT_MAX);
            }
        }
        __syncthreads();
    }
    int bad = 0;
    if (tid < NQ) { /* eight threads per block, four elements each (kernels.c:912-935) */
        float v[4], m = 0.0f;
        const float inv = PRO == DPRO_NORM ? L.inv : 1.0f;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const bool valid = 4 * tid + i < n;
            v[i] = xv[i];
            if constexpr (PRO == DPRO_NORM) {
                const float t = xv[i] * inv;
                v[i] = t * wv[i]; /* model.c:340 */
            }
            const float av = fabsf(v[i]);
            bad |= valid && !(av <= FLT_MAX);
            const float am = valid ? av : 0.0f;
            m = am > m ? am : m;
        }
        float o = dpp_f<0xB1>(m); /* the block's other seven threads: lane^1, lane^2, the other quad */
        m = o > m ? o : m;
        o = dpp_f<0x4E>(m);
        m = o > m ? o : m;
        o = dpp_f<0x141>(m);
        m = o > m ? o : m;
        const float scale = m / 127.0f;
        const float qinv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
        uint32_t word = 0;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            int qv = 0;
            if (4 * tid + i < n) {
                const float pq = v[i] * qinv;
                qv = (int)__builtin_rintf(pq);
                qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
            }
            word |= ((uint32_t)qv & 0xffu) << (8 * i);
        }
        L.act[9 * (tid / 8) + 1 + tid % 8] = word;
        if (tid % 8 == 0) L.act[9 * (tid / 8)] = __float_as_uint(scale);
    }
    if (bad && a.flag) *a.flag = 1;
    if (PRO == DPRO_NORM && tid == 0 && L.bad && a.flag) *a.flag = 1;
    if (GLU && tid < 32) L.etab[tid] = ev;
    __syncthreads();

    /* 4. every dword of the thread's pieces meets the activation dword of the same index: a
     * scale dword gives d = wscale * xscale, a lane dword float(s) of its dot4 */
    if (owner) {
        const u4a A = *(const u4a *)&L.act[4 * pc];
        const uint32_t aw[4] = {A.x, A.y, A.z, A.w};
#pragma unroll
        for (uint32_t j = 0; j < CPT; ++j) {
            const uint32_t wd[4] = {W[j].x, W[j].y, W[j].z, W[j].w};
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                const float pd = __uint_as_float(wd[q]) * __uint_as_float(aw[q]);
                const float ps = (float)dot4(wd[q], aw[q], 0);
                L.f[at[q] + j * SLAB] = isd[q] ? pd : ps;
            }
        }
    }
    __syncthreads();

    /* 5. chains: thread (row r, lane l) adds d*float(s) in block order; the lane tree */
    float v = 0.0f;
    if (tid < RT * 8) {
        const float4 *sp = (const float4 *)&L.f[(cr * 9 + 1 + cl) * SP];
        const float4 *dp = (const float4 *)&L.f[cr * 9 * SP];
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
        const uint32_t row = r0 + cr;
        if constexpr (ROPE) {
            const bool mine = tid < RT * 8 && cl == 7 && row < It.rows;
            float x = v;
            if (It.bias) x = x + pre.bias; /* model.c:259-262 */
            if (mine && a.flag && !(fabsf(x) <= FLT_MAX)) *a.flag = 1;
            const float xp = __shfl_xor(x, 8, 64); /* the pair partner's row (row ^ 1), every lane */
            if (mine) {
                const uint32_t j = row % a.rope.head_dim;
                float o = x;
                if (role < 2 && rok && j / 2 < a.rope.pairs) { /* rope4's ac - bs and as + bc */
                    if (j & 1u) {
                        const float as = xp * rs, bc = x * rc;
                        o = as + bc;
                    } else {
                        const float ac = x * rc, bs = xp * rs;
                        o = ac - bs;
                    }
                }
                It.y[row] = o;
                if (role > 0 && rok) (role == 1 ? a.rope.kcache : a.rope.vcache)[(size_t)rpos * a.rope.kv_dim + row] = o;
            }
            if (!rok && tid == 0 && a.flag) *a.flag = 1; /* the position is past the context */
            return;
        }
        if (tid < RT * 8 && cl == 7 && row < It.rows) store_out_pre(It, a.flag, 0, row, v, pre);
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
                    e = exp_det_tab(-uu, L.etab);
                } else {
                    e = exp_det_tab(-gv, L.etab);
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

template <bool GLU, int PRO, bool ROPE = false>
hipError_t launch_dec(FusedArgs a, hipStream_t s) {
    constexpr uint32_t RT = GLU ? 64 : 16;
    constexpr uint32_t CPT = RT / (DC_NT / 63); /* slabs of 16 rows (63 pieces each) */
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
    hipLaunchKernelGGL((k_decode_ct<GLU, PRO, 28, RT, CPT, ROPE>), dim3(blocks), dim3(DC_NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool decode_ct_ok(const FusedArgs &a, bool q5, int pro, bool glu) {
    if (a.rope.kcache) { /* items q, k, v; whole heads of an even width; every row's pair in its tile */
        const RopeStore &r = a.rope;
        if (glu || pro != DPRO_NORM || a.nitems != 3 || !r.head_dim || r.head_dim % 2 || 2 * r.pairs > r.head_dim ||
            a.item[1].rows != r.kv_dim || a.item[2].rows != r.kv_dim || r.kv_dim % r.head_dim ||
            a.item[0].rows % r.head_dim)
            return false;
        for (uint32_t i = 0; i < 3; ++i)
            if (a.item[i].accumulate) return false;
    }
    if (q5 || a.nb != 28 || a.n > 28 * QK || a.n + QK <= 28 * QK || (pro != DPRO_NORM && pro != DPRO_F32)) return false;
    if (a.n % 4 || ((uintptr_t)a.src & 15u) || (pro == DPRO_NORM && ((uintptr_t)a.norm & 15u))) return false;
    if (glu && (!a.hd || !a.hq || a.nitems != 2 || ((uintptr_t)a.hd & 3u))) return false;
    for (uint32_t i = 0; i < a.nitems; ++i) {
        const Item &it = a.item[i];
        if ((((uintptr_t)it.w) & 15u) || it.row_bytes != 28 * Q8_BYTES || !it.rows) return false;
    }
    return true;
}

hipError_t launch_decode_ct(const FusedArgs &a, int pro, bool glu, hipStream_t s) {
    if (a.rope.kcache) /* decode_ct_ok admitted: pro RMSNorm, no glu */
        return pro == DPRO_NORM && !glu ? launch_dec<false, DPRO_NORM, true>(a, s) : hipErrorInvalidValue;
    if (glu) return pro == DPRO_NORM ? launch_dec<true, DPRO_NORM>(a, s) : launch_dec<true, DPRO_F32>(a, s);
    return pro == DPRO_NORM ? launch_dec<false, DPRO_NORM>(a, s) : launch_dec<false, DPRO_F32>(a, s);
}

}  // namespace smq
