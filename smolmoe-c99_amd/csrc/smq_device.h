/* Device helpers shared by the gfx950 kernel files: the integer lane
 * products, Q5 unpacking, the fixed lane tree, the in-order chains of the
 * arithmetic contract (src/kernels.c:36-79) and the binary64 exp of
 * src/vecmath.c:61-76. Internal; each including file gets its own copy. */
#ifndef SMQ_DEVICE_H
#define SMQ_DEVICE_H

#include <float.h>
#include <hip/hip_runtime.h>

#include "smq_internal.h"

namespace smq {
namespace {

constexpr int WG = 256;

typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u3a __attribute__((ext_vector_type(3), aligned(4)));
typedef float f4v __attribute__((ext_vector_type(4))); /* register-resident float4 (no struct copies) */

/* Exact int32 sum of four int8 products plus c (v_dot4_i32_i8). The
 * compiler's own instruction, not inline assembly: a dot product's result
 * needs wait states before a VALU reads it, and only the compiler's hazard
 * pass inserts them. The clamp bit selects the three-operand VOP3P form
 * (the two-operand v_dot4c has no clamp): without it the compiler emits
 * v_dot4c, which accumulates into its destination, and copies c (or a zero)
 * there first, one v_mov per product. Clamping saturates only past the int32
 * range; every sum here is below 2^24 in magnitude, so the value is the same. */
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, true);
}

/* IEEE binary16 bits (the low 16 bits of h) to float: one v_cvt_f32_f16,
 * exact for every finite input including subnormals (f16 denormals are not
 * flushed in this build), infinities kept (reference: src/f16.h:10-27). A NaN
 * stays a NaN, quieted as the reference's F16C path quiets it
 * (src/kernels.c:259-261). */
__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

/* One lane step of the contract: acc + d*f with two roundings, or fmaf. */
template <bool FAST>
__device__ __forceinline__ float lane_step(float acc, float d, int s) {
    const float f = (float)s;
    if (FAST) return __builtin_fmaf(d, f, acc);
    const float p = d * f;
    return acc + p;
}

/* The fixed lane reduction over eight consecutive threads (lane = tid & 7):
 * thread 0 ends with ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). IEEE addition is
 * commutative, so the partner's copy of each pair sum is the same bits. */
__device__ __forceinline__ float reduce8(float a) {
    const float s = a + __shfl_xor(a, 4, 8);
    const float t = s + __shfl_xor(s, 2, 8);
    return t + __shfl_xor(t, 1, 8);
}

/* Q5 block fields (docs/FORMAT.md:124-134). */
struct Q5Fields {
    float scale;
    uint32_t high;   /* bit j = bit 4 of element j */
    uint32_t nib[4]; /* byte j: element j low nibble, element j+16 high nibble */
    uint32_t even, odd; /* (high << 4) & 0xf0f0f0f0 and high & 0xf0f0f0f0 (q5_codes) */
};

/* The two words whose bytes feed q5_codes' multiplies, formed once per block and
 * hidden from the optimiser by an empty asm: each lane's byte then reaches its
 * v_mul_u32_u24 as an operand byte select (SDWA src0_sel) instead of a shift
 * and a mask per lane (folded together, the two masks left no byte pattern). */
__device__ __forceinline__ void q5_spread_words(Q5Fields &b) {
    b.even = (b.high << 4) & 0xf0f0f0f0u;
    b.odd = b.high & 0xf0f0f0f0u;
    asm("" : "+v"(b.even), "+v"(b.odd));
}

/* A pair of Q5 blocks is 44 bytes = 11 dwords: the first block's fields sit
 * at 2-byte offsets inside the dwords, the second block's are dword aligned. */
__device__ __forceinline__ void q5_parse_pair(const uint32_t d[11], Q5Fields &b0, Q5Fields &b1) {
    b0.scale = half_to_float(d[0] & 0xffffu);
    b0.high = __builtin_amdgcn_alignbit(d[1], d[0], 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) b0.nib[k] = __builtin_amdgcn_alignbit(d[k + 2], d[k + 1], 16);
    b1.scale = half_to_float(d[5] >> 16);
    b1.high = d[6];
#pragma unroll
    for (int k = 0; k < 4; ++k) b1.nib[k] = d[7 + k];
    q5_spread_words(b0);
    q5_spread_words(b1);
}

/* Lane l's four 5-bit codes q in [0, 31] as bytes: low nibble | high bit << 4.
 * The lane's high bits (h bits 4l..4l+3) sit in the upper nibble of byte l/2
 * of one of two words shared by four lanes each (even lanes (h << 4) &
 * 0xf0f0f0f0, odd lanes h & 0xf0f0f0f0). That byte v = bits << 4 times
 * 0x204081 puts bit i at 8i + 4: the sixteen partial products land on
 * distinct bits (no carries) and the mask keeps the four wanted ones. */
__device__ __forceinline__ uint32_t q5_codes(const Q5Fields &b, int l) {
    const uint32_t src = (l & 1) ? b.odd : b.even;
    /* byte l/2, already shifted: the multiply needs no constant wider than 24
     * bits, so it stays one v_mul_u32_u24 */
    const uint32_t spread = __umul24((src >> (8 * (l >> 1))) & 0xffu, 0x204081u);
    const uint32_t nib = l < 4 ? (b.nib[l] & 0x0f0f0f0fu) : ((b.nib[l - 4] >> 4) & 0x0f0f0f0fu);
    return (spread & 0x10101010u) | nib;
}

/* Product tile layout (pitch GS floats per four blocks): lane l of block bb
 * sits at (bb/4)*GS + tr*32 + l*4 + bb%4, so a chain thread (row tr, lane l)
 * reads four consecutive blocks as one float4. tile_slot is where the task
 * starting at block bb0 writes; a Q5 pair starts at an even bb0, so its two
 * floats of lane l are adjacent: one 8-byte write (put_lane<2>). */
typedef float f2v __attribute__((ext_vector_type(2)));
template <int GS>
__device__ __forceinline__ float *tile_slot(float *pb, uint32_t tr, uint32_t bb0) {
    return pb + (bb0 / 4) * GS + tr * 32 + (bb0 % 4);
}
template <int TB>
__device__ __forceinline__ void put_lane(float *slot, int l, float v0, float v1) {
    if constexpr (TB == 2) *(f2v *)(slot + l * 4) = f2v{v0, v1};
    else slot[l * 4] = v0;
}

/* Signed weights q - 16 as int8 bytes: (q + 112) ^ 0x80 per byte, no carries. */
__device__ __forceinline__ uint32_t q5_signed(const Q5Fields &b, int l) {
    return (q5_codes(b, l) + 0x70707070u) ^ 0x80808080u;
}

__device__ __forceinline__ void store_out(const Item &I, int *flag, uint32_t t, uint32_t r, float v) {
    if (I.bias) v = v + I.bias[r]; /* model.c:259-262 */
    if (flag && !(fabsf(v) <= FLT_MAX)) *flag = 1;
    float *cell = &I.y[(size_t)t * I.y_stride + r];
    if (I.accumulate) v = *cell + v; /* residual: x += out (model.c:452-455) */
    *cell = v;
}

/* The item holding tile `tile` of a fused launch, as a value: every item's
 * fields are read at constant offsets of the kernel arguments and selected, so
 * they arrive in one scalar round trip at entry instead of a second load that
 * waits for the chosen index. */
template <class Args>
__device__ __forceinline__ Item pick_item(const Args &a, uint32_t tile) {
    Item I = a.item[0];
#pragma unroll
    for (uint32_t k = 1; k < MAX_ITEMS; ++k) {
        const Item c = a.item[k];
        const bool take = k < a.nitems && tile >= c.tile_begin;
        I.w = take ? c.w : I.w;
        I.row_bytes = take ? c.row_bytes : I.row_bytes;
        I.bias = take ? c.bias : I.bias;
        I.y = take ? c.y : I.y;
        I.y_stride = take ? c.y_stride : I.y_stride;
        I.rows = take ? c.rows : I.rows;
        I.tile_begin = take ? c.tile_begin : I.tile_begin;
        I.accumulate = take ? c.accumulate : I.accumulate;
    }
    return I;
}

/* A uniform value made ready here: its kernel-argument load is issued with
 * the entry's others instead of inside a later branch. */
template <class T>
__device__ __forceinline__ void sgpr_now(T v) {
    asm volatile("" : : "s"(v));
}

/* store_out with its two reads issued early (load_out at kernel entry): the
 * bias and, for an accumulating item, the cell's old value. The cell is
 * written only by its own thread, at the end, so the early read sees what the
 * late one would. */
struct OutPre {
    float bias, cell;
};
__device__ __forceinline__ OutPre load_out(const Item &I, uint32_t t, uint32_t r) {
    OutPre p = {0.0f, 0.0f};
    if (I.bias) p.bias = I.bias[r];
    if (I.accumulate) p.cell = I.y[(size_t)t * I.y_stride + r];
    return p;
}
__device__ __forceinline__ void store_out_pre(const Item &I, int *flag, uint32_t t, uint32_t r, float v, OutPre p) {
    if (I.bias) v = v + p.bias; /* model.c:259-262 */
    if (flag && !(fabsf(v) <= FLT_MAX)) *flag = 1;
    if (I.accumulate) v = p.cell + v; /* residual: x += out (model.c:452-455) */
    I.y[(size_t)t * I.y_stride + r] = v;
}

/* DPP row shift by N lanes (row_shr:N): lane i reads lane i-N of its row of 16. */
template <int N>
__device__ __forceinline__ float shr_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + N, 0xf, 0xf, false));
}

/* The fixed lane reduction with DPP shifts (no LDS round trip). For eight
 * consecutive threads holding lanes a0..a7, thread 4+i first holds
 * a_i + a_{4+i} = s_i; thread 6 then s0 + s2 and thread 7 s1 + s3; thread 7
 * ends with (s0+s2) + (s1+s3). Only thread 7 of each group is meaningful;
 * every add is one the reference makes, with its operands swapped at most. */
__device__ __forceinline__ float reduce8_to_lane7(float a) {
    const float s = a + shr_dpp<4>(a);
    const float t = s + shr_dpp<2>(s);
    return t + shr_dpp<1>(t);
}

/* One chain thread's step over `count` (<= 4*NQ) products in block order:
 * float4 p[q*ps] holds blocks 4q..4q+3 (fast mode: their scales in
 * d[q*dst]). Up to eight float4 are read at once before the first add
 * (clamped indices); the adds run in block order: acc = acc + p (exact) or
 * fma(d, p, acc). */
template <bool FAST, int G>
__device__ __forceinline__ void chain_read(float4 (&v)[G], float4 (&w)[G], const float4 *p, uint32_t ps,
                                           const float4 *d, uint32_t dst, uint32_t q0, uint32_t nq) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
        const uint32_t qq = q0 + (uint32_t)u < nq ? q0 + (uint32_t)u : nq - 1;
        v[u] = p[qq * ps];
        if (FAST) w[u] = d[qq * dst];
    }
}
template <bool FAST, int G>
__device__ __forceinline__ void chain_add(float &acc, const float4 (&v)[G], const float4 (&w)[G], uint32_t q0,
                                          uint32_t count) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
        const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        const float f[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * (q0 + (uint32_t)u) + (uint32_t)c < count) acc = FAST ? __builtin_fmaf(f[c], e[c], acc) : acc + e[c];
    }
}
/* One chain thread's step over nq <= NQ groups of four products (block
 * order), where every slot of a group past the row's last block holds +0.0:
 * adding +0.0 (or fma(0, 0, acc) in fast mode) leaves acc unchanged, since
 * acc is never -0.0 (it starts at +0.0, and a round-to-nearest sum is -0.0
 * only when both terms are). So the chain is NQ*4 plain dependent adds, with
 * no per-element guard on it; every group is read at once and groups past nq
 * read as zeros, selected off the chain. */
template <bool FAST, int NQ>
__device__ __forceinline__ void chain_sum_padded(float &acc, const float4 *p, uint32_t ps, const float4 *d,
                                                 uint32_t dst, uint32_t nq) {
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 x[NQ], w[NQ];
#pragma unroll
    for (uint32_t u = 0; u < NQ; ++u) {
        const uint32_t gc = u < nq ? u : 0;
        const float4 t = p[gc * ps];
        x[u] = u < nq ? t : zero;
        if (FAST) {
            const float4 tw = d[gc * dst];
            w[u] = u < nq ? tw : zero;
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < NQ; ++u) {
        if (FAST) {
            acc = __builtin_fmaf(w[u].x, x[u].x, acc);
            acc = __builtin_fmaf(w[u].y, x[u].y, acc);
            acc = __builtin_fmaf(w[u].z, x[u].z, acc);
            acc = __builtin_fmaf(w[u].w, x[u].w, acc);
        } else {
            acc = acc + x[u].x;
            acc = acc + x[u].y;
            acc = acc + x[u].z;
            acc = acc + x[u].w;
        }
    }
}

__device__ __forceinline__ float chain_lds_strided(float s, const float4 *a4, uint32_t st, uint32_t n);

template <bool FAST, int NQ>
__device__ __forceinline__ void chain_sum(float &acc, const float4 *p, uint32_t ps, const float4 *d, uint32_t dst,
                                          uint32_t count) {
    const uint32_t nq = (count + 3) / 4;
    if (NQ <= 8) { /* short rows: every read at once */
        float4 x[NQ <= 8 ? NQ : 1], xw[NQ <= 8 ? NQ : 1];
        chain_read<FAST, NQ <= 8 ? NQ : 1>(x, xw, p, ps, d, dst, 0, nq);
        chain_add<FAST, NQ <= 8 ? NQ : 1>(acc, x, xw, 0, count);
        return;
    }
    if (!FAST) { /* wide rows (a few chain threads, many blocks): batched reads */
        acc = chain_lds_strided(acc, p, ps, count);
        return;
    }
    /* fast contract, wide rows: whole float4 first (the compiler unrolls this loop and batches
     * its reads), then the tail */
    const uint32_t full = count / 4;
    uint32_t q = 0;
    for (; q < full; ++q) {
        const float4 v = p[q * ps];
        if (FAST) {
            const float4 dv = d[q * dst];
            acc = __builtin_fmaf(dv.x, v.x, acc);
            acc = __builtin_fmaf(dv.y, v.y, acc);
            acc = __builtin_fmaf(dv.z, v.z, acc);
            acc = __builtin_fmaf(dv.w, v.w, acc);
        } else {
            acc = acc + v.x;
            acc = acc + v.y;
            acc = acc + v.z;
            acc = acc + v.w;
        }
    }
    const uint32_t rem = count - 4 * full;
    if (rem) {
        const float4 v = p[q * ps];
        const float4 dv = FAST ? d[q * dst] : v;
        acc = FAST ? __builtin_fmaf(dv.x, v.x, acc) : acc + v.x;
        if (rem > 1) acc = FAST ? __builtin_fmaf(dv.y, v.y, acc) : acc + v.y;
        if (rem > 2) acc = FAST ? __builtin_fmaf(dv.z, v.z, acc) : acc + v.z;
    }
}

/* s = ((0 + a[0]) + a[1]) + ... + a[n-1] in f32, by one lane: the order of
 * the reference's sequential loops (model.c:337, kernels.c:1150). a is
 * 16-byte aligned LDS. Two register batches alternate so that the reads of
 * one batch are in flight while the other is added (the scheduling barriers
 * keep the compiler from sinking the reads below the adds). */
__device__ __forceinline__ void add_batch(float &s, const float4 (&v)[8]) {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        s = s + v[b].x;
        s = s + v[b].y;
        s = s + v[b].z;
        s = s + v[b].w;
    }
}
__device__ __forceinline__ void read_batch(float4 (&v)[8], const float4 *p, uint32_t stride = 1) {
#pragma unroll
    for (int b = 0; b < 8; ++b) v[b] = p[b * stride];
}
/* lgkmcnt(8) (vmcnt and expcnt at their maxima): at most eight LDS/scalar
 * operations outstanding. LDS reads return in issue order, so after two
 * batches of eight reads this means the older batch has arrived. */
__device__ __forceinline__ void lgkm_wait8() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC87F);
    __builtin_amdgcn_sched_barrier(0);
}

/* s + a[0] + a[1] + ... + a[n-1] in f32, added one at a time in that order
 * (the order of the reference's sequential loops, model.c:337,
 * kernels.c:1150, 1165). a is 16-byte aligned LDS with room for
 * 4*ceil(n/4) floats, each lane may pass its own row, n is uniform across the
 * wave. Batches of 32 floats (eight 16-byte
 * reads) alternate: the next batch's reads are issued, then one wait for the
 * older batch, then its 32 adds, so the chain issues little beyond its adds
 * (measured on MI355X: 6.6-7.0 cycles per add run by a whole wave, against
 * about 10 with a wait before every four adds in one lane). Faster run by a
 * whole wave than by one lane: callers pass every lane of the wave, each
 * with a valid pointer. chain_lds_strided: element 4q + i is component i of
 * a4[q * st]. */
__device__ __forceinline__ float chain_lds_strided(float s, const float4 *a4, uint32_t st, uint32_t n) {
    const uint32_t batches = n / 32; /* 32 floats = 8 float4 per batch */
    uint32_t c = 0;
    if (batches) {
        float4 x[8], y[8];
        read_batch(x, a4, st);
        for (; c + 2 <= batches; c += 2) {
            read_batch(y, a4 + 8 * (c + 1) * st, st);
            lgkm_wait8(); /* x is in */
            add_batch(s, x);
            __builtin_amdgcn_sched_barrier(0);
            read_batch(x, a4 + 8 * (c + 2 < batches ? c + 2 : c + 1) * st, st); /* clamped re-read past the end */
            lgkm_wait8(); /* y is in */
            add_batch(s, y);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < batches) {
            add_batch(s, x);
            ++c;
        }
    }
    const uint32_t rest = n - c * 32; /* < 32: one more batch of 16-byte reads up to the float4 holding
                                         element n-1, terms past it replaced by -0.0f (s + -0.0f == s, bit for bit) */
    if (rest) {
        const float4 *t4 = a4 + 8 * c * st;
        const uint32_t last = (rest - 1) / 4;
        float4 v[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) v[k] = t4[(k < last ? k : last) * st];
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            if (4 * k < rest) { /* uniform */
                s = s + (4 * k + 0 < rest ? v[k].x : -0.0f);
                s = s + (4 * k + 1 < rest ? v[k].y : -0.0f);
                s = s + (4 * k + 2 < rest ? v[k].z : -0.0f);
                s = s + (4 * k + 3 < rest ? v[k].w : -0.0f);
            }
        }
    }
    return s;
}

__device__ __forceinline__ float chain_lds(float s, const float *a, uint32_t n) {
    return chain_lds_strided(s, (const float4 *)a, 1, n);
}

__device__ __forceinline__ float serial_sum_lds(const float *a, uint32_t n) { return chain_lds(0.0f, a, n); }

/* ((0 + t_0) + t_1) + ... + t_{64K-1} in f32 by one whole wave with every term in registers: lane i
 * holds terms K*i .. K*i+K-1 in t[], and the running sum moves one lane per step (a DPP wave_shr:1
 * operand of the step's first add), so lane i adds its K terms to the sum of lanes 0..i-1. Lane 63
 * ends with the total (the other lanes hold partial or unused sums). Every add is one of the
 * sequential loop's, in its order: about 4.8 cycles per term on MI355X, against 7.5 for a chain fed
 * from LDS. Terms past the end of a shorter sequence must be +0.0 or -0.0 (a sum that starts at
 * +0.0 and adds non-negative terms never becomes -0.0, and s + 0.0 == s then). */
template <int K>
__device__ __forceinline__ float wave_chain(const float (&t)[K]) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        /* wave_shr:1 (dpp_ctrl 0x138): lane i reads lane i-1; lane 0 reads the old value 0 */
        s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x138, 0xf, 0xf, false));
#pragma unroll
        for (int k = 0; k < K; ++k) s = s + t[k];
    }
    return s;
}

/* ((0 + a[0]) + a[1]) + ... + a[n-1] from LDS (16-byte aligned) by one whole wave through
 * wave_chain: lane i reads its K consecutive terms (K = the smallest of 4, 8, 10, 12, 16 with 64K >= n;
 * -0.0 past n), then the register chain; longer sequences take the LDS chain. Lane 63 ends with the
 * total (every lane of the wave must call, with the same n). */
template <int K>
__device__ __forceinline__ float wave_chain_lds_k(const float *a, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63u;
    float t[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint32_t i = K * lane + k;
        t[k] = i < n ? a[i] : -0.0f;
    }
    return wave_chain<K>(t);
}
__device__ __forceinline__ float serial_sum_wave(const float *a, uint32_t n) {
    if (n <= 64 * 4) return wave_chain_lds_k<4>(a, n);
    if (n <= 64 * 8) return wave_chain_lds_k<8>(a, n);
    if (n <= 64 * 10) return wave_chain_lds_k<10>(a, n);
    if (n <= 64 * 12) return wave_chain_lds_k<12>(a, n);
    if (n <= 64 * 16) return wave_chain_lds_k<16>(a, n);
    const float s = serial_sum_lds(a, n); /* lane-parallel LDS chain: every lane ends with the total */
    return s;
}

/* 2^(j/32) correctly rounded to binary64, minus j << 47 (vecmath.c:44-52). */
__constant__ uint64_t EXP2_TABLE[32] = {
    0x3ff0000000000000u, 0x3fefd9b0d3158574u, 0x3fefb5586cf9890fu, 0x3fef9301d0125b51u,
    0x3fef72b83c7d517bu, 0x3fef54873168b9aau, 0x3fef387a6e756238u, 0x3fef1e9df51fdee1u,
    0x3fef06fe0a31b715u, 0x3feef1a7373aa9cbu, 0x3feedea64c123422u, 0x3feece086061892du,
    0x3feebfdad5362a27u, 0x3feeb42b569d4f82u, 0x3feeab07dd485429u, 0x3feea47eb03a5585u,
    0x3feea09e667f3bcdu, 0x3fee9f75e8ec5f74u, 0x3feea11473eb0187u, 0x3feea589994cce13u,
    0x3feeace5422aa0dbu, 0x3feeb737b0cdc5e5u, 0x3feec49182a3f090u, 0x3feed503b23e255du,
    0x3feee89f995ad3adu, 0x3feeff76f2fb5e47u, 0x3fef199bdd85529cu, 0x3fef3720dcef9069u,
    0x3fef5818dcfba487u, 0x3fef7c97337b9b5fu, 0x3fefa4afa2a490dau, 0x3fefd0765b6e4540u,
};

/* e^x in binary64, rounded once (vecmath.c:61-76): k = round(32x/ln2) from the
 * low bits of z + 1.5*2^52, remainder r, degree-4 Taylor polynomial of
 * e^(r ln2/32) with separate multiplies and adds, times 2^(k/32). */
__device__ __forceinline__ float exp_det_tab(float x, const uint64_t *tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+5, shift = 0x1.8p+52;
    const double ea = 0x1.62e42fefa39efp-1 / 32;
    const double c1 = ea, c2 = ea * ea / 2, c3 = ea * ea * ea / 6, c4 = ea * ea * ea * ea / 24;
    if (x != x) return x;
    x = x > 89.0f ? 89.0f : (x < -104.0f ? -104.0f : x);
    const double z = inv_ln2_n * (double)x;
    double kd = z + shift;
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - shift;
    const double r = z - kd;
    double p = c4 * r + c3;
    p = p * r + c2;
    p = p * r + c1;
    p = p * r + 1.0;
    const double scale = __longlong_as_double((long long)(tab[ki & 31u] + (ki << 47)));
    return (float)(p * scale);
}

__device__ __forceinline__ float exp_det(float x) { return exp_det_tab(x, EXP2_TABLE); }

/* DPP move of v from another lane of its row of 16 (ctrl: a dpp_ctrl code). */
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

/* Maximum over the 32 lanes of each half-wave (exact: max is order-free):
 * lane^1 and lane^2 (quad_perm), the other quad (row_half_mirror), the other
 * eight (row_mirror), then the other row of 16. All 32 lanes take part. */
__device__ __forceinline__ float max32(float m) {
    float o;
    o = dpp_f<0xB1>(m);
    m = o > m ? o : m;
    o = dpp_f<0x4E>(m);
    m = o > m ? o : m;
    o = dpp_f<0x141>(m);
    m = o > m ? o : m;
    o = dpp_f<0x140>(m);
    m = o > m ? o : m;
    o = __shfl_xor(m, 16, 32);
    return o > m ? o : m;
}

/* Q8 of element i = v of a zero-padded row (kernels.c:912-935): the 32
 * elements of a block sit in 32 consecutive lanes, which all call this. A
 * non-finite element sets bad (its block's values are then unspecified). */
__device__ __forceinline__ void stage_q8(float v, bool valid, uint32_t i, int8_t *q8, float *act_d, int &bad) {
    const float av = fabsf(v);
    bad |= valid && !(av <= FLT_MAX);
    const float m = max32(valid ? av : 0.0f);
    const float scale = m / 127.0f;
    const float inv = scale >= FLT_MIN ? 1.0f / scale : 0.0f;
    int qv = 0;
    if (valid) {
        const float p = v * inv;
        qv = (int)__builtin_rintf(p);
        qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
    }
    q8[i] = (int8_t)qv;
    if ((i & 31u) == 0) act_d[i / QK] = scale;
}

}  // namespace
}  // namespace smq

#endif
