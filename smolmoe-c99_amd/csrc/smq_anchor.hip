/* HBM bandwidth anchors (no reference counterpart): what this device's HBM
 * delivers to a plain kernel, measured beside the GEMVs so their share of the
 * 8 TB/s peak can be read against an achievable rate.
 *
 * k_stream_read: every thread reads 16-byte pieces i, i + stride, ... of the
 * buffer (stride = threads in the grid), so each wave instruction reads 1 KiB
 * of consecutive bytes; UNROLL pieces are requested before the first is used.
 * The pieces are folded by xor into one word that is stored only if it equals
 * a constant no test data hits, so no load can be dropped and nothing is
 * written. k_stream_copy moves the pieces the same way (load, then store).
 *
 * Cross-workgroup hand-off anchor: k_grid_barrier measures what one barrier
 * among resident workgroups costs (three kinds, below), against which a
 * persistent kernel replacing dependent launches would be priced.
 */
#include "smq_device.h"
#include "smq_internal.h"

namespace smq {
namespace {

constexpr uint32_t ANCHOR_UNROLL = 8;
constexpr uint32_t ANCHOR_MAGIC = 0x9e3779b9u;

template <bool NT>
__device__ __forceinline__ u4a load16(const u4a *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <bool NT>
__global__ __launch_bounds__(1024) void k_stream_read(const u4a *p, size_t n16, uint32_t *sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (ANCHOR_UNROLL - 1) * stride < n16; i += ANCHOR_UNROLL * stride) {
        u4a v[ANCHOR_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < ANCHOR_UNROLL; ++u) v[u] = load16<NT>(p + i + u * stride);
#pragma unroll
        for (uint32_t u = 0; u < ANCHOR_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u4a v = load16<NT>(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == ANCHOR_MAGIC) *sink = acc;
}

template <bool NT>
__global__ __launch_bounds__(1024) void k_stream_copy(const u4a *src, u4a *dst, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (ANCHOR_UNROLL - 1) * stride < n16; i += ANCHOR_UNROLL * stride) {
        u4a v[ANCHOR_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < ANCHOR_UNROLL; ++u) v[u] = load16<NT>(src + i + u * stride);
#pragma unroll
        for (uint32_t u = 0; u < ANCHOR_UNROLL; ++u) {
            if constexpr (NT) __builtin_nontemporal_store(v[u], dst + i + u * stride);
            else dst[i + u * stride] = v[u];
        }
    }
    for (; i < n16; i += stride) {
        const u4a v = load16<NT>(src + i);
        if constexpr (NT) __builtin_nontemporal_store(v, dst + i);
        else dst[i] = v;
    }
}

/* Grid barrier probe: `episodes` barriers among gridDim.x workgroups, one per CU (the LDS pad keeps a
 * second one off every CU, so a grid no larger than the CU count is resident at once). The words at
 * w: [0, 8*BAR_PAD) eight arrival counters (KIND 1) or one generation word per workgroup (KIND 2),
 * [8*BAR_PAD] the release counter, [9*BAR_PAD] the abort word, [9*BAR_PAD + 16] the timed-out count.
 * Every wait polls at most BAR_SPINS times; a workgroup that gives up raises the abort word, which
 * ends every other wait, so every wave exits whatever the residency. */
constexpr uint32_t BAR_PAD = 64;
constexpr uint32_t BAR_SPINS = 1u << 20;
constexpr uint32_t BAR_LDS_FLOATS = 96 * 1024 / 4;

__device__ __forceinline__ uint32_t bar_acquire(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

/* waits until *word >= target; false if it gave up or another workgroup did */
__device__ __forceinline__ bool bar_wait(uint32_t *word, uint32_t target, uint32_t *abort_word) {
    uint32_t spins = 0;
    while (bar_acquire(word) < target) {
        if (++spins > BAR_SPINS || __hip_atomic_load(abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_store(abort_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    return true;
}

template <int KIND>
__device__ bool grid_barrier(uint32_t *w, uint32_t gen) {
    const uint32_t G = gridDim.x;
    uint32_t *rel = w + 8 * BAR_PAD, *abort_word = w + 9 * BAR_PAD;
    __shared__ int s_ok;
    __syncthreads(); /* the workgroup's work of this phase is done */
    bool ok = true;
    if (KIND == 2) { /* no atomics: own word, workgroup 0 gathers and publishes */
        if (threadIdx.x == 0) __hip_atomic_store(w + blockIdx.x, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        if (blockIdx.x == 0) {
            for (uint32_t i = threadIdx.x; i < G && ok; i += blockDim.x) ok = bar_wait(w + i, gen, abort_word);
            ok = __syncthreads_and(ok);
            if (threadIdx.x == 0 && ok) __hip_atomic_store(rel, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else if (threadIdx.x == 0) {
            ok = bar_wait(rel, gen, abort_word);
        }
    } else if (threadIdx.x == 0) {
        uint32_t target;
        if (KIND == 0) { /* one counter */
            __hip_atomic_fetch_add(rel, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            target = gen * G;
        } else { /* a counter per XCD (workgroups are dealt to the eight XCDs in turn), then one */
            const uint32_t x = blockIdx.x % 8, per = (G - x + 7) / 8;
            const uint32_t old = __hip_atomic_fetch_add(w + x * BAR_PAD, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if (old == gen * per - 1) __hip_atomic_fetch_add(rel, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            target = gen * (G < 8 ? G : 8);
        }
        ok = bar_wait(rel, target, abort_word);
    }
    if (threadIdx.x == 0) s_ok = ok;
    __syncthreads();
    return s_ok != 0;
}

template <int KIND>
__global__ __launch_bounds__(256) void k_grid_barrier(uint32_t *w, uint32_t episodes) {
    __shared__ float pad[BAR_LDS_FLOATS];
    pad[threadIdx.x * 97 % BAR_LDS_FLOATS] = (float)threadIdx.x;
    for (uint32_t e = 1; e <= episodes; ++e) {
        if (!grid_barrier<KIND>(w, e)) {
            if (threadIdx.x == 0) __hip_atomic_fetch_add(w + 9 * BAR_PAD + 16, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
    __syncthreads();
    if (pad[(threadIdx.x * 89 + 5) % BAR_LDS_FLOATS] == -1.0f) w[9 * BAR_PAD + 17] = 1; /* keeps the pad */
}

__global__ __launch_bounds__(256) void k_bar_clear(uint32_t *w, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) w[i] = 0;
}

}  // namespace

hipError_t launch_grid_barrier(uint32_t *words, uint32_t wgs, uint32_t episodes, uint32_t kind, hipStream_t s) {
    hipLaunchKernelGGL(k_bar_clear, dim3(1), dim3(256), 0, s, words, GRID_BARRIER_WORDS);
    if (kind == 0) hipLaunchKernelGGL(k_grid_barrier<0>, dim3(wgs), dim3(256), 0, s, words, episodes);
    else if (kind == 1) hipLaunchKernelGGL(k_grid_barrier<1>, dim3(wgs), dim3(256), 0, s, words, episodes);
    else hipLaunchKernelGGL(k_grid_barrier<2>, dim3(wgs), dim3(256), 0, s, words, episodes);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void *p, size_t bytes, uint32_t wgs, uint32_t threads, bool nt, uint32_t *sink,
                              hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (!n16) return hipSuccess;
    if (nt) hipLaunchKernelGGL(k_stream_read<true>, dim3(wgs), dim3(threads), 0, s, (const u4a *)p, n16, sink);
    else hipLaunchKernelGGL(k_stream_read<false>, dim3(wgs), dim3(threads), 0, s, (const u4a *)p, n16, sink);
    return hipGetLastError();
}

hipError_t launch_stream_copy(void *dst, const void *src, size_t bytes, uint32_t wgs, uint32_t threads, bool nt,
                              hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (!n16) return hipSuccess;
    if (nt) hipLaunchKernelGGL(k_stream_copy<true>, dim3(wgs), dim3(threads), 0, s, (const u4a *)src, (u4a *)dst, n16);
    else hipLaunchKernelGGL(k_stream_copy<false>, dim3(wgs), dim3(threads), 0, s, (const u4a *)src, (u4a *)dst, n16);
    return hipGetLastError();
}

}  // namespace smq
