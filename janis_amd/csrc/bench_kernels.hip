// Measurement kernels for bench.py (libjanis_bench.so; not part of the
// backend's C ABI): a plain streaming read and a copy of device memory. They do
// nothing but move bytes, so their time for a given byte count is the floor a
// decode product reading that many bytes in one launch can reach, and the copy
// gives the device's measured bandwidth beside the 8 TB/s specification. An
// empty kernel gives the fixed cost of one node of a HIP graph, and the read
// with the default cache policy (the decode products' weight loads are
// non-temporal) shows whether the memory-side cache serves a re-read. The
// chained read is the alternative to one launch per stage: every stage of a
// token's reads in one persistent launch, a grid-wide barrier between stages.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every block reads UNROLL 16-byte chunks per lane per step, all issued before
// any is used (the way the decode tiles issue a pass's weight loads), and
// strides over the buffer by the grid. The loaded words are folded into one
// value that is stored only if it equals a constant, so the loads stay.
template <int UNROLL, bool NT = true>
__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                   uint32_t* __restrict__ sink) {
    u32x4 acc = {0u, 0u, 0u, 0u};
    const int64_t step = (int64_t)gridDim.x * 256 * UNROLL;
    for (int64_t base = (int64_t)blockIdx.x * 256 * UNROLL + threadIdx.x; base < n16; base += step) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int64_t i = base + (int64_t)u * 256;
            if constexpr (NT)
                v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
            else
                v[u] = i < n16 ? src[i] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < UNROLL; u++) acc ^= v[u];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = acc.x;
}

template <int UNROLL>
__global__ __launch_bounds__(256) void copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                   int64_t n16) {
    const int64_t step = (int64_t)gridDim.x * 256 * UNROLL;
    for (int64_t base = (int64_t)blockIdx.x * 256 * UNROLL + threadIdx.x; base < n16; base += step) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int64_t i = base + (int64_t)u * 256;
            if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int64_t i = base + (int64_t)u * 256;
            if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
        }
    }
}

__global__ void empty_kernel() {}

// `rounds` grid-wide barriers in one launch: in each round every block adds 1
// to a counter (agent scope) and polls it until the round's blocks have all
// arrived -- the synchronisation a persistent kernel running dependent stages
// pays per stage. ORDERED: release on the add and acquire on the polls (what
// makes one stage's global writes visible to the next stage on other XCDs);
// otherwise relaxed (the atomic round trips alone). The grid must be resident
// at once (one 64-thread block per CU); the polls are bounded, and a block
// that gives up sets *failed and stops.
template <bool ORDERED>
__global__ __launch_bounds__(64) void barrier_kernel(unsigned* counter, int rounds, unsigned spin, unsigned* failed) {
    __shared__ int stop;
    if (threadIdx.x == 0) stop = 0;
    __syncthreads();
    for (int r = 1; r <= rounds && !stop; r++) {
        if (threadIdx.x == 0) {
            if constexpr (ORDERED)
                __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else
                __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned target = (unsigned)r * gridDim.x;
            unsigned n = 0;
            for (;;) {
                const unsigned v = ORDERED ? __hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT)
                                           : __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (v >= target) break;
                if (++n > spin) {
                    __hip_atomic_fetch_or(failed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    stop = 1;
                    break;
                }
            }
        }
        __syncthreads();
    }
}

// One stage of a chained read: a range of 16-byte units.
struct ChainStage {
    const u32x4* p;
    int64_t n16;
};

// The stages in order in one launch of one T-thread block per CU -- what a
// persistent kernel chaining dependent products would pay per stage in place
// of a graph node. Block b reads units [n16 b / nb, n16 (b+1) / nb) of every
// stage (UNROLL non-temporal loads per lane per step), then stores the stage
// number + 1 into its own arrival flag (one flag per 128-byte line: flags
// sharing a line made the barrier several times slower) and wave 0 polls every
// block's flag until all have arrived; before waiting, every lane requests the
// first step of its part of the next stage, which does not depend on the
// barrier (as a product's weights do not depend on its input). The grid must
// be resident at once; the polls are bounded, and a block that gives up sets
// *failed and stops.
template <int T, int UNROLL>
__global__ __launch_bounds__(T) void chain_read_kernel(const ChainStage* __restrict__ st, int nst,
                                                       unsigned* flags, unsigned spin, unsigned* failed,
                                                       uint32_t* __restrict__ sink) {
    constexpr int PAD = 32;  // words between flags
    __shared__ int stop;
    const int tid = threadIdx.x;
    const unsigned nb = gridDim.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    u32x4 v[UNROLL];
    bool have = false;  // v holds the first step of the current stage
    for (int s = 0; s < nst; s++) {
        const u32x4* p = st[s].p;
        const int64_t n16 = st[s].n16;
        const int64_t hi = n16 * (blockIdx.x + 1) / nb;
        int64_t b0 = n16 * blockIdx.x / nb + tid;
        if (have) {
#pragma unroll
            for (int u = 0; u < UNROLL; u++) acc ^= v[u];
            b0 += (int64_t)T * UNROLL;
            have = false;
        }
        for (; b0 < hi; b0 += (int64_t)T * UNROLL) {
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const int64_t i = b0 + (int64_t)u * T;
                v[u] = i < hi ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < UNROLL; u++) acc ^= v[u];
        }
        if (s + 1 == nst) break;
        __syncthreads();
        if (tid == 0) {
            stop = 0;
            __hip_atomic_store(flags + blockIdx.x * PAD, (unsigned)(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        {
            const u32x4* q = st[s + 1].p;
            const int64_t m16 = st[s + 1].n16;
            const int64_t c0 = m16 * blockIdx.x / nb + tid, h2 = m16 * (blockIdx.x + 1) / nb;
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const int64_t i = c0 + (int64_t)u * T;
                v[u] = i < h2 ? __builtin_nontemporal_load(q + i) : u32x4{0u, 0u, 0u, 0u};
            }
            have = true;
        }
        if (tid < 64) {
            const unsigned target = (unsigned)(s + 1);
            bool seen = false;
            for (unsigned n = 0; n < spin; n++) {
                bool ok = true;
                for (unsigned j = tid; j < nb; j += 64)
                    ok &= __hip_atomic_load(flags + j * PAD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
                if (__all(ok)) {
                    seen = true;
                    break;
                }
            }
            if (!seen && tid == 0) {
                __hip_atomic_fetch_or(failed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                stop = 1;
            }
        }
        __syncthreads();
        if (stop) break;
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = acc.x;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned) at src with `blocks`
// blocks of 256 threads and `unroll` (4, 8 or 16) loads per lane in flight, on
// `stream`. Returns 0, or the HIP error code.
__attribute__((visibility("default"))) int jhb_read(const void* src, int64_t bytes, void* sink, int blocks,
                                                    int unroll, void* stream) {
    if (bytes <= 0 || (bytes & 15) || ((uintptr_t)src & 15) || blocks <= 0) return (int)hipErrorInvalidValue;
    const int64_t n16 = bytes / 16;
    auto st = static_cast<hipStream_t>(stream);
    auto s = static_cast<const u32x4*>(src);
    auto k = static_cast<uint32_t*>(sink);
    if (unroll == 4) hipLaunchKernelGGL(read_kernel<4>, dim3(blocks), dim3(256), 0, st, s, n16, k);
    else if (unroll == 8) hipLaunchKernelGGL(read_kernel<8>, dim3(blocks), dim3(256), 0, st, s, n16, k);
    else if (unroll == 16) hipLaunchKernelGGL(read_kernel<16>, dim3(blocks), dim3(256), 0, st, s, n16, k);
    else return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

// jhb_read with the default cache policy (8 loads per lane in flight).
__attribute__((visibility("default"))) int jhb_read_cached(const void* src, int64_t bytes, void* sink, int blocks,
                                                           void* stream) {
    if (bytes <= 0 || (bytes & 15) || ((uintptr_t)src & 15) || blocks <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((read_kernel<8, false>), dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(src), bytes / 16, static_cast<uint32_t*>(sink));
    return (int)hipGetLastError();
}

// One launch of an empty kernel with `blocks` blocks of 64 threads.
__attribute__((visibility("default"))) int jhb_empty(int blocks, void* stream) {
    if (blocks <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(64), 0, static_cast<hipStream_t>(stream));
    return (int)hipGetLastError();
}

// One launch of `blocks` 64-thread blocks passing `rounds` grid-wide barriers
// on *counter (which must be 0; it ends at rounds * blocks), ordered
// (release/acquire) or relaxed; *failed is set if a block gave up waiting
// (after `spin` polls). blocks must not exceed the CU count.
__attribute__((visibility("default"))) int jhb_barriers(void* counter, int blocks, int rounds, int ordered,
                                                        unsigned spin, void* failed, void* stream) {
    if (!counter || !failed || blocks <= 0 || rounds < 0) return (int)hipErrorInvalidValue;
    auto st = static_cast<hipStream_t>(stream);
    auto c = static_cast<unsigned*>(counter);
    auto f = static_cast<unsigned*>(failed);
    if (ordered) hipLaunchKernelGGL(barrier_kernel<true>, dim3(blocks), dim3(64), 0, st, c, rounds, spin, f);
    else hipLaunchKernelGGL(barrier_kernel<false>, dim3(blocks), dim3(64), 0, st, c, rounds, spin, f);
    return (int)hipGetLastError();
}

// Copies `bytes` (a multiple of 16, both pointers 16-byte aligned) src -> dst.
__attribute__((visibility("default"))) int jhb_copy(void* dst, const void* src, int64_t bytes, int blocks,
                                                    void* stream) {
    if (bytes <= 0 || (bytes & 15) || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || blocks <= 0)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_kernel<4>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<u32x4*>(dst), static_cast<const u32x4*>(src), bytes / 16);
    return (int)hipGetLastError();
}

// The chained read: `nst` stages {pointer (16-byte aligned), units of 16
// bytes} at `stages` (device memory), `blocks` blocks (one per CU) of
// `threads` (512 or 1024) threads, 8 loads per lane per step; `flags` =
// blocks x 32 words, zero before the launch. Returns 0, or the HIP error code.
__attribute__((visibility("default"))) int jhb_chain_read(const void* stages, int nst, void* flags, unsigned spin,
                                                          void* failed, void* sink, int blocks, int threads,
                                                          void* stream) {
    if (nst <= 0 || blocks <= 0) return (int)hipErrorInvalidValue;
    auto st = static_cast<hipStream_t>(stream);
    auto S = static_cast<const ChainStage*>(stages);
    auto f = static_cast<unsigned*>(flags);
    auto fl = static_cast<unsigned*>(failed);
    auto k = static_cast<uint32_t*>(sink);
    if (threads == 512)
        hipLaunchKernelGGL((chain_read_kernel<512, 8>), dim3(blocks), dim3(512), 0, st, S, nst, f, spin, fl, k);
    else if (threads == 1024)
        hipLaunchKernelGGL((chain_read_kernel<1024, 8>), dim3(blocks), dim3(1024), 0, st, S, nst, f, spin, fl, k);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

}  // extern "C"
