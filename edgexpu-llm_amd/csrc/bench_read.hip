// Ceilings for the benchmark, built into their own library
// (lib/libexq_bench_read.so; the product library does not contain them):
//  * read: a plain streaming read of a device buffer (one 16-byte load per
//    lane per step, grid-stride, an xor per lane so the loads stay live, one
//    word stored per lane).  bench.py times it in the same HIP-graph harness
//    as the decode GEMV, over the same byte counts, so that the GEMV launches
//    can be set against what a launch that only reads the weights takes;
//  * write and read+write: the bulk dequant's bytes without its arithmetic --
//    16-byte stores of a constant over the output, and a pass that reads the
//    source (16 bytes per lane) and writes the output (8 floats per lane per
//    source word, one 16-byte load per two 16-byte stores, as Q8_0's ratio);
//  * synchronisation costs: an empty launch (a dependent kernel boundary in a
//    graph) against a grid barrier inside one launch, the cost a persistent
//    multi-phase kernel would pay instead of each boundary.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_kernel(const v4u *__restrict__ p, long long n16,
                                                   unsigned *__restrict__ out) {
    v4u acc = {0u, 0u, 0u, 0u};
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        acc ^= __builtin_nontemporal_load(p + i);
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

__global__ __launch_bounds__(256) void write_kernel(v4u *__restrict__ p, long long n16, unsigned v) {
    const long long stride = (long long)gridDim.x * 256;
    const v4u val = {v, v, v, v};
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) p[i] = val;
}

// dst gets n16 16-byte words, lane-contiguous; word o takes source word
// o / ratio, so each source word is read by `ratio` neighbouring lanes (one
// HBM read, the rest L1 / L2 hits).
__global__ __launch_bounds__(256) void read_write_kernel(const v4u *__restrict__ src, long long s16,
                                                         v4u *__restrict__ dst, long long n16, int ratio) {
    const long long stride = (long long)gridDim.x * 256;
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < n16; o += stride) {
        const long long i = min(o / ratio, s16 - 1);
        dst[o] = src[i] + (unsigned)(o - i * ratio);
    }
}

__global__ void empty_kernel() {}

// Barrier words: arrivals, finished workgroups, error flag (separate lines);
// per-XCD arrival counters and release words (one line each) and a phase
// buffer of 16 words per workgroup for the hierarchical barriers.
struct BarWords {
    unsigned arrive, pad0[31];
    unsigned done, pad1[31];
    int err, pad2[31];
    unsigned xcd[8][32];
    unsigned go[8][32];
    unsigned data[256 * 16];
    unsigned sink[256];
};

// `rounds` grid barriers.  Workgroups of XCD 0 only (b % 8 == 0: workgroups
// are dispatched to the 8 XCDs round robin) when xcd0, else all.  mode 0:
// release add / acquire fence at agent scope (every store before the barrier
// visible to every load after it, on any XCD: an L2 writeback and an L2
// invalidate per workgroup); mode 1: relaxed agent-scope add and polls only
// (the synchronisation without the data visibility).  Every wait is bounded
// (spin polls, then err = 1 and on); the last workgroup resets the words.
template <int MODE>
__global__ void barrier_kernel(BarWords *w, int rounds, int xcd0, int spin) {
    if (xcd0 && blockIdx.x % 8 != 0) return;
    const unsigned n = xcd0 ? gridDim.x / 8 : gridDim.x;
    for (int r = 1; r <= rounds; ++r) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            if (MODE == 0) __hip_atomic_fetch_add(&w->arrive, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else __hip_atomic_fetch_add(&w->arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int k = 0;
            while (__hip_atomic_load(&w->arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)r * n) {
                if (++k >= spin) {
                    __hip_atomic_store(&w->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (MODE == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(&w->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == n - 1u) {
            __hip_atomic_store(&w->arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&w->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// `rounds` hierarchical grid barriers over all workgroups (gridDim.x a
// multiple of 8, one per CU): each workgroup arrives on its XCD's counter
// (workgroup b runs on XCD b % 8), the last arrival of an XCD on the global
// counter, and the last of those releases every XCD through its own word, so
// at most gridDim.x / 8 workgroups poll one word.  Relaxed agent-scope
// atomics only.  MODE 3 also exchanges data the way a persistent kernel's
// phases would without fences: before arriving, threads 0-15 store the
// workgroup's 16 words with agent-scope atomic stores (written through to
// the device-coherent level, no L2 writeback needed); after the barrier every
// thread reads 4 of the 256 x 16 words with agent-scope atomic loads (no L2
// invalidate needed) and folds them into a word it stores at the end.  Every
// wait is bounded as in barrier_kernel; the last workgroup resets the words.
template <int MODE>
__global__ __launch_bounds__(1024) void xcd_barrier_kernel(BarWords *w, int rounds, int spin) {
    const unsigned nx = gridDim.x / 8u;
    const unsigned xc = blockIdx.x % 8u;
    unsigned acc = 0u;
    for (int r = 1; r <= rounds; ++r) {
        if (MODE == 3 && threadIdx.x < 16)
            __hip_atomic_store(&w->data[blockIdx.x * 16 + threadIdx.x], (unsigned)r ^ blockIdx.x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old = __hip_atomic_fetch_add(&w->xcd[xc][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == (unsigned)r * nx - 1u) {
                const unsigned g = __hip_atomic_fetch_add(&w->arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (g == (unsigned)r * 8u - 1u)
                    for (int k = 0; k < 8; ++k)
                        __hip_atomic_store(&w->go[k][0], (unsigned)r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            int k = 0;
            while (__hip_atomic_load(&w->go[xc][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)r) {
                if (++k >= spin) {
                    __hip_atomic_store(&w->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (MODE == 3) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc ^= __hip_atomic_load(&w->data[(threadIdx.x * 4 + j) % (gridDim.x * 16)], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (MODE == 3 && threadIdx.x == 0) w->sink[blockIdx.x] = acc;
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(&w->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1u) {
            __hip_atomic_store(&w->arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int k = 0; k < 8; ++k) {
                __hip_atomic_store(&w->xcd[k][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&w->go[k][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(&w->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace

// An empty kernel of grid x threads.  0 on success.
extern "C" int exq_bench_empty(int grid, int threads, void *stream) {
    if (grid < 1 || grid > 65536 || threads < 64 || threads > 1024) return 1;
    hipLaunchKernelGGL(empty_kernel, dim3((unsigned)grid), dim3((unsigned)threads), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Bytes of the barrier words (zeroed by the caller once).
extern "C" long long exq_bench_barrier_words(void) { return (long long)sizeof(BarWords); }

// One launch of `rounds` grid barriers over grid workgroups of `threads`
// (one per CU at 1024 threads: grid <= the CU count keeps every workgroup
// resident, which the barrier needs).  0 on success; the error flag sits at
// byte 256 of the words.
// mode 2 / 3: the hierarchical barrier (xcd_barrier_kernel, all workgroups,
// grid a multiple of 8, xcd0 ignored), 3 with its data exchange.
extern "C" int exq_bench_barrier(void *words, int grid, int threads, int rounds, int mode, int xcd0, void *stream) {
    if (words == nullptr || grid < 8 || grid > 256 || threads < 64 || threads > 1024 || rounds < 1 || rounds > 1000 ||
        mode < 0 || mode > 3 || (mode >= 2 && grid % 8 != 0))
        return 1;
    constexpr int kSpin = 1 << 18;
    if (mode == 2 || mode == 3) {
        if (mode == 2)
            hipLaunchKernelGGL(xcd_barrier_kernel<2>, dim3((unsigned)grid), dim3((unsigned)threads), 0,
                               (hipStream_t)stream, static_cast<BarWords *>(words), rounds, kSpin);
        else
            hipLaunchKernelGGL(xcd_barrier_kernel<3>, dim3((unsigned)grid), dim3((unsigned)threads), 0,
                               (hipStream_t)stream, static_cast<BarWords *>(words), rounds, kSpin);
        return hipGetLastError() == hipSuccess ? 0 : 2;
    }
    if (mode == 0)
        hipLaunchKernelGGL(barrier_kernel<0>, dim3((unsigned)grid), dim3((unsigned)threads), 0, (hipStream_t)stream,
                           static_cast<BarWords *>(words), rounds, xcd0, kSpin);
    else
        hipLaunchKernelGGL(barrier_kernel<1>, dim3((unsigned)grid), dim3((unsigned)threads), 0, (hipStream_t)stream,
                           static_cast<BarWords *>(words), rounds, xcd0, kSpin);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Writes bytes (a multiple of 16, dst 16-byte aligned) with grid workgroups
// of 256 threads.  0 on success.
extern "C" int exq_bench_write(void *dst, long long bytes, int grid, void *stream) {
    if (dst == nullptr || bytes <= 0 || (bytes & 15) != 0 || ((uintptr_t)dst & 15) != 0 || grid < 1 || grid > 65536)
        return 1;
    hipLaunchKernelGGL(write_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, static_cast<v4u *>(dst),
                       bytes / 16, 0x3f800000u);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Reads src_bytes of src and writes dst_bytes of dst (both multiples of 16,
// 16-byte aligned, dst_bytes = ratio * src_bytes rounded to a multiple of 16
// at most), grid workgroups of 256 threads.  0 on success.
extern "C" int exq_bench_read_write(const void *src, long long src_bytes, void *dst, long long dst_bytes, int grid,
                                    void *stream) {
    if (src == nullptr || dst == nullptr || src_bytes <= 0 || dst_bytes <= 0 || ((src_bytes | dst_bytes) & 15) != 0 ||
        (((uintptr_t)src | (uintptr_t)dst) & 15) != 0 || grid < 1 || grid > 65536)
        return 1;
    const long long s16 = src_bytes / 16, n16 = dst_bytes / 16;
    const int ratio = (int)((n16 + s16 - 1) / s16);
    if (ratio < 1 || ratio > 16) return 1;
    hipLaunchKernelGGL(read_write_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const v4u *>(src), s16, static_cast<v4u *>(dst), n16, ratio);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Reads bytes (a multiple of 16, src 16-byte aligned) of src with grid
// workgroups of 256 threads; out holds grid * 256 words.  0 on success.
extern "C" int exq_bench_read(const void *src, long long bytes, unsigned *out, int grid, void *stream) {
    if (src == nullptr || out == nullptr || bytes <= 0 || (bytes & 15) != 0 || ((uintptr_t)src & 15) != 0 ||
        grid < 1 || grid > 65536)
        return 1;
    hipLaunchKernelGGL(read_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const v4u *>(src), bytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
