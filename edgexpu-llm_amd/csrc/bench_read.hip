// Read ceiling for the decode benchmark: a plain streaming read of a device
// buffer (one 16-byte load per lane per step, grid-stride, an xor per lane
// so the loads stay live, one word stored per lane).  bench.py times it in
// the same HIP-graph harness as the decode GEMV, over the same byte counts,
// so that the GEMV launches can be set against what a launch that only
// reads the weights takes.  Built into its own library
// (lib/libexq_bench_read.so); the product library does not contain it.

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

}  // namespace

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
