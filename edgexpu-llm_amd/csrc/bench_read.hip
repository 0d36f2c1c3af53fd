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
//    source word, one 16-byte load per two 16-byte stores, as Q8_0's ratio).

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

}  // namespace

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
