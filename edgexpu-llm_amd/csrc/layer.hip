// Elementwise layer ops around the projections, on device-resident
// activations: RMSNorm (src/cpu_kernel.c:220-242), SiLU (:244-252), the
// product and sum of two vectors (:200-218), and SiLU of one vector times
// another in one pass (the reference's silu followed by mul,
// src/native.c:2577-2578).  Arithmetic follows the reference op for op:
//
//   rmsnorm: squares summed in double, mean = (float)(ss / n),
//            scale = 1.0f / sqrtf(mean + eps), out = x * scale, out *= w;
//   silu:    out = x / (1.0f + e), e = expf(-x).
//
// Differences that can remain, stated where they arise: the double sum of
// squares runs as a tree instead of in index order, so (float)(ss / n) can
// differ only where the float rounding of the mean falls within the double
// sum's error (about n * 2^-53 relative); e is the device expf (within
// about one ulp, the host libm's within 0.502), so silu can differ from the
// reference's by a few ulp (measured bound in the tests).
// Division and sqrtf are IEEE (correctly rounded); no contraction
// (-ffp-contract=off).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace exq {

// One workgroup of 256 threads per row of n elements.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ out, int n, float eps) {
    __shared__ double part[4];
    const size_t row = blockIdx.x;
    const float *xr = x + row * (size_t)n;
    float *orow = out + row * (size_t)n;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = (double)xr[i];
        s += v * v;  // a float square is exact in double
    }
    s = wave_sum_f64(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = rms_scale(ss, n, eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i] * scale;
        orow[i] = v * w[i];
    }
}

// kind 0: silu(a); 1: a * b; 2: a + b; 3: silu(a) * b.
__global__ __launch_bounds__(256) void elementwise_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                          float *__restrict__ out, long long n, int kind) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float va = a[i];
    float r;
    if (kind == 0) r = silu_f32(va);
    else if (kind == 1) r = va * b[i];
    else if (kind == 2) r = va + b[i];
    else r = silu_f32(va) * b[i];
    out[i] = r;
}

}  // namespace exq

using namespace exq;

hipError_t launch_rmsnorm(const float *x, const float *w, float *out, int m, int n, float eps, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)m), dim3(256), 0, st, x, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_elementwise(const float *a, const float *b, float *out, long long n, int kind, hipStream_t st) {
    const long long grid = (n + 255) / 256;
    hipLaunchKernelGGL(elementwise_kernel, dim3((unsigned)grid), dim3(256), 0, st, a, b, out, n, kind);
    return hipGetLastError();
}
