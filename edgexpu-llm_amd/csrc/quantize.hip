// Activation quantizers for the integer block dots.
//
//  * Q8_0 (32 elements): the x86 AVX2 variant of edgexpu_gguf_quantize_q8_0,
//    src/gguf_dot_q8.c:276-324 -- amax over |x|, d = amax/127 stored as fp16
//    (round-to-nearest-even), id = 127/amax, q = saturate8(round-half-even(x*id))
//    where a NaN / out-of-range product converts to the integer-indefinite
//    value and therefore saturates to -128.
//  * Q8_K (256 elements): edgexpu_gguf_quantize_q8_k, src/gguf_dot_q8.c:360-412
//    -- signed value of the first element with the largest |x| (strict '>'),
//    iscale = -127/maxv, q = clamp(lrintf(iscale*x), -127, 127), 16-element
//    int16 sums, d = 1/iscale; an all-zero block is stored as zeros.
//
// Both write the reference's own block bytes (34 B per 32 / 292 B per 256), so
// the drop-in quantize entry points return byte-identical buffers and the
// GEMV kernels read the same bytes the reference's integer dots consume.
#include "common.h"
#include "q8k.h"

namespace exq {

// One 32-element block per 8 lanes; each lane owns 4 consecutive elements.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(
    const float *__restrict__ x, int m, int K, int ldx, uint8_t *__restrict__ packed) {
    const int nb = K / kQK8_0;
    const long long total = (long long)m * nb;
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long blk = gid >> 3;
    const int part = (int)(gid & 7);
    if (blk >= total) return;  // the 8 lanes of a block exit together
    const int tok = (int)(blk / nb);
    const int b = (int)(blk % nb);
    const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)tok * ldx + (size_t)b * kQK8_0 + part * 4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const uint32_t dh = f32_to_f16_rne(d);
    const float xs[4] = {v.x, v.y, v.z, v.w};
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float r = rintf(xs[e] * id);
        int q = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT32_MIN;
        q = q < -128 ? -128 : (q > 127 ? 127 : q);
        word |= (uint32_t)(q & 0xff) << (8 * e);
    }
    uint8_t *blkp = packed + ((size_t)tok * nb + b) * kBytesQ8_0;
    uint16_t *w16 = reinterpret_cast<uint16_t *>(blkp + 2 + part * 4);  // 2-byte aligned
    w16[0] = (uint16_t)(word & 0xffffu);
    w16[1] = (uint16_t)(word >> 16);
    if (part == 0) *reinterpret_cast<uint16_t *>(blkp) = (uint16_t)dh;
}

// One 256-element block per wavefront; lane l owns elements 4l..4l+3.
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(
    const float *__restrict__ x, int m, int K, int ldx, uint8_t *__restrict__ packed) {
    const int nb = K / kQKK;
    const int lane = threadIdx.x & 63;
    const long long blk = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (blk >= (long long)m * nb) return;  // whole wavefront exits together
    const int tok = (int)(blk / nb);
    const int b = (int)(blk % nb);
    const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)tok * ldx + (size_t)b * kQKK + lane * 4);
    const Q8KLane r = q8k_quantize_lane(v, lane);
    uint8_t *blkp = packed + ((size_t)tok * nb + b) * kBytesQ8_K;  // 4-byte aligned
    if (r.zero) {
        reinterpret_cast<uint32_t *>(blkp + 4)[lane] = 0u;
        if (lane < 8) reinterpret_cast<uint32_t *>(blkp + 260)[lane] = 0u;
        if (lane == 0) *reinterpret_cast<uint32_t *>(blkp) = 0u;
        return;
    }
    int sum = r.sum4;
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    reinterpret_cast<uint32_t *>(blkp + 4)[lane] = r.word;
    if ((lane & 3) == 0) reinterpret_cast<int16_t *>(blkp + 260)[lane >> 2] = (int16_t)sum;
    if (lane == 0) *reinterpret_cast<float *>(blkp) = r.d;
}

}  // namespace exq

using namespace exq;

// Launch helpers (C++ linkage; used by the shim).
hipError_t launch_quantize_q8_0(const float *x, int m, int K, int ldx, uint8_t *packed, hipStream_t st) {
    const long long threads = (long long)m * (K / kQK8_0) * 8;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid), dim3(256), 0, st, x, m, K, ldx, packed);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_k(const float *x, int m, int K, int ldx, uint8_t *packed, hipStream_t st) {
    const long long threads = (long long)m * (K / kQKK) * 64;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(quantize_q8_k_kernel, dim3(grid), dim3(256), 0, st, x, m, K, ldx, packed);
    return hipGetLastError();
}

