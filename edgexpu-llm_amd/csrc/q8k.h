// Q8_K quantization of one 256-element block by one wavefront (lane l owns
// elements 4l..4l+3): edgexpu_gguf_quantize_q8_k, src/gguf_dot_q8.c:360-412.
//   maxv   = signed value of the first element with the largest |x| (strict '>'
//            from amax = 0, so zeros and NaN never win)
//   iscale = -127 / maxv, q = clamp(lrintf(iscale * x), -127, 127)
//   bsums  = int16 sums of 16 consecutive q, d = 1 / iscale
//   an all-zero block (maxv == 0) is stored as zeros.
// Shared by the Q8_K block writer (quantize.hip) and the prefill GEMM's
// operand packer (gemm.hip), so both produce the same codes bit for bit.
#pragma once

#include "common.h"

namespace exq {

struct Q8KLane {
    uint32_t word;  // the lane's 4 codes, element 4l+e in byte e
    int q[4];       // the same codes as integers
    int sum4;       // sum of the lane's 4 codes
    float d;        // block scale (0 for an all-zero block)
    bool zero;      // all-zero block
};

__device__ __forceinline__ Q8KLane q8k_quantize_lane(const float4 v, int lane) {
    const float xs[4] = {v.x, v.y, v.z, v.w};
    // First-index signed maximum of |x|: one 64-bit max over keys
    // (|x| bits << 32) | (~index << 1) | sign -- equal magnitudes -> lowest
    // index wins; zeros and NaN never enter.
    unsigned long long key = 0ull;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float av = fabsf(xs[e]);
        const uint32_t idx = (uint32_t)(lane * 4 + e);
        unsigned long long k = ((unsigned long long)__float_as_uint(av) << 32) | (((~idx) & 0x7fffffffu) << 1) |
                               (xs[e] < 0.0f ? 1u : 0u);
        k = av > 0.0f ? k : 0ull;
        key = k > key ? k : key;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(key, off, 64);
        key = o > key ? o : key;
    }
    Q8KLane r;
    r.zero = key == 0ull;
    r.word = 0u;
    r.sum4 = 0;
    r.d = 0.0f;
    r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
    if (r.zero) return r;  // wavefront-uniform
    const float amax = __uint_as_float((uint32_t)(key >> 32));
    const float maxv = (key & 1ull) ? -amax : amax;
    const float iscale = -127.0f / maxv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float p = iscale * xs[e];
        // lrintf: a NaN or infinite product gives LONG_MIN, whose low 32 bits are 0.
        int q = fabsf(p) < 2147483648.0f ? (int)rintf(p) : 0;
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        r.q[e] = q;
        r.sum4 += q;
        r.word |= (uint32_t)(q & 0xff) << (8 * e);
    }
    r.d = 1.0f / iscale;
    return r;
}

}  // namespace exq
