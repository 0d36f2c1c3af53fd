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
    // First-index signed maximum of |x| (zeros and NaN never enter): the
    // largest magnitude over the wave as bits (non-negative floats order as
    // their bits), then the first lane holding it (ballot) and its first
    // element there; the sign is that element's.
    uint32_t b[4], amax_bits = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float av = fabsf(xs[e]);
        b[e] = av > 0.0f ? __float_as_uint(av) : 0u;
        amax_bits = max(amax_bits, b[e]);
    }
    amax_bits = row16_max_u32(amax_bits);
    amax_bits = max(amax_bits, (uint32_t)__shfl_xor((int)amax_bits, 16, 64));
    amax_bits = max(amax_bits, (uint32_t)__shfl_xor((int)amax_bits, 32, 64));
    bool hit = false, neg = false;
#pragma unroll
    for (int e = 3; e >= 0; --e) {  // the first element of this lane wins
        const bool h = amax_bits != 0u && b[e] == amax_bits;
        neg = h ? xs[e] < 0.0f : neg;
        hit = hit || h;
    }
    const unsigned long long hits = __ballot(hit);
    const int first = hits != 0ull ? __ffsll((long long)hits) - 1 : 0;
    const bool negative = __shfl((int)neg, first, 64) != 0;
    (void)lane;
    Q8KLane r;
    r.zero = amax_bits == 0u;
    r.word = 0u;
    r.sum4 = 0;
    r.d = 0.0f;
    r.q[0] = r.q[1] = r.q[2] = r.q[3] = 0;
    if (r.zero) return r;  // wavefront-uniform
    const float amax = __uint_as_float(amax_bits);
    const float maxv = negative ? -amax : amax;
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
