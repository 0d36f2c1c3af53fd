// Device-side helpers shared by the gfx950 kernels of the GGUF quantized-
// weight path: block layouts, fp16 codecs with the reference's rounding, and
// wavefront reductions.
//
// Block byte maps (little-endian), as laid out by the reference
// (src/gguf_quant.c:17-26,138-302; src/gguf_dot_q8.c:18-26,98-110):
//   Q8_0  34 B / 32 elem : fp16 d | int8 q[32]
//   Q4_0  18 B / 32 elem : fp16 d | qs[16] (element j low nibble, j+16 high; value c-8)
//   Q5_0  22 B / 32 elem : fp16 d | u32 qh (bit e = fifth bit of element e) | qs[16] (value c-16)
//   Q4_K 144 B / 256 elem: fp16 d | fp16 dmin | scales[12] (6-bit sc/m) | qs[128]
//   Q5_K 176 B / 256 elem: fp16 d | fp16 dmin | scales[12] | qh[32] | qs[128] (chunk j: bits 2j, 2j+1 of qh[l])
//   Q6_K 210 B / 256 elem: ql[128] | qh[64] | int8 sc[16] | fp16 d
//   Q8_K 292 B / 256 elem: f32 d | int8 q[256] | int16 bsums[16]
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

namespace exq {

// Launch-shape tuning knobs (EXQ_* names).  The library fixes every knob at
// its default at compile time; only a build with -DEXQ_TUNING_ENV (a
// launch-shape sweep, never the shipped library) reads the environment
// variable of the same name, once per process.
#ifdef EXQ_TUNING_ENV
inline int tuning_knob(const char *name, int dflt) {
    const char *e = getenv(name);
    return e != nullptr ? atoi(e) : dflt;
}
#else
constexpr int tuning_knob(const char *, int dflt) { return dflt; }
#endif

constexpr int kTypeF32 = 0;
constexpr int kTypeF16 = 1;
constexpr int kTypeQ4_0 = 2;
constexpr int kTypeQ5_0 = 6;
constexpr int kTypeQ8_0 = 8;
constexpr int kTypeQ4_K = 12;
constexpr int kTypeQ5_K = 13;
constexpr int kTypeQ6_K = 14;

constexpr int kQK8_0 = 32;
constexpr int kQKK = 256;
constexpr int kBytesQ8_0 = 34;
constexpr int kBytesQ4_0 = 18;
constexpr int kBytesQ5_0 = 22;
constexpr int kBytesQ4_K = 144;
constexpr int kBytesQ5_K = 176;
constexpr int kBytesQ6_K = 210;
constexpr int kBytesQ8_K = 292;

// Activation families of the reference's dispatcher (src/gguf_dot_q8.c:414-434):
// Q4_0 / Q5_0 / Q8_0 rows take Q8_0 activations, the K-quants Q8_K.
__host__ __device__ constexpr bool q8_0_family(int t) { return t == kTypeQ8_0 || t == kTypeQ4_0 || t == kTypeQ5_0; }
__host__ __device__ constexpr bool k_family(int t) { return t == kTypeQ4_K || t == kTypeQ5_K || t == kTypeQ6_K; }

// Loads that tolerate the 2-byte alignment of Q8_0 / Q6_K blocks: gfx950
// global memory runs in unaligned-access mode, so these become plain
// global_load_dword{,x2,x4} instructions.
template <typename T>
__device__ __forceinline__ T ldg_unaligned(const uint8_t *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return ldg_unaligned<uint4>(p); }
__device__ __forceinline__ uint2 ldg8(const uint8_t *p) { return ldg_unaligned<uint2>(p); }
__device__ __forceinline__ uint32_t ldg4(const uint8_t *p) { return ldg_unaligned<uint32_t>(p); }

// 16 / 8 bytes at an even address p from 4-byte-aligned loads: the words
// from p - (p & 3) and the 16-bit word ending the range, joined with
// v_alignbyte.  Measured on gfx950: wide loads at addresses 2 mod 4 (every
// other Q8_0 / Q6_K / Q4_0 / Q5_0 block) run several times slower than
// these.  Only bytes in [p - 2, p + 16) are read, and p - 2 only when p is
// 2 mod 4, so never before the 4-byte-aligned start of the buffer that holds
// p.  p must be even.  The aligned address is formed by subtracting from p,
// not through an integer, so the loads stay global ones.
__device__ __forceinline__ uint4 ldg16_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3];
    const uint32_t t = *reinterpret_cast<const uint16_t *>(p + 14);
    return make_uint4(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                      __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(t, w3, sh));
}
__device__ __forceinline__ uint2 ldg8_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t w0 = q[0], w1 = q[1];
    const uint32_t t = *reinterpret_cast<const uint16_t *>(p + 6);
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(t, w1, sh));
}

// IEEE half -> float; exact for every input including subnormals.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
    return (float)v;
}

// float -> IEEE half with round-to-nearest-even and gradual underflow, the
// behaviour of F16C _mm_cvtps_ph(_MM_FROUND_TO_NEAREST_INT) that the
// reference uses for the Q8_0 activation scale (src/gguf_dot_q8.c:33-35).
// Done in integer arithmetic so it does not depend on the shader's float
// mode register.
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u | ((a >> 13) & 0x3ffu);
    if (a >= 0x477ff000u) return sign | 0x7c00u;
    if (a >= 0x38800000u) {
        uint32_t r = a - 0x38000000u;
        r += 0x0fffu + ((r >> 13) & 1u);
        return sign | (r >> 13);
    }
    if (a < 0x33000000u) return sign;
    uint32_t e = a >> 23;
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t sh = 126u - e;
    uint32_t q = mant >> sh;
    uint32_t rem = mant & ((1u << sh) - 1u);
    uint32_t half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | q;
}

// Signed 8-bit 4-way dot product with accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 16-bit pair dot with accumulate: lo(a)*lo(b) + hi(a)*hi(b) + c, signed.
__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c) {
    typedef short short2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}

// All-reduces within each 16-lane DPP row (lanes 16r..16r+15), every lane
// active: two quad_perm exchanges (partner lane ^1, ^2) leave each quad with
// its result, then the half-row mirror (lane i <-> 7-i) pairs the two quads
// of each half-row and the row mirror (i <-> 15-i) the two halves.  Each step
// is one VALU instruction with a DPP operand, no LDS round trip.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
constexpr int kDppRor8 = 0x128;        // row_ror:8 (lane l of a 16-lane row gets lane l ^ 8)
__device__ __forceinline__ float row8_max(float v) {
    v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v))));
    return fmaxf(v, __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v))));
}
__device__ __forceinline__ float row16_max(float v) {
    v = row8_max(v);
    return fmaxf(v, __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v))));
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = max(v, dpp_u32<kDppXor1>(v));
    v = max(v, dpp_u32<kDppXor2>(v));
    v = max(v, dpp_u32<kDppHalfMirror>(v));
    return max(v, dpp_u32<kDppMirror>(v));
}
__device__ __forceinline__ uint32_t row16_min(uint32_t v) {
    v = min(v, dpp_u32<kDppXor1>(v));
    v = min(v, dpp_u32<kDppXor2>(v));
    v = min(v, dpp_u32<kDppHalfMirror>(v));
    return min(v, dpp_u32<kDppMirror>(v));
}

// SiLU as src/cpu_kernel.c:244-252 computes it, x / (1.0f + expf(-x)), with
// the device expf (within about one ulp; the host libm's is within 0.502),
// so the two silu values can differ by a few ulp.  (A double-precision exp
// rounded once is correctly rounded but costs registers the fused GEMV
// epilogue does not have.)
__device__ __forceinline__ float silu_f32(float v) {
    const float e = expf(-v);
    return v / (1.0f + e);
}

// RMSNorm scale from the double sum of squares of n elements, as
// src/cpu_kernel.c:232-235: mean rounded to float, then 1 / sqrtf(mean + eps)
// (IEEE sqrt and division).
__device__ __forceinline__ float rms_scale(double ss, int n, float eps) {
    const float mean = (float)(ss / (double)n);
    return 1.0f / sqrtf(mean + eps);
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// The partner value l ^ off of a level of group_reduce's plain butterfly:
// ^ 32 by bpermute, ^ 16 and ^ 4 by swizzle, inside 16-lane rows ^ 8 as the
// DPP rotation by 8 and ^ 2, ^ 1 as quad permutes.  Every level pairs l with
// l ^ off, as the transposing levels do, so a value's tree does not depend
// on how many values a lane reduces (V).
__device__ __forceinline__ float reduce_partner(float v, int off) {
    switch (off) {
        case 1: return __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
        case 2: return __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
        case 4: return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101f));
        case 8: return __uint_as_float(dpp_u32<kDppRor8>(__float_as_uint(v)));
        case 16: return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
        default: return shfl_xor_f(v, off);
    }
}

// Sum of a double over the 64 lanes of a wave (every lane gets the total):
// partners l ^ 32, ^ 16, ..., ^ 1 in that order, each double moved as its
// two words by reduce_partner (bpermute for ^ 32, swizzles and DPP below),
// so every lane adds the same pairs in the same order.
__device__ __forceinline__ double wave_sum_f64(double s) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t b = __builtin_bit_cast(uint64_t, s);
        const uint32_t lo = __float_as_uint(reduce_partner(__uint_as_float((uint32_t)b), off));
        const uint32_t hi = __float_as_uint(reduce_partner(__uint_as_float((uint32_t)(b >> 32)), off));
        s += __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
    }
    return s;
}

// Sum of V per-lane values over aligned groups of G lanes (G a power of two
// <= 64).  On return vals[0] in every lane holds the group total of value
// index vidx(lane), where the indices are distributed over the group's lanes
// by the bit pattern the halving steps leave behind: after the call, lane l
// owns value index ((l & (G-1)) / (G / min(V, G))) ... folded as computed by
// out_index().  V must be a power of two.
template <int V>
__device__ __forceinline__ void group_reduce(float (&vals)[V], int G, int lane) {
    int nv = V;
    int off = G >> 1;
    // Transposing halving steps: each exchange halves the number of live values.
#pragma unroll
    for (int step = V; step > 1; step >>= 1) {
        if (off == 0) break;
        const int half = step >> 1;
        const bool upper = (lane & off) != 0;
#pragma unroll
        for (int k = 0; k < half; ++k) {
            float send = upper ? vals[k] : vals[k + half];
            float keep = upper ? vals[k + half] : vals[k];
            vals[k] = keep + shfl_xor_f(send, off);
        }
        nv = half;
        off >>= 1;
    }
    // Plain butterfly for the remaining group bits.
    for (; off > 0; off >>= 1) {
        vals[0] += reduce_partner(vals[0], off);
    }
    (void)nv;
}

// Value index lane `lane` owns after group_reduce<V>(…, G, …).
__device__ __forceinline__ int group_reduce_index(int V, int G, int lane) {
    int idx = 0;
    int off = G >> 1;
    for (int step = V; step > 1 && off > 0; step >>= 1) {
        const int half = step >> 1;
        if (lane & off) idx += half;
        off >>= 1;
    }
    return idx;
}

// Number of distinct values that survive group_reduce<V> with group size G.
__host__ __device__ constexpr int group_reduce_live(int V, int G) {
    int nv = V;
    int off = G >> 1;
    while (nv > 1 && off > 0) {
        nv >>= 1;
        off >>= 1;
    }
    return nv;
}

}  // namespace exq
