// Bulk dequantization of GGUF blocks to f32 (edgexpu_gguf_dequantize,
// src/gguf_quant.c:355-411).  Each thread writes 8 consecutive outputs with
// two 16-byte stores, so a wavefront writes 2 KiB of contiguous f32.
//
// Bit-exactness: the reference x86 build is gcc -std=c11, which does not
// contract a*b-c into an FMA.  This file is compiled with -ffp-contract=off
// and keeps the reference's operation order:
//   Q8_0  y = d * q                                  (src/gguf_quant.c:152)
//   Q4_K  y = (d*sc) * q - (dmin*m)                  (src/gguf_quant.c:251-260)
//   Q6_K  y = (d*sc) * (q-32)                        (src/gguf_quant.c:291-294)
//   Q4_0  y = ((float)c - 8) * d                     (src/gguf_quant.c:205-206)
//   Q5_0  y = (float)(c - 16) * d                    (src/gguf_quant.c:176-177)
//   Q5_K  y = (d*sc) * c - (dmin*m)                  (src/gguf_quant.c:339-343)
//   F16   y = (float)h                               (src/gguf_quant.c:183-191)
//   F32   y = x, a copy                              (src/gguf_quant.c:376-378)
#include "common.h"

namespace exq {

__device__ __forceinline__ void store8(float *dst, const float (&y)[8]) {
    float4 *p = reinterpret_cast<float4 *>(dst);
    p[0] = make_float4(y[0], y[1], y[2], y[3]);
    p[1] = make_float4(y[4], y[5], y[6], y[7]);
}

// 4 threads per 34-byte block.
__device__ __forceinline__ void dq_q8_0(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    const long long b = t >> 2;
    const int p = (int)(t & 3);
    const uint8_t *blk = src + b * kBytesQ8_0;
    const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
    const uint2 q = ldg8(blk + 2 + 8 * p);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = e < 4 ? q.x : q.y;
        const int8_t c = (int8_t)((w >> (8 * (e & 3))) & 0xff);
        y[e] = d * (float)c;
    }
    store8(dst + b * kQK8_0 + 8 * p, y);
}

__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_threads) return;
    dq_q8_0(src, t, dst);
}

// Output stores of the bulk kernels: the f32 output (up to 8x the source)
// is not read again by the kernel, so it streams past the caches.
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store8_nt(float *dst, const float (&y)[8]) {
    v4f *p = reinterpret_cast<v4f *>(dst);
    __builtin_nontemporal_store(v4f{y[0], y[1], y[2], y[3]}, p);
    __builtin_nontemporal_store(v4f{y[4], y[5], y[6], y[7]}, p + 1);
}

// Units per thread of the Q4_K and Q6_K bulk kernels: both units' loads
// are issued before either's arithmetic.
constexpr int kDqUnits = 2;

// 32 threads per 144-byte super-block; thread p covers elements 8p..8p+7,
// which lie in sub-block s = p/4 (64-chunk j = s/2, nibble half s&1).
struct Q4KUnit {
    uint4 h;  // d, dmin, scales[12]
    uint2 q;
};

__device__ __forceinline__ void dq_q4_k_load(const uint8_t *__restrict__ src, long long t, Q4KUnit &u) {
    const long long b = t >> 5;
    const int p = (int)(t & 31);
    const uint8_t *sb = src + b * kBytesQ4_K;
    u.h = *reinterpret_cast<const uint4 *>(sb);
    u.q = *reinterpret_cast<const uint2 *>(sb + 16 + 32 * (p >> 3) + 8 * (p & 3));
}

__device__ __forceinline__ void dq_q4_k_finish(const Q4KUnit &u, long long t, float *__restrict__ dst) {
    const long long b = t >> 5;
    const int p = (int)(t & 31);
    const uint4 h = u.h;
    const float d = f16_bits_to_f32(h.x & 0xffffu);
    const float dmin = f16_bits_to_f32(h.x >> 16);
    const int s = p >> 2;
    // get_scale_min_k4 (src/gguf_quant.c:212-220) on the 12 scale bytes held in h.y,h.z,h.w
    const uint32_t sw[3] = {h.y, h.z, h.w};
    auto byte_at = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    int sc, mn;
    if (s < 4) {
        sc = byte_at(s) & 63;
        mn = byte_at(s + 4) & 63;
    } else {
        sc = (byte_at(s + 4) & 0x0f) | ((byte_at(s - 4) >> 6) << 4);
        mn = (byte_at(s + 4) >> 4) | ((byte_at(s) >> 6) << 4);
    }
    const float ds = d * (float)sc;
    const float ms = dmin * (float)mn;
    const int shift = (s & 1) * 4;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = e < 4 ? u.q.x : u.q.y;
        const int c = (int)((w >> (8 * (e & 3) + shift)) & 0x0fu);
        const float prod = ds * (float)c;
        y[e] = prod - ms;
    }
    store8_nt(dst + b * kQKK + 8 * p, y);
}

__device__ __forceinline__ void dq_q4_k(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    Q4KUnit u;
    dq_q4_k_load(src, t, u);
    dq_q4_k_finish(u, t, dst);
}

__global__ __launch_bounds__(256) void dequant_q4_k_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    const long long t0 = (long long)blockIdx.x * (256 * kDqUnits) + threadIdx.x;
    Q4KUnit u[kDqUnits];
#pragma unroll
    for (int k = 0; k < kDqUnits; ++k)
        if (t0 + 256 * k < n_threads) dq_q4_k_load(src, t0 + 256 * k, u[k]);
#pragma unroll
    for (int k = 0; k < kDqUnits; ++k)
        if (t0 + 256 * k < n_threads) dq_q4_k_finish(u[k], t0 + 256 * k, dst);
}

// 32 threads per 210-byte super-block; thread p covers elements 8p..8p+7:
// half h = p/16, quarter k = (p%16)/4, position l0 = 8*(p%4).  Used by the
// row gather; the bulk kernel below gives a thread all four quarters.
__device__ __forceinline__ void dq_q6_k(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    const long long b = t >> 5;
    const int p = (int)(t & 31);
    const uint8_t *sb = src + b * kBytesQ6_K;
    const int h = p >> 4;
    const int k = (p >> 2) & 3;
    const int l0 = 8 * (p & 3);
    const uint2 ql = ldg8(sb + 64 * h + 32 * (k & 1) + l0);
    const uint2 qh = ldg8(sb + 128 + 32 * h + l0);
    const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(sb + 208));
    const float ds = d * (float)(int8_t)sb[192 + (p >> 1)];
    const int nshift = (k >> 1) * 4;
    const int hshift = 2 * k;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t wl = e < 4 ? ql.x : ql.y;
        const uint32_t wh = e < 4 ? qh.x : qh.y;
        const int lo = (int)((wl >> (8 * (e & 3) + nshift)) & 0x0fu);
        const int hi = (int)((wh >> (8 * (e & 3) + hshift)) & 0x03u);
        y[e] = ds * (float)((lo | (hi << 4)) - 32);
    }
    store8(dst + b * kQKK + 8 * p, y);
}

// Bulk Q6_K: 16 threads per super-block; thread p writes the 16 contiguous
// elements 128 h + 32 k + l0 .. + 15 (h = p / 8, quarter k = (p / 2) % 4,
// l0 = 16 (p % 2)) -- one 16-element sub-block, one scale -- from 16 bytes
// of ql, 16 of qh (each from aligned words, the block being only 2-byte
// aligned), the scale byte and d.  Two units per thread, both units' loads
// before either's arithmetic.
struct Q6KUnit {
    uint4 ql, qh;
    uint32_t s4, dw;  // the scale byte, d's bits
};

__device__ __forceinline__ void dq_q6_k16_load(const uint8_t *__restrict__ src, long long t, Q6KUnit &u) {
    const long long b = t >> 4;
    const int p = (int)(t & 15);
    const int h = p >> 3, k = (p >> 1) & 3, l0 = 16 * (p & 1);
    const uint8_t *sb = src + b * kBytesQ6_K;
    u.ql = ldg16_a2(sb + 64 * h + 32 * (k & 1) + l0);
    u.qh = ldg16_a2(sb + 128 + 32 * h + l0);
    u.s4 = sb[192 + p];                                        // sc[8h + 2k + p % 2] = sc[p]
    u.dw = *reinterpret_cast<const uint16_t *>(sb + 208);      // d (2-byte aligned)
}

// The unit's 16 outputs (values only; the caller places them).
__device__ __forceinline__ void dq_q6_k16_values(const Q6KUnit &u, int p, float (&y)[16]) {
    const int k = (p >> 1) & 3;
    const float d = f16_bits_to_f32(u.dw);
    const float ds = d * (float)(int8_t)(u.s4 & 0xffu);
    const int nshift = (k >> 1) * 4, hshift = 2 * k;
    const uint32_t ql[4] = {u.ql.x, u.ql.y, u.ql.z, u.ql.w}, qh[4] = {u.qh.x, u.qh.y, u.qh.z, u.qh.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int lo = (int)((ql[e >> 2] >> (8 * (e & 3) + nshift)) & 0x0fu);
        const int hi = (int)((qh[e >> 2] >> (8 * (e & 3) + hshift)) & 0x03u);
        y[e] = ds * (float)((lo | (hi << 4)) - 32);
    }
}

// A wave's 64 units are 4 super-blocks of contiguous output (4 KiB).  Each
// lane's 16 values go to LDS, then come back so that each of the four
// stores writes 1 KiB of consecutive float4 (lane i: float4 64 s + i): whole
// lines per store instruction, which streaming stores need.
__global__ __launch_bounds__(256) void dequant_q6_k_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    __shared__ v4f stage[4][4 * 64];  // [wave][float4 of the wave's 4 KiB]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const long long t0 = (long long)blockIdx.x * (256 * kDqUnits) + threadIdx.x;
    Q6KUnit u[kDqUnits];
    // loads clamped to the last unit (in bounds, no branch around them)
#pragma unroll
    for (int k = 0; k < kDqUnits; ++k) dq_q6_k16_load(src, min(t0 + 256 * k, n_threads - 1), u[k]);
#pragma unroll
    for (int k = 0; k < kDqUnits; ++k) {
        const long long t = t0 + 256 * k;
        // the wave's first unit: units are 16 per super-block and a wave's 64
        // units are whole super-blocks (n_threads is a multiple of 16)
        const long long wt0 = t - lane;
        if (wt0 >= n_threads) break;  // wave-uniform
        float y[16];
        dq_q6_k16_values(u[k], (int)(t & 15), y);  // lanes past the end: discarded below
#pragma unroll
        for (int q = 0; q < 4; ++q) stage[wv][4 * lane + q] = v4f{y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]};
        // one wave's LDS operations execute in issue order, so only the
        // compiler must not move the reads above the writes (a fence would
        // also wait for the other unit's loads)
        asm volatile("" ::: "memory");
        // the wave's output starts at super-block wt0 / 16; float4 64 s + lane of it
        v4f *out = reinterpret_cast<v4f *>(dst + (wt0 >> 4) * kQKK);
        const long long live4 = (min(n_threads, wt0 + 64) - wt0) * 4;  // float4s of live units
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int f = 64 * s + lane;
            if (f < live4) __builtin_nontemporal_store(stage[wv][f], out + f);
        }
        asm volatile("" ::: "memory");
    }
}

// 4 threads per 18-byte Q4_0 block; thread p covers elements 8p..8p+7: the
// low (p < 2) or high nibbles of qs[8(p&1) .. 8(p&1)+7].
__device__ __forceinline__ void dq_q4_0(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    const long long b = t >> 2;
    const int p = (int)(t & 3);
    const uint8_t *blk = src + b * kBytesQ4_0;
    const float d = f16_bits_to_f32(ldg_unaligned<uint16_t>(blk));
    const uint2 q = ldg8(blk + 2 + 8 * (p & 1));
    const int shift = (p >> 1) * 4;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = e < 4 ? q.x : q.y;
        const int c = (int)((w >> (8 * (e & 3) + shift)) & 0x0fu);
        y[e] = ((float)c - 8.0f) * d;
    }
    store8(dst + b * kQK8_0 + 8 * p, y);
}

__global__ __launch_bounds__(256) void dequant_q4_0_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_threads) return;
    dq_q4_0(src, t, dst);
}

// 4 threads per 22-byte Q5_0 block, elements as Q4_0; the fifth bit of
// element e is bit e of the block's qh word.
__device__ __forceinline__ void dq_q5_0(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    const long long b = t >> 2;
    const int p = (int)(t & 3);
    const uint8_t *blk = src + b * kBytesQ5_0;
    const float d = f16_bits_to_f32(ldg_unaligned<uint16_t>(blk));
    const uint32_t qh = ldg_unaligned<uint32_t>(blk + 2) >> (8 * p);
    const uint2 q = ldg8(blk + 6 + 8 * (p & 1));
    const int shift = (p >> 1) * 4;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = e < 4 ? q.x : q.y;
        const int c = (int)((w >> (8 * (e & 3) + shift)) & 0x0fu) | (int)(((qh >> e) & 1u) << 4);
        y[e] = (float)(c - 16) * d;
    }
    store8(dst + b * kQK8_0 + 8 * p, y);
}

__global__ __launch_bounds__(256) void dequant_q5_0_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_threads) return;
    dq_q5_0(src, t, dst);
}

// 32 threads per 176-byte Q5_K super-block; thread p covers elements
// 8p..8p+7 of sub-block s = p/4 (64-chunk j = s/2, nibble half s&1), whose
// fifth bits are bit s of qh[8(p&3) .. 8(p&3)+7].
__device__ __forceinline__ void dq_q5_k(const uint8_t *__restrict__ src, long long t, float *__restrict__ dst) {
    const long long b = t >> 5;
    const int p = (int)(t & 31);
    const uint8_t *sb = src + b * kBytesQ5_K;
    const uint4 h = ldg16(sb);  // d, dmin, scales[12]
    const float d = f16_bits_to_f32(h.x & 0xffffu);
    const float dmin = f16_bits_to_f32(h.x >> 16);
    const int s = p >> 2;
    const uint32_t sw[3] = {h.y, h.z, h.w};
    auto byte_at = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    int sc, mn;
    if (s < 4) {
        sc = byte_at(s) & 63;
        mn = byte_at(s + 4) & 63;
    } else {
        sc = (byte_at(s + 4) & 0x0f) | ((byte_at(s - 4) >> 6) << 4);
        mn = (byte_at(s + 4) >> 4) | ((byte_at(s) >> 6) << 4);
    }
    const float ds = d * (float)sc;
    const float ms = dmin * (float)mn;
    const int j = s >> 1;
    const int shift = (s & 1) * 4;
    const uint2 q = ldg8(sb + 48 + 32 * j + 8 * (p & 3));
    const uint2 qh = ldg8(sb + 16 + 8 * (p & 3));
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w = e < 4 ? q.x : q.y;
        const uint32_t wh = e < 4 ? qh.x : qh.y;
        const int c = (int)((w >> (8 * (e & 3) + shift)) & 0x0fu) + (int)(((wh >> (8 * (e & 3) + s)) & 1u) << 4);
        const float prod = ds * (float)c;
        y[e] = prod - ms;
    }
    store8(dst + b * kQKK + 8 * p, y);
}

__global__ __launch_bounds__(256) void dequant_q5_k_kernel(const uint8_t *__restrict__ src,
                                                           long long n_threads, float *__restrict__ dst) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_threads) return;
    dq_q5_k(src, t, dst);
}

// F16: one thread per 8 elements (the last thread of an n not divisible by
// 8 converts the remainder one by one).
__device__ __forceinline__ void dq_f16(const uint8_t *__restrict__ src, long long t, long long n,
                                       float *__restrict__ dst) {
    const long long e0 = 8 * t;
    if (e0 >= n) return;
    if (e0 + 8 <= n) {
        const uint4 v = ldg16(src + 2 * e0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = f16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        store8(dst + e0, y);
    } else {
        for (long long e = e0; e < n; ++e) dst[e] = f16_bits_to_f32(ldg_unaligned<uint16_t>(src + 2 * e));
    }
}

__global__ __launch_bounds__(256) void dequant_f16_kernel(const uint8_t *__restrict__ src, long long n,
                                                          float *__restrict__ dst) {
    dq_f16(src, (long long)blockIdx.x * blockDim.x + threadIdx.x, n, dst);
}

// F32: one thread per 8 elements, a copy (the last thread of an n not
// divisible by 8 copies the remainder one by one).
__device__ __forceinline__ void dq_f32(const uint8_t *__restrict__ src, long long t, long long n,
                                       float *__restrict__ dst) {
    const long long e0 = 8 * t;
    if (e0 >= n) return;
    if (e0 + 8 <= n) {
        const uint4 a = ldg16(src + 4 * e0), b = ldg16(src + 4 * e0 + 16);
        const float y[8] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w),
                            __uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w)};
        store8(dst + e0, y);
    } else {
        for (long long e = e0; e < n; ++e) dst[e] = __uint_as_float(ldg4(src + 4 * e));
    }
}

__global__ __launch_bounds__(256) void dequant_f32_kernel(const uint8_t *__restrict__ src, long long n,
                                                          float *__restrict__ dst) {
    dq_f32(src, (long long)blockIdx.x * blockDim.x + threadIdx.x, n, dst);
}

// Rows of a GGUF matrix gathered by index (the embedding lookup of
// src/native.c:428-443 through edgexpu_gguf_dequantize_row,
// src/gguf_quant.c:428-466): token y's row ids[y] dequantized into
// out[y][0..n_embd) with the bulk kernels' per-thread arithmetic
// (threads_per_row threads of 8 outputs each).  An index outside
// [0, n_rows) gives a row of zeros and sets *bad (when given) to 1.
template <int TYPE>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t *__restrict__ table, size_t row_bytes,
                                                           long long n_rows, const int32_t *__restrict__ ids,
                                                           int n_embd, long long threads_per_row,
                                                           float *__restrict__ out, int *bad) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= threads_per_row) return;
    const int id = ids[blockIdx.y];
    float *dst = out + (size_t)blockIdx.y * n_embd;
    if (id < 0 || (long long)id >= n_rows) {
        for (long long e = 8 * t; e < 8 * t + 8 && e < n_embd; ++e) dst[e] = 0.0f;
        if (t == 0 && bad != nullptr) *bad = 1;
        return;
    }
    const uint8_t *src = table + (size_t)id * row_bytes;
    if constexpr (TYPE == kTypeQ8_0) dq_q8_0(src, t, dst);
    else if constexpr (TYPE == kTypeQ4_0) dq_q4_0(src, t, dst);
    else if constexpr (TYPE == kTypeQ5_0) dq_q5_0(src, t, dst);
    else if constexpr (TYPE == kTypeQ4_K) dq_q4_k(src, t, dst);
    else if constexpr (TYPE == kTypeQ5_K) dq_q5_k(src, t, dst);
    else if constexpr (TYPE == kTypeQ6_K) dq_q6_k(src, t, dst);
    else if constexpr (TYPE == kTypeF16) dq_f16(src, t, n_embd, dst);
    else dq_f32(src, t, n_embd, dst);
}

}  // namespace exq

using namespace exq;

// n_ids rows ids[0..n_ids) of a [n_rows x n_embd] matrix of `type` into
// out[n_ids][n_embd] (16-byte aligned; n_embd a multiple of the block, of
// 4 for F16 and F32).
hipError_t launch_dequantize_rows(const uint8_t *table, int type, long long n_rows, int n_embd, const int32_t *ids,
                                  int n_ids, float *out, int *bad, hipStream_t st) {
    const bool q80 = q8_0_family(type);
    const int be = q80 ? kQK8_0 : (k_family(type) ? kQKK : 1);
    const int bb = type == kTypeQ8_0 ? kBytesQ8_0 : type == kTypeQ4_0 ? kBytesQ4_0 : type == kTypeQ5_0 ? kBytesQ5_0
                 : type == kTypeQ4_K ? kBytesQ4_K : type == kTypeQ5_K ? kBytesQ5_K : type == kTypeQ6_K ? kBytesQ6_K
                 : type == kTypeF16 ? 2 : 4;
    const size_t row_bytes = (size_t)(n_embd / be) * bb;
    // threads per row: 4 per 32-element block, 32 per super-block, n/8 for F16 and F32
    const long long tpr = q80 ? (long long)(n_embd / kQK8_0) * 4 : k_family(type) ? (long long)(n_embd / kQKK) * 32
                                                                               : (long long)((n_embd + 7) / 8);
    const dim3 grid((unsigned)((tpr + 255) / 256), (unsigned)n_ids);
#define EXQ_ROWS(T)                                                                                                 \
    hipLaunchKernelGGL(dequant_rows_kernel<T>, grid, dim3(256), 0, st, table, row_bytes, n_rows, ids, n_embd, tpr, \
                       out, bad)
    switch (type) {
        case kTypeQ8_0: EXQ_ROWS(kTypeQ8_0); break;
        case kTypeQ4_0: EXQ_ROWS(kTypeQ4_0); break;
        case kTypeQ5_0: EXQ_ROWS(kTypeQ5_0); break;
        case kTypeQ4_K: EXQ_ROWS(kTypeQ4_K); break;
        case kTypeQ5_K: EXQ_ROWS(kTypeQ5_K); break;
        case kTypeQ6_K: EXQ_ROWS(kTypeQ6_K); break;
        case kTypeF16: EXQ_ROWS(kTypeF16); break;
        case kTypeF32: EXQ_ROWS(kTypeF32); break;
        default: return hipErrorInvalidValue;
    }
#undef EXQ_ROWS
    return hipGetLastError();
}

hipError_t launch_dequantize(const uint8_t *src, int type, unsigned long long n, float *dst, hipStream_t st) {
    long long threads;
    switch (type) {
        case kTypeQ8_0:
            threads = (long long)(n / kQK8_0) * 4;
            hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src,
                               threads, dst);
            break;
        case kTypeQ4_K:
            threads = (long long)(n / kQKK) * 32;
            hipLaunchKernelGGL(dequant_q4_k_kernel, dim3((unsigned)((threads + 256 * kDqUnits - 1) / (256 * kDqUnits))),
                               dim3(256), 0, st, src, threads, dst);
            break;
        case kTypeQ6_K:
            threads = (long long)(n / kQKK) * 16;
            hipLaunchKernelGGL(dequant_q6_k_kernel, dim3((unsigned)((threads + 256 * kDqUnits - 1) / (256 * kDqUnits))),
                               dim3(256), 0, st, src, threads, dst);
            break;
        case kTypeQ4_0:
        case kTypeQ5_0:
            threads = (long long)(n / kQK8_0) * 4;
            hipLaunchKernelGGL(type == kTypeQ4_0 ? dequant_q4_0_kernel : dequant_q5_0_kernel,
                               dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src, threads, dst);
            break;
        case kTypeQ5_K:
            threads = (long long)(n / kQKK) * 32;
            hipLaunchKernelGGL(dequant_q5_k_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src,
                               threads, dst);
            break;
        case kTypeF16:
        case kTypeF32:
            threads = (long long)((n + 7) / 8);
            hipLaunchKernelGGL(type == kTypeF16 ? dequant_f16_kernel : dequant_f32_kernel,
                               dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src, (long long)n, dst);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
