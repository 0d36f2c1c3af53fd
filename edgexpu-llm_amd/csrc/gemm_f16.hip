// Prefill GEMM (m >= 64 tokens) on the fp16 matrix cores: out[t][o] =
// bias[o] + sum_k A[t][k] * W[o][k] with
//   A[t][k] = fp16(dx[t][sb] * q8[t][k])       the Q8_K activation the
//                                              reference's integer dots use
//                                              (src/gguf_dot_q8.c:360-412)
//   W[o][k] = fp16(d1 * q - m1)                the Q4_K weight
//                                              (dequant_q4_k, src/gguf_quant.c:223-266)
// each rounded once from its f32 value, products and sums in fp32
// (v_mfma_f32_32x32x16_f16).  A rounding of at most 2^-11 on each factor
// bounds every output's error by about 2^-10 of its conditioning scale
// sum |dx*d*sc*q*q8| + |dx*dmin*m*q8| (the prefill bound of 1e-3); unlike the
// int8 path (gemm.hip), whose block integers are exact, this one trades the
// last bits for a single accumulator and no per-super-block epilogue.
//
// Tiling: a workgroup of 4 waves computes 128 tokens x 128 output rows, each
// wave 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.  The K loop steps one 32-element
// sub-block at a time (one scale and min per row per step): every step the
// workgroup stages the fp16 activation tile and dequantizes the 128 weight
// rows' sub-block into LDS, in two alternating stages, with the next step's
// global loads issued into registers before the current step is computed.
//
// MFMA operand layout (both operands the same K permutation, as checked on
// the device for the int8 shapes): lane l supplies row/column l%32 and the
// 8 K indices 8*(l/32) .. 8*(l/32)+7 of a 16-wide K slice; accumulator
// register r of lane l holds C[8*(r/4) + 4*(l/32) + r%4][l%32].
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace exq {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kF16TileT = 128;
constexpr int kF16TileO = 128;
constexpr int kF16Pitch = 40;                          // halfs per LDS row (32 + 8: spreads the banks)
constexpr int kF16Stage = (kF16TileT + kF16TileO) * kF16Pitch * 2;  // 20480 bytes
constexpr int kF16Lds = 2 * kF16Stage;

// Q8_K activations (reference block bytes) -> fp16 dx*q8, [m][K].
__global__ __launch_bounds__(256) void q8k_to_f16_kernel(const uint8_t *__restrict__ xq, size_t xq_stride, int m,
                                                         int K, _Float16 *__restrict__ a16) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // 8 elements each
    const long long total = (long long)m * K / 8;
    if (i >= total) return;
    const int t = (int)(i / (K / 8));
    const int k = (int)(i - (long long)t * (K / 8)) * 8;
    const uint8_t *blk = xq + (size_t)t * xq_stride + (size_t)(k / kQKK) * kBytesQ8_K;
    const float dx = *reinterpret_cast<const float *>(blk);
    const uint2 q = ldg8(blk + 4 + (k % kQKK));
    const uint32_t qw[2] = {q.x, q.y};
    v8h out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)(dx * (float)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xffu));
    *reinterpret_cast<v8h *>(a16 + (size_t)t * K + k) = out;
}

struct F16Args {
    const uint8_t *w;  // [n_out][row_bytes] Q4_K
    size_t row_bytes;
    const _Float16 *a;  // [m][K]
    const float *bias;
    float *out;  // [m][ldo]
    int ldo, m, n_out, K;
};

// Registers between a step's global loads and its LDS stores: two 16-byte
// chunks of the activation tile, and for weight row tid>>1 the 16 nibble
// bytes of its half (tid&1) of the sub-block plus the block header.
struct F16Stage {
    uint4 a0, a1, q, h;
};

__device__ __forceinline__ void f16_load(const F16Args &a, int step, int t0, int o0, F16Stage &st) {
    const int tid = threadIdx.x;
    const int k0 = 32 * step;
    // activation tile: 128 rows x 32 halfs = 512 chunks of 8 halfs
    {
        const int q0 = tid, q1 = tid + 256;
        const int r0 = min(t0 + (q0 >> 2), a.m - 1), r1 = min(t0 + (q1 >> 2), a.m - 1);
        st.a0 = *reinterpret_cast<const uint4 *>(a.a + (size_t)r0 * a.K + k0 + 8 * (q0 & 3));
        st.a1 = *reinterpret_cast<const uint4 *>(a.a + (size_t)r1 * a.K + k0 + 8 * (q1 & 3));
    }
    // weight row tid>>1, elements 32j + 16*(tid&1) .. +15 of super-block sb:
    // nibble (j&1) of qs bytes 32*(j>>1) + 16*(tid&1) .. +15
    {
        const int sb = step >> 3, j = step & 7;
        const int o = min(o0 + (tid >> 1), a.n_out - 1);
        const uint8_t *blk = a.w + (size_t)o * a.row_bytes + (size_t)sb * kBytesQ4_K;
        st.h = *reinterpret_cast<const uint4 *>(blk);
        st.q = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * (j >> 1) + 16 * (tid & 1));
    }
}

__device__ __forceinline__ void f16_store(const F16Stage &st, int step, uint8_t *stage) {
    const int tid = threadIdx.x;
    _Float16 *sA = reinterpret_cast<_Float16 *>(stage);
    _Float16 *sB = sA + kF16TileT * kF16Pitch;
    *reinterpret_cast<uint4 *>(sA + (tid >> 2) * kF16Pitch + 8 * (tid & 3)) = st.a0;
    *reinterpret_cast<uint4 *>(sA + ((tid + 256) >> 2) * kF16Pitch + 8 * ((tid + 256) & 3)) = st.a1;
    // dequantize 16 weights: d1 = d*sc_j, m1 = dmin*m_j (get_scale_min_k4,
    // src/gguf_quant.c:212-220), w = d1*q - m1 in f32, rounded once to fp16
    const int j = step & 7;
    const uint32_t hw[4] = {st.h.x, st.h.y, st.h.z, st.h.w};
    // byte i of the 12 packed scale bytes (words 1..3), selected without
    // indexing a register array by a run-time value
    auto sbyte = [&](int i) -> uint32_t {
        const uint32_t wd = i < 4 ? hw[1] : (i < 8 ? hw[2] : hw[3]);
        return (wd >> (8 * (i & 3))) & 0xffu;
    };
    uint32_t sc, mn;
    if (j < 4) {
        sc = sbyte(j) & 63u;
        mn = sbyte(j + 4) & 63u;
    } else {
        sc = (sbyte(j + 4) & 0xFu) | ((sbyte(j - 4) >> 6) << 4);
        mn = (sbyte(j + 4) >> 4) | ((sbyte(j) >> 6) << 4);
    }
    const float d1 = f16_bits_to_f32(hw[0] & 0xffffu) * (float)sc;
    const float m1 = f16_bits_to_f32(hw[0] >> 16) * (float)mn;
    const int sh = 4 * (j & 1);
    const uint32_t qw[4] = {st.q.x, st.q.y, st.q.z, st.q.w};
    v8h lo, hi;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const float qv = (float)((qw[e >> 2] >> (8 * (e & 3) + sh)) & 0x0fu);
        const _Float16 wv = (_Float16)(d1 * qv - m1);
        if (e < 8) lo[e] = wv;
        else hi[e - 8] = wv;
    }
    _Float16 *row = sB + (tid >> 1) * kF16Pitch + 16 * (tid & 1);
    *reinterpret_cast<v8h *>(row) = lo;
    *reinterpret_cast<v8h *>(row + 8) = hi;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_f16_kernel(F16Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wave & 1, wo = wave >> 1;  // wave tile: tokens 64*wt.., rows 64*wo..
    const int t0 = blockIdx.y * kF16TileT, o0 = blockIdx.x * kF16TileO;
    const int l32 = lane & 31, g = lane >> 5;
    const int nsteps = a.K / 32;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = v16f{};

    F16Stage st;
    f16_load(a, 0, t0, o0, st);
    f16_store(st, 0, smem);
    __syncthreads();

    for (int s = 0; s < nsteps; ++s) {
        const bool more = s + 1 < nsteps;
        // unconditional (the last step reloads itself): a conditional load
        // would keep the staging registers in memory
        f16_load(a, min(s + 1, nsteps - 1), t0, o0, st);
        const _Float16 *sA = reinterpret_cast<const _Float16 *>(smem + (s & 1) * kF16Stage);
        const _Float16 *sB = sA + kF16TileT * kF16Pitch;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            v8h av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                av[i] = *reinterpret_cast<const v8h *>(sA + (64 * wt + 32 * i + l32) * kF16Pitch + 16 * kk + 8 * g);
                bv[i] = *reinterpret_cast<const v8h *>(sB + (64 * wo + 32 * i + l32) * kF16Pitch + 16 * kk + 8 * g);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[jj], acc[i][jj], 0, 0, 0);
        }
        // the other stage was last read before the previous barrier
        if (more) f16_store(st, s + 1, smem + ((s + 1) & 1) * kF16Stage);
        __syncthreads();
    }

#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int o = o0 + 64 * wo + 32 * jj + l32;
        if (o >= a.n_out) continue;
        const float b = a.bias != nullptr ? a.bias[o] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + 64 * wt + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (t < a.m) a.out[(size_t)t * a.ldo + o] = b + acc[i][jj][r];
            }
    }
}

}  // namespace exq

using namespace exq;

// a16: [m][K] fp16 scratch the caller provides (m*K*2 bytes).
hipError_t launch_gemm_f16(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                           size_t xq_stride, _Float16 *a16, const float *bias, float *out, int ldo, hipStream_t st) {
    if (K % kQKK != 0 || m < 1 || n_out < 1) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)a16 & 15u) != 0) return hipErrorInvalidValue;
    const long long n8 = (long long)m * K / 8;
    hipLaunchKernelGGL(q8k_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, xq, xq_stride, m, K,
                       a16);
    F16Args a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.a = a16;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.K = K;
    const dim3 grid((unsigned)((n_out + kF16TileO - 1) / kF16TileO), (unsigned)((m + kF16TileT - 1) / kF16TileT));
    hipLaunchKernelGGL(gemm_f16_kernel, grid, dim3(256), kF16Lds, st, a);
    return hipGetLastError();
}
