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
// wave 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.  The K loop steps 64 elements
// at a time: one pair of Q4_K sub-blocks, whose 64 weights per row are the low
// and high nibbles of the same 32 bytes.  Every step the workgroup stages the
// fp16 activation tile and dequantizes the 128 rows' sub-block pair into LDS
// (two alternating LDS stages); the global loads of a step are issued two
// steps ahead into two register sets, so a load has two step-times to land.
//
// Split K: when the (token, row) tiles cannot fill the chip, grid.z slices
// the K range; each slice writes its partial tile to a workspace and a second
// kernel adds bias and the slices in a fixed order (the result does not
// depend on scheduling).
//
// MFMA operand layout (both operands the same K permutation): lane l supplies
// row/column l%32 and the 8 K indices 8*(l/32) .. 8*(l/32)+7 of a 16-wide K
// slice; accumulator register r of lane l holds C[8*(r/4) + 4*(l/32) + r%4][l%32].
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "common.h"

namespace exq {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
// staging registers as a native vector: HIP's uint4 struct is copied through
// private memory (scratch) when it is loaded from global and stored to LDS
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kF16TileT = 128;
constexpr int kF16TileO = 128;
constexpr int kF16KStep = 64;
constexpr int kF16Pitch = kF16KStep + 8;  // halfs per LDS row (+8 spreads the banks)
constexpr int kF16Stage = (kF16TileT + kF16TileO) * kF16Pitch * 2;  // 36864 bytes
constexpr int kF16Lds = 2 * kF16Stage;
constexpr int kF16MaxSplit = 8;
constexpr int kF16TargetGroups = 512;  // two resident workgroups per CU (LDS-bound)

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
    float *out;   // [m][ldo]            (split == 1)
    float *part;  // [split][m][n_out]   (split > 1)
    int ldo, m, n_out, K;
    int steps_per_split;  // even
};

// Registers between a step's global loads and its LDS stores: four 16-byte
// chunks of the activation tile, and for weight row tid>>1 the 16 nibble
// bytes of its half (tid&1) of the sub-block pair plus the block header.
struct F16Stage {
    v4u a0, a1, a2, a3;
    v4u q, h;
};

__device__ __forceinline__ void f16_load(const F16Args &a, int step, int t0, int o0, F16Stage &st) {
    const int tid = threadIdx.x;
    const int k0 = kF16KStep * step;
    // activation tile: 128 rows x 64 halfs = 1024 chunks of 8 halfs
    // chunk c = tid + 256*i: row c/8 = tid/8 + 32*i, column 8*(tid%8)
    const _Float16 *src = a.a + k0 + 8 * (tid & 7);
    const int r = t0 + (tid >> 3);
    st.a0 = *reinterpret_cast<const v4u *>(src + (size_t)min(r, a.m - 1) * a.K);
    st.a1 = *reinterpret_cast<const v4u *>(src + (size_t)min(r + 32, a.m - 1) * a.K);
    st.a2 = *reinterpret_cast<const v4u *>(src + (size_t)min(r + 64, a.m - 1) * a.K);
    st.a3 = *reinterpret_cast<const v4u *>(src + (size_t)min(r + 96, a.m - 1) * a.K);
    // weight row tid>>1: super-block step/4, pair step%4 = qs bytes
    // 32*(step%4) .. +31, this thread's half 16*(tid&1) .. +15
    const int sb = step >> 2, jp = step & 3;
    const int o = min(o0 + (tid >> 1), a.n_out - 1);
    const uint8_t *blk = a.w + (size_t)o * a.row_bytes + (size_t)sb * kBytesQ4_K;
    st.h = *reinterpret_cast<const v4u *>(blk);
    st.q = *reinterpret_cast<const v4u *>(blk + 16 + 32 * jp + 16 * (tid & 1));
}

__device__ __forceinline__ uint32_t f16_pack(float lo, float hi) {
    const _Float16 l = (_Float16)lo, h = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

__device__ __forceinline__ void f16_store(const F16Stage &st, int step, uint8_t *stage) {
    const int tid = threadIdx.x;
    _Float16 *sA = reinterpret_cast<_Float16 *>(stage);
    _Float16 *sB = sA + kF16TileT * kF16Pitch;
    _Float16 *dstA = sA + (tid >> 3) * kF16Pitch + 8 * (tid & 7);
    *reinterpret_cast<v4u *>(dstA) = st.a0;
    *reinterpret_cast<v4u *>(dstA + 32 * kF16Pitch) = st.a1;
    *reinterpret_cast<v4u *>(dstA + 64 * kF16Pitch) = st.a2;
    *reinterpret_cast<v4u *>(dstA + 96 * kF16Pitch) = st.a3;
    // scales and mins of sub-blocks j0 = 2*(step%4) and j0 + 1
    // (get_scale_min_k4, src/gguf_quant.c:212-220): bytes j of the 12 packed
    // bytes (header words 1..3); for j < 4 sc = s[j]&63, m = s[j+4]&63, else
    // sc = (s[j+4]&15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4
    const int jp = step & 3;
    const int sh = 16 * (jp & 1);  // byte (j0 & 3) of a word, j0 and j0+1 adjacent
    const uint32_t w1 = st.h[1] >> sh, w2 = st.h[2] >> sh, w3 = st.h[3] >> sh;
    uint32_t sc0, mn0, sc1, mn1;
    if (jp < 2) {
        sc0 = w1 & 63u;
        sc1 = (w1 >> 8) & 63u;
        mn0 = w2 & 63u;
        mn1 = (w2 >> 8) & 63u;
    } else {
        sc0 = (w3 & 15u) | (((w1 >> 6) & 3u) << 4);
        sc1 = ((w3 >> 8) & 15u) | (((w1 >> 14) & 3u) << 4);
        mn0 = ((w3 >> 4) & 15u) | (((w2 >> 6) & 3u) << 4);
        mn1 = ((w3 >> 12) & 15u) | (((w2 >> 14) & 3u) << 4);
    }
    const float d = f16_bits_to_f32(st.h[0] & 0xffffu), dm = f16_bits_to_f32(st.h[0] >> 16);
    const float d0 = d * (float)sc0, m0 = dm * (float)mn0;
    const float d1 = d * (float)sc1, m1 = dm * (float)mn1;
    // w = d1*q - m1 in f32, rounded once to fp16: low nibbles -> sub-block j0,
    // high nibbles -> j0 + 1, elements 16*(tid&1) + 4*i .. +3 from word i
    const uint32_t qw[4] = {st.q[0], st.q[1], st.q[2], st.q[3]};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t l = qw[i] & 0x0f0f0f0fu, h = (qw[i] >> 4) & 0x0f0f0f0fu;
        lo[2 * i] = f16_pack(d0 * (float)(l & 0xffu) - m0, d0 * (float)((l >> 8) & 0xffu) - m0);
        lo[2 * i + 1] = f16_pack(d0 * (float)((l >> 16) & 0xffu) - m0, d0 * (float)(l >> 24) - m0);
        hi[2 * i] = f16_pack(d1 * (float)(h & 0xffu) - m1, d1 * (float)((h >> 8) & 0xffu) - m1);
        hi[2 * i + 1] = f16_pack(d1 * (float)((h >> 16) & 0xffu) - m1, d1 * (float)(h >> 24) - m1);
    }
    _Float16 *row = sB + (tid >> 1) * kF16Pitch + 16 * (tid & 1);
    *reinterpret_cast<v4u *>(row) = v4u{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<v4u *>(row + 8) = v4u{lo[4], lo[5], lo[6], lo[7]};
    *reinterpret_cast<v4u *>(row + 32) = v4u{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<v4u *>(row + 40) = v4u{hi[4], hi[5], hi[6], hi[7]};
}

__device__ __forceinline__ void f16_compute(const uint8_t *stage, int wt, int wo, int l32, int g, v16f (&acc)[2][2]) {
    const _Float16 *sA = reinterpret_cast<const _Float16 *>(stage);
    const _Float16 *sB = sA + kF16TileT * kF16Pitch;
#pragma unroll
    for (int kk = 0; kk < kF16KStep / 16; ++kk) {
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
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_f16_kernel(F16Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wave & 1, wo = wave >> 1;  // wave tile: tokens 64*wt.., rows 64*wo..
    const int t0 = blockIdx.y * kF16TileT, o0 = blockIdx.x * kF16TileO;
    const int l32 = lane & 31, g = lane >> 5;
    const int total = a.K / kF16KStep;
    const int s0 = blockIdx.z * a.steps_per_split;
    const int n = min(a.steps_per_split, total - s0);  // even, >= 2 (host sizing)
    const int last = s0 + n - 1;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = v16f{};

    // ra holds the step after the one computed, rb the one after that; loads
    // past the slice reload its last step (unconditional loads keep the
    // staging registers in registers)
    F16Stage ra, rb;
    f16_load(a, s0, t0, o0, ra);
    f16_store(ra, s0, smem);
    f16_load(a, s0 + 1, t0, o0, ra);
    f16_load(a, min(s0 + 2, last), t0, o0, rb);
    __syncthreads();

    for (int s = 0; s < n; s += 2) {
        // step s from stage 0; step s + 1 (ra) into stage 1, last read before
        // the previous barrier
        f16_compute(smem, wt, wo, l32, g, acc);
        f16_store(ra, s0 + s + 1, smem + kF16Stage);
        f16_load(a, min(s0 + s + 3, last), t0, o0, ra);
        __syncthreads();
        // step s + 1 from stage 1; step s + 2 (rb) into stage 0
        f16_compute(smem + kF16Stage, wt, wo, l32, g, acc);
        if (s + 2 < n) f16_store(rb, s0 + s + 2, smem);
        f16_load(a, min(s0 + s + 4, last), t0, o0, rb);
        __syncthreads();
    }

    const bool split = gridDim.z > 1;
    float *dst = split ? a.part + (size_t)blockIdx.z * a.m * a.n_out : a.out;
    const int ld = split ? a.n_out : a.ldo;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int o = o0 + 64 * wo + 32 * jj + l32;
        if (o >= a.n_out) continue;
        const float b = (!split && a.bias != nullptr) ? a.bias[o] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + 64 * wt + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (t < a.m) dst[(size_t)t * ld + o] = b + acc[i][jj][r];
            }
    }
}

// out[t][o] = bias[o] + part[0][t][o] + part[1][t][o] + ... (fixed order)
__global__ __launch_bounds__(256) void f16_split_reduce_kernel(const float *__restrict__ part, int split, int m,
                                                               int n_out, const float *__restrict__ bias,
                                                               float *__restrict__ out, int ldo) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long plane = (long long)m * n_out;
    if (i >= plane) return;
    const int t = (int)(i / n_out), o = (int)(i - (long long)t * n_out);
    float v = bias != nullptr ? bias[o] : 0.0f;
    for (int z = 0; z < split; ++z) v += part[(size_t)z * plane + i];
    out[(size_t)t * ldo + o] = v;
}

// Split count and steps per split for an m x n_out x K product.
void f16_split(int m, int n_out, int K, int &split, int &per) {
    const int tiles = ((n_out + kF16TileO - 1) / kF16TileO) * ((m + kF16TileT - 1) / kF16TileT);
    const int total = K / kF16KStep;  // a multiple of 4
    int s = kF16TargetGroups / tiles;
    if (const char *e = getenv("EXQ_F16_SPLIT")) s = atoi(e);
    s = s < 1 ? 1 : (s > kF16MaxSplit ? kF16MaxSplit : s);
    if (s > total / 2) s = total / 2;
    per = (total + s - 1) / s;
    per += per & 1;
    split = (total + per - 1) / per;
}

}  // namespace exq

using namespace exq;

// Workspace of the fp16 prefill GEMM: fp16 activations [m][K] and, when the
// K range is split, the partial tiles [split][m][n_out] (bytes).
size_t gemm_f16_workspace(int m, int n_out, int K) {
    int split, per;
    f16_split(m, n_out, K, split, per);
    const size_t a16 = ((size_t)m * K * sizeof(_Float16) + 255) & ~(size_t)255;
    return a16 + (split > 1 ? (size_t)split * m * n_out * sizeof(float) : 0);
}

// ws: gemm_f16_workspace(m, n_out, K) bytes, 256-byte aligned.
hipError_t launch_gemm_f16(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                           size_t xq_stride, void *ws, const float *bias, float *out, int ldo, hipStream_t st) {
    if (K % kQKK != 0 || m < 1 || n_out < 1) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)ws & 255u) != 0) return hipErrorInvalidValue;
    int split, per;
    f16_split(m, n_out, K, split, per);
    _Float16 *a16 = (_Float16 *)ws;
    const size_t a16_bytes = ((size_t)m * K * sizeof(_Float16) + 255) & ~(size_t)255;
    const long long n8 = (long long)m * K / 8;
    hipLaunchKernelGGL(q8k_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, xq, xq_stride, m, K,
                       a16);
    F16Args a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.a = a16;
    a.bias = bias;
    a.out = out;
    a.part = split > 1 ? (float *)((uint8_t *)ws + a16_bytes) : nullptr;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.K = K;
    a.steps_per_split = per;
    const dim3 grid((unsigned)((n_out + kF16TileO - 1) / kF16TileO), (unsigned)((m + kF16TileT - 1) / kF16TileT),
                    (unsigned)split);
    // more than 64 KiB of LDS per workgroup must be allowed first
    static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_f16_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kF16Lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(gemm_f16_kernel, grid, dim3(256), kF16Lds, st, a);
    if (split > 1) {
        const long long plane = (long long)m * n_out;
        hipLaunchKernelGGL(f16_split_reduce_kernel, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, st, a.part,
                           split, m, n_out, bias, out, ldo);
    }
    return hipGetLastError();
}
