// Prefill GEMM (m >= 16 tokens) on the fp16 matrix cores: out[t][o] =
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
// Tiling: a workgroup of 4 waves computes 128 tokens x 128 output rows; wave
// w owns rows 32w .. 32w+31 for all 128 tokens (4 MFMA tiles of 32 x 32).
// The K loop steps 64 elements at a time: one pair of Q4_K sub-blocks, whose
// 64 weights per row are the low and high nibbles of the same 32 bytes.  The
// weights never pass through LDS: each lane loads its row's 16 bytes of the
// pair (and the block header) from global memory and dequantizes them
// straight into its MFMA B operands, so every weight is read and converted
// once per workgroup.  The fp16 activation tile, shared by the 4 waves, goes
// from global memory straight into LDS (global_load_lds, no registers) in a
// ring of four stages; each step issues the loads of the step three ahead.
//
// Split K: when the (token, row) tiles cannot fill the chip, grid.z slices
// the K range; each slice writes its partial tile to a workspace and a second
// kernel adds bias and the slices in a fixed order (the result does not
// depend on scheduling).
//
// MFMA operand layout: lane l supplies row/column l%32 and 8 K indices of a
// 16-wide K slice, chosen by l/32 (any permutation of K works when both
// operands use the same one); accumulator register r of lane l holds
// C[8*(r/4) + 4*(l/32) + r%4][l%32], C[token][row].
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
constexpr int kF16Stage = kF16TileT * kF16KStep * 2;  // 16 KiB: the activation tile of one step
constexpr int kF16Lds = 4 * kF16Stage;                 // four stages in flight
constexpr int kF16MaxSplit = 8;
constexpr int kF16TargetGroups = 512;  // two resident workgroups per CU

// Range: fp16 holds magnitudes up to 65504, the Q8_K activations and the
// dequantized weights are f32.  Every token row t gets an exact power-of-two
// prescale 2^-e_t, chosen so that the row's largest possible magnitude is at
// most 2^15 (e_t = 0 for any row already below it).  Every weight row gets a
// running exponent e_o, raised at a super-block whose header bound needs it,
// with the row's partial sums rescaled by the same exact power of two (the
// accumulators of one lane all belong to its one weight row).  The epilogue
// multiplies the fp32 sums back by 2^(e_t + e_o).

// Exponent e >= 0 with bound * 2^-e <= 2^15.
__device__ __forceinline__ int f16_prescale_exp(float bound) {
    int e;
    (void)frexpf(bound, &e);  // bound = f * 2^e, 0.5 <= f < 1 (bound >= 0, finite)
    return e > 15 ? e - 15 : 0;
}

// Q8_K activations (reference block bytes) -> fp16 2^-e_t * dx*q8, [m][K];
// one workgroup per token row.  The row bound is 128 * max |dx| (|q8| <= 128).
__global__ __launch_bounds__(256) void q8k_to_f16_kernel(const uint8_t *__restrict__ xq, size_t xq_stride, int K,
                                                         _Float16 *__restrict__ a16, int *__restrict__ exp_t) {
    __shared__ float wmax[4];
    const int t = blockIdx.x;
    const uint8_t *row = xq + (size_t)t * xq_stride;
    const int nb = K / kQKK;
    float mx = 0.0f;
    for (int b = threadIdx.x; b < nb; b += 256)
        mx = fmaxf(mx, fabsf(*reinterpret_cast<const float *>(row + (size_t)b * kBytesQ8_K)));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, shfl_xor_f(mx, off));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int e = f16_prescale_exp(128.0f * mx);
    if (threadIdx.x == 0) exp_t[t] = e;
    for (int k = 8 * threadIdx.x; k < K; k += 8 * 256) {
        const uint8_t *blk = row + (size_t)(k / kQKK) * kBytesQ8_K;
        const float dx = ldexpf(*reinterpret_cast<const float *>(blk), -e);
        const uint2 q = ldg8(blk + 4 + (k % kQKK));
        const uint32_t qw[2] = {q.x, q.y};
        v8h out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (_Float16)(dx * (float)(int8_t)((qw[j >> 2] >> (8 * (j & 3))) & 0xffu));
        *reinterpret_cast<v8h *>(a16 + (size_t)t * K + k) = out;
    }
}

struct F16Args {
    const uint8_t *w;  // [n_out][row_bytes] Q4_K
    size_t row_bytes;
    const _Float16 *a;  // [m][K]
    const float *bias;
    float *out;   // [m][ldo]            (split == 1)
    float *part;  // [split][m][n_out]   (split > 1)
    const int *exp_t;  // [m rounded up to 128] prescale exponents of the token rows
    int ldo, m, n_out, K;
    int steps_per_split;  // a multiple of 4
};

typedef __attribute__((address_space(3))) void lds_void;

// This lane's weight loads of one step: its row's block header and the 16
// nibble bytes of its half (lane/32) of the step's sub-block pair.
struct F16W {
    v4u q, h;
};

__device__ __forceinline__ void f16_load_w(const F16Args &a, int step, int orow, int g, F16W &w) {
    // super-block step/4, pair step%4 = qs bytes 32*(step%4) .. +31
    const uint8_t *blk = a.w + (size_t)orow * a.row_bytes + (size_t)(step >> 2) * kBytesQ4_K;
    w.h = *reinterpret_cast<const v4u *>(blk);
    w.q = *reinterpret_cast<const v4u *>(blk + 16 + 32 * (step & 3) + 16 * g);
}

// Activation tile of one step, global -> LDS without registers: wave w's
// four 1 KiB loads fill tile rows 32w .. 32w+31 (8 rows of 128 bytes each);
// lane L of load i writes 16-byte slot L%8 of row r = 32w + 8i + L/8.  Chunk
// c (halfs 8c .. 8c+7) of row r sits in slot c ^ ((r/2) % 8): an MFMA read
// of one chunk down 16 consecutive rows then covers all 64 LDS banks once
// (rows of 128 bytes alternate between the two bank halves).
__device__ __forceinline__ void f16_load_a(const F16Args &a, int step, int t0, int wave, int lane, uint8_t *stage) {
    const int rl = lane >> 3, slot = lane & 7;
    const _Float16 *src = a.a + kF16KStep * step;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = min(t0 + 32 * wave + 8 * i + rl, a.m - 1);
        const int chunk = slot ^ ((4 * i + (rl >> 1)) & 7);  // ((32w + 8i + rl) / 2) % 8
        __builtin_amdgcn_global_load_lds(src + (size_t)r * a.K + 8 * chunk,
                                         (lds_void *)(stage + 1024 * (4 * wave + i)), 16, 0, 0);
    }
}

__device__ __forceinline__ uint32_t f16_pack(float lo, float hi) {
    const _Float16 l = (_Float16)lo, h = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Two weights d*q - m from nibbles q0, q1 (bytes 0 and 2 of nib) as an fp16
// pair: the bytes 0x64 | q give the fp16 values 1024 + q, from which one
// packed fp16 subtraction recovers q exactly; each d*q - m is then one
// mixed-precision fma (fp16 q, f32 d and m) rounded once to fp16.
__device__ __forceinline__ uint32_t f16_dequant2(uint32_t nib, uint32_t sel, float d, float negm) {
    const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, nib, sel);
    const h2 q = __builtin_bit_cast(h2, biased) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 r{(_Float16)__builtin_fmaf((float)q.x, d, negm), (_Float16)__builtin_fmaf((float)q.y, d, negm)};
    return __builtin_bit_cast(uint32_t, r);
}

// 8 weights from the low (HI = 0) or high nibbles of two words, K order =
// byte order
template <int HI>
__device__ __forceinline__ v8h f16_dequant8(uint32_t w0, uint32_t w1, float d, float negm) {
    const uint32_t x = (w0 >> (4 * HI)) & 0x0f0f0f0fu, y = (w1 >> (4 * HI)) & 0x0f0f0f0fu;
    // v_perm selectors: result bytes (byte 0 of nib, 0x64, byte 1, 0x64) and
    // (byte 2, 0x64, byte 3, 0x64)
    const v4u r{f16_dequant2(x, 0x04010400u, d, negm), f16_dequant2(x, 0x04030402u, d, negm),
                f16_dequant2(y, 0x04010400u, d, negm), f16_dequant2(y, 0x04030402u, d, negm)};
    return __builtin_bit_cast(v8h, r);
}

// The step's MFMA B operands for this lane's row and K half g: slice kk
// holds the K indices 32*(kk/2) + 16*g + 8*(kk%2) .. +7 of the step, i.e.
// the low (kk < 2, sub-block j0) or high (kk >= 2, sub-block j0+1) nibbles
// of qs bytes 16*g + 8*(kk%2) .. +7 of the pair.
template <int JP>
__device__ __forceinline__ void f16_dequant(const F16W &st, float wscale, v8h (&b)[4]) {
    // scales and mins of sub-blocks j0 = 2*(step%4) and j0 + 1
    // (get_scale_min_k4, src/gguf_quant.c:212-220): bytes j of the 12 packed
    // bytes (header words 1..3); for j < 4 sc = s[j]&63, m = s[j+4]&63, else
    // sc = (s[j+4]&15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4
    constexpr int sh = 16 * (JP & 1);  // byte (j0 & 3) of a word, j0 and j0+1 adjacent
    const uint32_t w1 = st.h[1] >> sh, w2 = st.h[2] >> sh, w3 = st.h[3] >> sh;
    uint32_t sc0, mn0, sc1, mn1;
    if constexpr (JP < 2) {
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
    // the row prescale 2^-e_o is exact: folded into d and dmin
    const float d = f16_bits_to_f32(st.h[0] & 0xffffu) * wscale, dm = f16_bits_to_f32(st.h[0] >> 16) * wscale;
    const float d0 = d * (float)sc0, m0 = -(dm * (float)mn0);
    const float d1 = d * (float)sc1, m1 = -(dm * (float)mn1);
    b[0] = f16_dequant8<0>(st.q[0], st.q[1], d0, m0);
    b[1] = f16_dequant8<0>(st.q[2], st.q[3], d0, m0);
    b[2] = f16_dequant8<1>(st.q[0], st.q[1], d1, m1);
    b[3] = f16_dequant8<1>(st.q[2], st.q[3], d1, m1);
}

// 128 tokens x this wave's 32 rows: A operands from the LDS stage at the
// matching K columns (swizzled slots), B from registers.
__device__ __forceinline__ void f16_compute(const uint8_t *stage, int l32, int g, const v8h (&b)[4],
                                            v16f (&acc)[4]) {
    const uint8_t *row = stage + 128 * l32;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int chunk = 4 * (kk >> 1) + 2 * g + (kk & 1);  // columns 8*chunk .. +7
        const int slot = chunk ^ ((l32 >> 1) & 7);           // row 32i + l32: (row / 2) % 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v8h av = *reinterpret_cast<const v8h *>(row + 4096 * i + 16 * slot);
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b[kk], acc[i], 0, 0, 0);
        }
    }
}

// s_waitcnt vmcnt(N) (lgkmcnt and expcnt not waited on): gfx9 encoding,
// vmcnt bits [3:0] and [15:14]
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// End of a step: this wave's loads of the next step have landed (the two
// later steps' loads, kLoadsPerStep each, may stay in flight), its LDS reads
// are done, then the workgroup barrier.  The barrier carries no memory fence:
// a fence would wait for every load in flight, the prefetched ones included.
constexpr int kLoadsPerStep = 6;  // 4 activation chunks + 2 weight loads
__device__ __forceinline__ void f16_step_barrier() {
    wait_vmcnt<2 * kLoadsPerStep>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Step s + J of the K loop (s a multiple of 4 from the slice start, which is
// itself a multiple of 4, so the step's sub-block pair is J): dequantize its
// weights from w[J], issue the loads of step s + J + 3 into w[(J+3)%4] and
// LDS stage (J+3)%4, run its MFMAs on stage J, then the step barrier.
template <int J>
__device__ __forceinline__ void f16_step(const F16Args &a, int s, int last, int t0, int orow, int &eo, float &wscale,
                                         int wave, int lane, uint8_t *smem, F16W (&w)[4], v16f (&acc)[4]) {
    const int l32 = lane & 31, g = lane >> 5;
    if constexpr (J == 0) {
        // new super-block: |d*sc*q - dmin*m| <= |d|*63*15 + |dmin|*63
        const uint32_t h = w[0].h[0];
        const int need = f16_prescale_exp(fabsf(f16_bits_to_f32(h & 0xffffu)) * 945.0f +
                                          fabsf(f16_bits_to_f32(h >> 16)) * 63.0f);
        if (need > eo) {  // rare: rescale the row's sums to the new exponent
            const float f = ldexpf(1.0f, eo - need);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= f;
            eo = need;
            wscale = ldexpf(1.0f, -need);
        }
    }
    v8h b[4];
    f16_dequant<J>(w[J], wscale, b);
    const int ahead = min(s + J + 3, last);
    f16_load_w(a, ahead, orow, g, w[(J + 3) & 3]);
    f16_load_a(a, ahead, t0, wave, lane, smem + ((J + 3) & 3) * kF16Stage);
    __builtin_amdgcn_sched_barrier(0);  // issue the loads before the step's MFMAs
    f16_compute(smem + J * kF16Stage, l32, g, b, acc);
    f16_step_barrier();
}

// Workgroup of 4 waves: 128 tokens x 128 output rows, wave w owns rows
// 32*w .. 32*w+31 (one per lane%32) for all 128 tokens (4 MFMA tiles).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_f16_kernel(F16Args a) {
    __shared__ __align__(1024) uint8_t smem[kF16Lds];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t0 = blockIdx.y * kF16TileT, o0 = blockIdx.x * kF16TileO;
    const int l32 = lane & 31, g = lane >> 5;
    const int orow = min(o0 + 32 * wave + l32, a.n_out - 1);
    const int total = a.K / kF16KStep;
    const int s0 = blockIdx.z * a.steps_per_split;
    const int n = min(a.steps_per_split, total - s0);  // a multiple of 4 (host sizing)
    const int last = s0 + n - 1;
    int eo = 0;  // running exponent of the weight row
    float wscale = 1.0f;

    v16f acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = v16f{};

    // step s's weights in w[s%4], activations in LDS stage s%4; step s + 3
    // is loaded while step s is computed (loads past the slice reload its
    // last step, into a stage no later step reads)
    F16W w[4];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        f16_load_w(a, min(s0 + j, last), orow, g, w[j]);
        f16_load_a(a, min(s0 + j, last), t0, wave, lane, smem + j * kF16Stage);
    }
    f16_step_barrier();

    for (int s = s0; s <= last; s += 4) {
        f16_step<0>(a, s, last, t0, orow, eo, wscale, wave, lane, smem, w, acc);
        f16_step<1>(a, s, last, t0, orow, eo, wscale, wave, lane, smem, w, acc);
        f16_step<2>(a, s, last, t0, orow, eo, wscale, wave, lane, smem, w, acc);
        f16_step<3>(a, s, last, t0, orow, eo, wscale, wave, lane, smem, w, acc);
    }

    const bool split = gridDim.z > 1;
    float *dst = split ? a.part + (size_t)blockIdx.z * a.m * a.n_out : a.out;
    const int ld = split ? a.n_out : a.ldo;
    // undo the prescales (slices of a split product each undo their own, so
    // the partials add in one scale) and add bias before any store: a load
    // still in flight at a conditional store makes every store wait for all
    // earlier memory operations.  Tokens of register r of tile i:
    // t0 + 32i + 8*(r/4) + 4g + r%4, four consecutive per (i, r/4).
    const float bo = (!split && a.bias != nullptr) ? a.bias[orow] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // exp_t is padded to whole tiles; padded entries only reach rows
            // t >= m, which are never stored
            const int4 et = *reinterpret_cast<const int4 *>(a.exp_t + t0 + 32 * i + 8 * q + 4 * g);
            const int e4[4] = {et.x, et.y, et.z, et.w};
#pragma unroll
            for (int p = 0; p < 4; ++p) acc[i][4 * q + p] = ldexpf(acc[i][4 * q + p], e4[p] + eo) + bo;
        }
    const int o = o0 + 32 * wave + l32;
    if (o >= a.n_out) return;
    float *col = dst + o;
    if (t0 + kF16TileT <= a.m) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                col[(size_t)(t0 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3)) * ld] = acc[i][r];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (t < a.m) col[(size_t)t * ld] = acc[i][r];
            }
    }
}

// out[t][o] = bias[o] + part[0][t][o] + part[1][t][o] + ... (fixed order);
// VEC: four consecutive outputs of a row per thread (n_out and ldo multiples
// of 4, out 16-byte aligned)
template <bool VEC>
__global__ __launch_bounds__(256) void f16_split_reduce_kernel(const float *__restrict__ part, int split, int m,
                                                               int n_out, const float *__restrict__ bias,
                                                               float *__restrict__ out, int ldo) {
    constexpr int W = VEC ? 4 : 1;
    const long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * W;
    const long long plane = (long long)m * n_out;
    if (i >= plane) return;
    const int t = (int)(i / n_out), o = (int)(i - (long long)t * n_out);
    if constexpr (VEC) {
        float4 v = bias != nullptr ? *reinterpret_cast<const float4 *>(bias + o) : make_float4(0.f, 0.f, 0.f, 0.f);
        for (int z = 0; z < split; ++z) {
            const float4 p4 = *reinterpret_cast<const float4 *>(part + (size_t)z * plane + i);
            v.x += p4.x;
            v.y += p4.y;
            v.z += p4.z;
            v.w += p4.w;
        }
        *reinterpret_cast<float4 *>(out + (size_t)t * ldo + o) = v;
    } else {
        float v = bias != nullptr ? bias[o] : 0.0f;
        for (int z = 0; z < split; ++z) v += part[(size_t)z * plane + i];
        out[(size_t)t * ldo + o] = v;
    }
}

// Split count and steps per split for an m x n_out x K product.
void f16_split(int m, int n_out, int K, int &split, int &per) {
    const int tiles = ((n_out + kF16TileO - 1) / kF16TileO) * ((m + kF16TileT - 1) / kF16TileT);
    const int total = K / kF16KStep;  // a multiple of 4
    int s = kF16TargetGroups / tiles;
    s = s < 1 ? 1 : (s > kF16MaxSplit ? kF16MaxSplit : s);
    if (s > total / 2) s = total / 2;
    per = (total + s - 1) / s;
    per = (per + 3) & ~3;  // whole super-blocks
    split = (total + per - 1) / per;
}

// Workspace of the fp16 prefill GEMM, 256-byte aligned pieces: fp16
// activations [m][K], token exponents [m rounded up to 128] and, when the K
// range is split, the partial tiles [split][m][n_out] (bytes).
struct F16Ws {
    size_t a16, exp_t, part, total;
};

F16Ws f16_ws_layout(int m, int n_out, int K, int split) {
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    F16Ws l{};
    l.a16 = 0;
    l.exp_t = up((size_t)m * K * sizeof(_Float16));
    l.part = l.exp_t + up((size_t)((m + kF16TileT - 1) / kF16TileT) * kF16TileT * sizeof(int));
    l.total = l.part + (split > 1 ? (size_t)split * m * n_out * sizeof(float) : 0);
    return l;
}

}  // namespace exq

using namespace exq;

size_t gemm_f16_workspace(int m, int n_out, int K) {
    int split, per;
    f16_split(m, n_out, K, split, per);
    return f16_ws_layout(m, n_out, K, split).total;
}

// ws: gemm_f16_workspace(m, n_out, K) bytes, 256-byte aligned.
hipError_t launch_gemm_f16(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                           size_t xq_stride, void *ws, const float *bias, float *out, int ldo, hipStream_t st) {
    if (K % kQKK != 0 || m < 1 || n_out < 1) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)ws & 255u) != 0 ||
        ((uintptr_t)xq & 3u) != 0 || (xq_stride & 3u) != 0)
        return hipErrorInvalidValue;
    int split, per;
    f16_split(m, n_out, K, split, per);
    const F16Ws l = f16_ws_layout(m, n_out, K, split);
    uint8_t *base = (uint8_t *)ws;
    F16Args a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.a = (const _Float16 *)(base + l.a16);
    a.bias = bias;
    a.out = out;
    a.part = split > 1 ? (float *)(base + l.part) : nullptr;
    a.exp_t = (const int *)(base + l.exp_t);
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.K = K;
    a.steps_per_split = per;
    hipLaunchKernelGGL(q8k_to_f16_kernel, dim3((unsigned)m), dim3(256), 0, st, xq, xq_stride, K,
                       (_Float16 *)(base + l.a16), (int *)(base + l.exp_t));
    const dim3 grid((unsigned)((n_out + kF16TileO - 1) / kF16TileO), (unsigned)((m + kF16TileT - 1) / kF16TileT),
                    (unsigned)split);
    hipLaunchKernelGGL(gemm_f16_kernel, grid, dim3(256), 0, st, a);
    if (split > 1) {
        const long long plane = (long long)m * n_out;
        const bool vec = n_out % 4 == 0 && ldo % 4 == 0 && ((uintptr_t)out & 15u) == 0 &&
                         ((uintptr_t)bias & 15u) == 0;
        if (vec)
            hipLaunchKernelGGL(f16_split_reduce_kernel<true>, dim3((unsigned)((plane / 4 + 255) / 256)), dim3(256), 0,
                               st, a.part, split, m, n_out, bias, out, ldo);
        else
            hipLaunchKernelGGL(f16_split_reduce_kernel<false>, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0,
                               st, a.part, split, m, n_out, bias, out, ldo);
    }
    return hipGetLastError();
}
