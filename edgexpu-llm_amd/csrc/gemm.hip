// Prefill GEMM (m >= 64 tokens) of the quantized-weight path on the matrix
// cores: out[t][o] = bias[o] + sum_sb dx[t][sb] * (d[o][sb] * sumi - dmin[o][sb] * summ)
// for Q4_K weights against Q8_K activations -- edgexpu_cpu_linear_quant_batch
// (src/cpu_kernel.c:545-644) with dot_q4_k_q8_k's per-super-block integers
// (src/gguf_dot_q8.c:603-762):
//   sumi = sum_j sc_j * sum_{32} q4 * q8     summ = sum_j m_j * (bsum_2j + bsum_2j+1)
//
// Both integers are produced exactly by int8 MFMA (v_mfma_i32_16x16x64_i8,
// one instruction = one 64-element chunk = two 32-element sub-blocks):
//  * the weight operand carries the sub-block scale, split so that it fits
//    int8: sc = 8*(sc>>3) + (sc&7), nib*(sc>>3) <= 105 and nib*(sc&7) <= 105.
//    Two accumulators take the high and the low part: C = 8*C1 + C2 = sumi,
//    exact in int32.
//  * the min term: bsum_i = 128*hi_i + lo_i (hi in [-16,15], lo in [0,127]);
//    an activation operand [hi_0..15 | lo_0..15 | 0 | 0] against the weight
//    operand [m_{i/2} | 0 | 0 | 0] gives sum hi*m, shifted left by 7, then
//    against [0 | m_{i/2} | 0 | 0] adds sum lo*m: M = summ, exact.
// The fp32 combination happens once per super-block.  Results agree with the
// reference within its fp32 summation-order bound (not bit-identical: the
// reference sums in 8-lane FMA order).
//
// Tiling: a workgroup of 4 waves computes 64 tokens x 128 output rows; each
// wave 64 x 32 = 4 x 2 MFMA tiles of 16 x 16 and keeps the high- and
// low-scale sums in separate accumulators (C = 8*C1 + C2 per super-block),
// so each chunk's codes are read from LDS once.  Per super-block the
// workgroup stages in LDS the Q8_K codes of its 64 tokens (row pitch padded
// to spread LDS banks), their split 16-element sums and d, and the 128 raw
// Q4_K blocks of its rows; the next super-block's global loads are issued
// into registers before the current one is computed.  The weight operands
// are built from the raw blocks in registers (nibble extract + one 32-bit
// multiply per 4 codes: the byte products never carry).
//
// MFMA operand layout (v_mfma_i32_16x16x64_i8, checked on the device against
// a host product): lane l supplies row/column l%16 and the 16 K indices
// 16*(l/16) .. 16*(l/16)+15 of both operands; the 4 accumulator registers of
// lane l hold C[4*(l/16) + r][l%16].
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "common.h"

namespace exq {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmTileT = 64;   // tokens per workgroup
constexpr int kGemmTileO = 128;  // output rows per workgroup (32 per wave)
constexpr int kGemmPitchA = 272; // LDS row pitch of the staged codes (256 + 16: spreads the banks)
constexpr int kGemmLdsA = kGemmTileT * kGemmPitchA;   // 17408
constexpr int kGemmLdsS = kGemmTileT * 32;            // 2048: [hi 16 | lo 16] int8 per token
constexpr int kGemmLdsD = kGemmTileT * 4;             // 256
constexpr int kGemmLdsB = kGemmTileO * 128;           // 16384: the rows' nibbles (qs)
constexpr int kGemmLdsM = kGemmTileO * 32;            // 4096: per row m[8] bytes, d, dmin f32 | sc[8] bytes, pad
constexpr int kGemmStage = kGemmLdsA + kGemmLdsS + kGemmLdsD + kGemmLdsB + kGemmLdsM;  // 40192 (16-byte multiple)
static_assert(2 * kGemmStage <= 160 * 1024, "gfx950 LDS per workgroup");
constexpr int kGemmChunksA = kGemmTileT * 16 / 256;   // 16-byte chunks of codes per thread: 4
constexpr int kGemmChunksB = (kGemmTileO * 9 + 255) / 256;  // 16-byte chunks of weight blocks per thread: 5

struct GemmArgs {
    const uint8_t *w;   // [n_out][row_bytes] Q4_K
    size_t row_bytes;
    const uint8_t *xq;  // [m][xq_stride] Q8_K blocks
    size_t xq_stride;
    const float *bias;  // [n_out] or null
    float *out;         // [m][ldo]
    int ldo;
    int m, n_out, nblk;
};

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// 6-bit scale and min of sub-block j from the 12 packed bytes
// (get_scale_min_k4, src/gguf_quant.c:212-220).
__device__ __forceinline__ void scale_min_k4(const uint8_t *q, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// One super-block's operands of a workgroup, held in registers between the
// global loads (issued before the previous super-block is computed) and the
// LDS stores (after it): codes, weight blocks, and per token d + bsums.
struct GemmStage {
    uint4 a[kGemmChunksA];
    uint4 b[kGemmChunksB];
    uint32_t sd[9];  // token tid (< 64): d, then bsums 0..15 as 8 words
};

__device__ __forceinline__ void gemm_load(const GemmArgs &a, int sb, int t0, int o0, GemmStage &st) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kGemmChunksA; ++i) {
        const int q = tid + 256 * i;
        const int row = q >> 4, col = q & 15;
        const int t = min(t0 + row, a.m - 1);  // rows past m are computed and discarded
        st.a[i] = ldg16(a.xq + (size_t)t * a.xq_stride + (size_t)sb * kBytesQ8_K + 4 + 16 * col);
    }
#pragma unroll
    for (int i = 0; i < kGemmChunksB; ++i) {
        const int q = min(tid + 256 * i, kGemmTileO * 9 - 1);  // clamped; the store skips duplicates
        const int row = q / 9, part = q - row * 9;
        const int o = min(o0 + row, a.n_out - 1);
        st.b[i] = *reinterpret_cast<const uint4 *>(a.w + (size_t)o * a.row_bytes + (size_t)sb * kBytesQ4_K + 16 * part);
    }
    if (tid < kGemmTileT) {
        const int t = min(t0 + tid, a.m - 1);
        const uint8_t *blk = a.xq + (size_t)t * a.xq_stride + (size_t)sb * kBytesQ8_K;
        st.sd[0] = ldg4(blk);
#pragma unroll
        for (int p = 0; p < 8; ++p) st.sd[1 + p] = ldg4(blk + 260 + 4 * p);
    }
}

struct GemmLds {
    uint8_t *a;   // [64][kGemmPitchA] codes
    int8_t *s;    // [64][32] split 16-element sums
    float *d;     // [64] activation scales
    uint8_t *b;   // [128][128] nibbles
    uint8_t *m;   // [128][32]: m[8] d dmin (16-byte aligned) | sc[8] | pad
    __device__ GemmLds(uint8_t *base) {
        a = base;
        s = reinterpret_cast<int8_t *>(base + kGemmLdsA);
        d = reinterpret_cast<float *>(base + kGemmLdsA + kGemmLdsS);
        b = base + kGemmLdsA + kGemmLdsS + kGemmLdsD;
        m = base + kGemmLdsA + kGemmLdsS + kGemmLdsD + kGemmLdsB;
    }
};

__device__ __forceinline__ void gemm_store(const GemmStage &st, const GemmLds &L) {
    const int tid = threadIdx.x;
    uint8_t *sA = L.a;
    int8_t *sS = L.s;
    float *sD = L.d;
#pragma unroll
    for (int i = 0; i < kGemmChunksA; ++i) {
        const int q = tid + 256 * i;
        *reinterpret_cast<uint4 *>(sA + (q >> 4) * kGemmPitchA + 16 * (q & 15)) = st.a[i];
    }
#pragma unroll
    for (int i = 0; i < kGemmChunksB; ++i) {
        const int q = tid + 256 * i;
        if (q < kGemmTileO * 9) {
            const int row = q / 9, part = q - row * 9;
            if (part > 0) {
                *reinterpret_cast<uint4 *>(L.b + row * 128 + 16 * (part - 1)) = st.b[i];
            } else {
                // header: d, dmin, 12 packed scale bytes -> sc[8], m[8], d, dmin
                const uint32_t hw[4] = {st.b[i].x, st.b[i].y, st.b[i].z, st.b[i].w};
                uint8_t q12[12];
#pragma unroll
                for (int k = 0; k < 12; ++k) q12[k] = (uint8_t)(hw[1 + k / 4] >> (8 * (k % 4)));
                uint32_t scw[2] = {0u, 0u}, mw[2] = {0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int sc, mn;
                    scale_min_k4(q12, j, sc, mn);
                    scw[j >> 2] |= (uint32_t)sc << (8 * (j & 3));
                    mw[j >> 2] |= (uint32_t)mn << (8 * (j & 3));
                }
                uint32_t *dst = reinterpret_cast<uint32_t *>(L.m + row * 32);
                dst[0] = mw[0];
                dst[1] = mw[1];
                dst[2] = __float_as_uint(f16_bits_to_f32(hw[0] & 0xffffu));
                dst[3] = __float_as_uint(f16_bits_to_f32(hw[0] >> 16));
                dst[4] = scw[0];
                dst[5] = scw[1];
            }
        }
    }
    if (tid < kGemmTileT) {
        sD[tid] = __uint_as_float(st.sd[0]);
        // bsum_i = 128*hi_i + lo_i, hi in [-16, 15], lo in [0, 127]
        uint32_t hw[4] = {0u, 0u, 0u, 0u}, lw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int p = 0; p < 8; ++p) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int bs = (int)(int16_t)((st.sd[1 + p] >> (16 * h)) & 0xffffu);
                const int i = 2 * p + h;
                hw[i >> 2] |= ((uint32_t)(bs >> 7) & 0xffu) << (8 * (i & 3));
                lw[i >> 2] |= (uint32_t)(bs & 127) << (8 * (i & 3));
            }
        }
        uint4 *dst = reinterpret_cast<uint4 *>(sS + 32 * tid);
        dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        dst[1] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
}

// STAGES = 2: the next super-block is stored into the other LDS stage while
// this one is computed (one barrier per super-block); STAGES = 1: one stage,
// refilled after a barrier (two barriers, half the LDS, more workgroups per CU).
template <int STAGES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_q4k_q8k_kernel(GemmArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wo = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // rows 32*wo .. 32*wo+31
    const int t0 = blockIdx.y * kGemmTileT, o0 = blockIdx.x * kGemmTileO;
    const int li = lane & 15, g = lane >> 4;

    float acc[4][2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

    GemmStage st;
    gemm_load(a, 0, t0, o0, st);
    gemm_store(st, GemmLds(smem));
    __syncthreads();

    for (int sb = 0; sb < a.nblk; ++sb) {
        const GemmLds L(smem + (STAGES == 2 ? (sb & 1) * kGemmStage : 0));
        // the next super-block's global loads go out before this one is
        // computed, and land in the other stage afterwards
        const bool more = sb + 1 < a.nblk;
        if (more) gemm_load(a, sb + 1, t0, o0, st);

        // lane (li, g): row o = 32*wo + 16*jo + li, nibble half g>>1, so
        // chunk c uses sub-block 2c + (g>>1)
        uint32_t scw[2];
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
            const uint2 sc8 = *reinterpret_cast<const uint2 *>(L.m + (32 * wo + 16 * jo + li) * 32 + 16);
            // bytes 2c + (g>>1), c = 0..3
            const uint32_t h = g >> 1;
            const uint32_t lo = (sc8.x >> (8 * h)) & 0xffu, lo2 = (sc8.x >> (8 * (2 + h))) & 0xffu;
            const uint32_t hi = (sc8.y >> (8 * h)) & 0xffu, hi2 = (sc8.y >> (8 * (2 + h))) & 0xffu;
            scw[jo] = lo | (lo2 << 8) | (hi << 16) | (hi2 << 24);
        }

        // integer products: C1 with the high scale part, C2 with the low
        v4i c1[4][2], c2[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) c1[i][j] = c2[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v4i av[4];
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const uint4 u = *reinterpret_cast<const uint4 *>(L.a + (16 * jt + li) * kGemmPitchA + 64 * c + 16 * g);
                av[jt] = v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
            }
#pragma unroll
            for (int jo = 0; jo < 2; ++jo) {
                const uint4 u = *reinterpret_cast<const uint4 *>(L.b + (32 * wo + 16 * jo + li) * 128 + 32 * c +
                                                                 16 * (g & 1));
                const int sh = 4 * (g >> 1);
                const uint32_t s8 = (scw[jo] >> (8 * c)) & 0xffu;
                const uint32_t sh8 = s8 >> 3, sl8 = s8 & 7u;
                const uint32_t n0 = (u.x >> sh) & 0x0f0f0f0fu, n1 = (u.y >> sh) & 0x0f0f0f0fu;
                const uint32_t n2 = (u.z >> sh) & 0x0f0f0f0fu, n3 = (u.w >> sh) & 0x0f0f0f0fu;
                const v4i bh = {(int)(n0 * sh8), (int)(n1 * sh8), (int)(n2 * sh8), (int)(n3 * sh8)};
                const v4i bl = {(int)(n0 * sl8), (int)(n1 * sl8), (int)(n2 * sl8), (int)(n3 * sl8)};
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) {
                    c1[jt][jo] = mfma_i8(av[jt], bh, c1[jt][jo]);
                    c2[jt][jo] = mfma_i8(av[jt], bl, c2[jt][jo]);
                }
            }
        }

        // min term and the fp32 combination of this super-block
#pragma unroll
        for (int jo = 0; jo < 2; ++jo) {
            const uint4 mq = *reinterpret_cast<const uint4 *>(L.m + (32 * wo + 16 * jo + li) * 32);  // m[8], d, dmin
            const float dd = __uint_as_float(mq.z), dm = __uint_as_float(mq.w);
            // [m_0 m_0 m_1 m_1 ... m_7 m_7] on lane group 0 (sum hi*m) or 1 (sum lo*m)
            const uint32_t m4[2] = {mq.x, mq.y};
            uint32_t mw[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t m0 = (m4[k >> 1] >> (16 * (k & 1))) & 0xffu;
                const uint32_t m1 = (m4[k >> 1] >> (16 * (k & 1) + 8)) & 0xffu;
                mw[k] = m0 * 0x0101u | (m1 * 0x0101u) << 16;
            }
            const v4i mv = {(int)mw[0], (int)mw[1], (int)mw[2], (int)mw[3]};
            const v4i zero = {0, 0, 0, 0};
            const v4i mh = g == 0 ? mv : zero;
            const v4i ml = g == 1 ? mv : zero;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                v4i sv = {0, 0, 0, 0};
                if (g < 2) {
                    const uint4 u = *reinterpret_cast<const uint4 *>(L.s + 32 * (16 * jt + li) + 16 * g);
                    sv = v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
                }
                const float4 dx4 = *reinterpret_cast<const float4 *>(L.d + 16 * jt + 4 * g);
                const float dx[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
                v4i mm = mfma_i8(sv, mh, v4i{0, 0, 0, 0});
                mm = mm << 7;
                mm = mfma_i8(sv, ml, mm);
                const v4i ci = (c1[jt][jo] << 3) + c2[jt][jo];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = fmaf(-dm, (float)mm[r], dd * (float)ci[r]);
                    acc[jt][jo][r] = fmaf(dx[r], v, acc[jt][jo][r]);
                }
            }
        }

        // the other stage was last read in the previous iteration, before its
        // closing barrier, so it can be refilled now; one barrier per super-block
        if (STAGES == 2) {
            if (more) gemm_store(st, GemmLds(smem + ((sb + 1) & 1) * kGemmStage));
            __syncthreads();
        } else {
            __syncthreads();  // every wave is done with this super-block's operands
            if (more) {
                gemm_store(st, GemmLds(smem));
                __syncthreads();
            }
        }
    }

    // store: lane holds C[4*g + r][li] of each 16 x 16 tile.  Bias is added
    // before any store: a load still in flight at a conditional store makes
    // every store wait for all earlier memory operations.
#pragma unroll
    for (int jo = 0; jo < 2; ++jo) {
        const int o = min(o0 + 32 * wo + 16 * jo + li, a.n_out - 1);
        const float b = a.bias != nullptr ? a.bias[o] : 0.0f;
        asm volatile("" ::"v"(b));  // the load completes here, not at each store
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[jt][jo][r] += b;
    }
    const bool full = t0 + kGemmTileT <= a.m;
#pragma unroll
    for (int jo = 0; jo < 2; ++jo) {
        const int o = o0 + 32 * wo + 16 * jo + li;
        if (o >= a.n_out) continue;
        float *col = a.out + o;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + 16 * jt + 4 * g + r;
                if (full || t < a.m) col[(size_t)t * a.ldo] = acc[jt][jo][r];
            }
        }
    }
}

}  // namespace exq

using namespace exq;

bool gemm_q8_supported(int type, int n_out, int K, int m) {
    return type == kTypeQ4_K && K % kQKK == 0 && n_out > 0 && m >= 1;
}

hipError_t launch_gemm_q8(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                          size_t xq_stride, const float *bias, float *out, int ldo, hipStream_t st) {
    if (!gemm_q8_supported(type, n_out, K, m)) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)xq & 3u) != 0 || (xq_stride & 3u) != 0)
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.xq = xq;
    a.xq_stride = xq_stride;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.nblk = K / kQKK;
    static const int stages = getenv("EXQ_GEMM_STAGES") ? atoi(getenv("EXQ_GEMM_STAGES")) : 1;  // tuning override
    const dim3 grid((unsigned)((n_out + kGemmTileO - 1) / kGemmTileO), (unsigned)((m + kGemmTileT - 1) / kGemmTileT));
    if (stages == 2) {
        // more than 64 KiB of LDS per workgroup must be allowed first
        static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_q4k_q8k_kernel<2>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kGemmStage);
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL(gemm_q4k_q8k_kernel<2>, grid, dim3(256), 2 * kGemmStage, st, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(gemm_q4k_q8k_kernel<1>, grid, dim3(256), kGemmStage, st, a);
    return hipGetLastError();
}
