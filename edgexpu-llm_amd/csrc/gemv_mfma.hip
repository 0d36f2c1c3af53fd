// Decode GEMV (1..4 tokens) of Q4_K rows on the int8 matrix cores:
// edgexpu_cpu_linear_quant_batch (src/cpu_kernel.c:545-644) with the block
// integers of dot_q4_k_q8_k (src/gguf_dot_q8.c:603-666).
//
// Why the matrix cores at batch 1: the lane-per-unit GEMV spends 4-6 VALU
// lane-operations per weight byte (nibble unpacking, 16 sdot4 per 64
// weights, the per-row cross-lane sums, the scale unpacking per unit), so
// it keeps the VALU ~50 % busy while the weights stream at ~60 % of what a
// plain read reaches.  Here one v_mfma_i32_32x32x32_i8 takes a whole
// 32-element sub-block of 32 rows: B = the sub-block's nibbles as int8 (an
// AND, or a shift and an AND, per 4 weights), A = the tokens' Q8_K codes
// (token t in MFMA row t; rows t >= m read 16 zero bytes), and the exact
// int32 result for (token, row) is lane row, register token.  Per
// sub-block the 6-bit scale enters with one integer multiply-add per token,
// the min term (m_j against the 16-element code sums) with one sdot2 per
// sub-block and token, and the fp32 combination happens once per
// super-block:
//   acc += dx * (d * sumi - dmin * summ)
// ~1.5 VALU lane-operations per weight byte at one token.
//
// Layout: a wave owns 32 rows (lane l: row l % 32; lanes 32..63 hold the
// other half of each sub-block's K) and a contiguous slice of the row's
// super-blocks; KS waves of a workgroup split one row group's K and meet in
// LDS; RG = 8 / KS row groups per workgroup.  Row groups are numbered across
// up to 4 matrices of one launch (q/k/v, gate/up).  Each wave keeps two
// super-blocks of weights in flight (double-buffered registers).  The
// activation is quantized once per workgroup into LDS (the fused GEMV's
// staging, bit-identical to quantize_q8_k_kernel) while the first weights
// stream in.
//
// MFMA operand layout (v_mfma_i32_32x32x32_i8): lane l supplies row l % 32
// of A (a token) and column l % 32 of B (a weight row), K bytes
// 16 (l / 32) .. + 15; accumulator register r of lane l holds
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] -- tokens 0..3 are registers
// 0..3 of lanes 0..31.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_fused_kernel.h"

namespace exq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kMvWaves = 8;
constexpr int kMvThreads = 64 * kMvWaves;
constexpr int kMvMaxMats = 4;

struct MvArgs {
    int nmat;
    const uint8_t *w[kMvMaxMats];
    const float *bias[kMvMaxMats];
    float *out[kMvMaxMats];
    int n_out[kMvMaxMats];
    int grp_start[kMvMaxMats + 1];  // row groups of 32 before each matrix
    size_t row_bytes;
    int K, nb, m;
    int KS;       // waves per row group (K slices)
    int ngroups;  // row groups over all matrices
    const float *x;  // [m][K] f32
};

// One super-block of one row: the 16-byte header and the 4 x 16 bytes of
// qs this lane's half of the K bytes covers.
struct MvW {
    uint4 h;
    uint4 q[4];
};

__device__ __forceinline__ void mv_load(const uint8_t *row, int sb, int half, MvW &w) {
    const uint8_t *b = row + (size_t)sb * kBytesQ4_K;
    w.h = *reinterpret_cast<const uint4 *>(b);
#pragma unroll
    for (int c = 0; c < 4; ++c) w.q[c] = *reinterpret_cast<const uint4 *>(b + 16 + 32 * c + 16 * half);
}

__device__ __forceinline__ v4i as_v4i(uint4 u) { return v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w}; }

// One super-block for this lane's row: 8 MFMAs (sub-blocks 2c and 2c+1 from
// q[c]'s low and high nibbles), sumi and summ per token, the fp32 combine.
template <int M>
__device__ __forceinline__ void mv_superblock(const MvW &w, int sb, const int8_t *lq, const float *ld,
                                              const int16_t *lbs, const int8_t *zero16, int K, int nb, int lane,
                                              float (&acc)[M]) {
    const int t = lane & 31, half = lane >> 5;
    // the six-bit scales and mins of sub-blocks 0..7 (get_scale_min_k4,
    // src/gguf_quant.c:212-220), four per word
    const uint32_t sc_lo = w.h.y & 0x3f3f3f3fu, mn_lo = w.h.z & 0x3f3f3f3fu;
    const uint32_t sc_hi = (w.h.w & 0x0f0f0f0fu) | ((w.h.y >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((w.h.w >> 4) & 0x0f0f0f0fu) | ((w.h.z >> 2) & 0x30303030u);
    const float d = f16_bits_to_f32(w.h.x & 0xffffu), dmin = f16_bits_to_f32(w.h.x >> 16);
    // this lane's A operands: token t's codes of elements 32 j + 16 half .. + 15
    const int8_t *arow = t < M ? lq + (size_t)t * K + (size_t)sb * kQKK + 16 * half : zero16;
    const int astep = t < M ? 32 : 0;
    int sumi[M];
#pragma unroll
    for (int k = 0; k < M; ++k) sumi[k] = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint4 q = w.q[j >> 1];
        const uint4 b = (j & 1) ? make_uint4((q.x >> 4) & 0x0f0f0f0fu, (q.y >> 4) & 0x0f0f0f0fu,
                                             (q.z >> 4) & 0x0f0f0f0fu, (q.w >> 4) & 0x0f0f0f0fu)
                                : make_uint4(q.x & 0x0f0f0f0fu, q.y & 0x0f0f0f0fu, q.z & 0x0f0f0f0fu,
                                             q.w & 0x0f0f0f0fu);
        const uint4 a = *reinterpret_cast<const uint4 *>(arow + astep * j);
        const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(a), as_v4i(b), v16i{}, 0, 0, 0);
        const int sc = (int)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xffu);
#pragma unroll
        for (int k = 0; k < M; ++k) sumi[k] += __mul24(sc, c[k]);  // |c| < 2^23: full-rate 24-bit multiply
    }
    // summ per token: sum_j m_j * (bsum_2j + bsum_2j+1) over the token's
    // 16-element code sums (int16 pairs, one sdot2 per sub-block)
#pragma unroll
    for (int k = 0; k < M; ++k) {
        const uint4 *bp = reinterpret_cast<const uint4 *>(lbs + (size_t)k * (K / 16) + (size_t)sb * 16);
        const uint4 b0 = bp[0], b1 = bp[1];
        const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        int summ = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t mj = ((j < 4 ? mn_lo : mn_hi) >> (8 * (j & 3))) & 0xffu;
            summ = sdot2(bw[j], mj | (mj << 16), summ);
        }
        const float dx = ld[k * nb + sb];
        acc[k] = __builtin_fmaf(dx * d, (float)sumi[k], acc[k]);
        acc[k] = __builtin_fmaf(-(dx * dmin), (float)summ, acc[k]);
    }
}

template <int M>
__global__ __launch_bounds__(kMvThreads) void gemv_mfma_q4k_kernel(MvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int KS = a.KS, RG = kMvWaves / KS;
    const int rg = wave / KS, ks = wave - rg * KS;
    const int half = lane >> 5;

    // LDS: codes [m][K] | d [m][nb] | bsums [m][K/16] | 16 zero bytes | partials [8][M][32]
    const FusedLds L(a.m, a.K, a.nb, true, 1, 1, 1, true);
    int8_t *lq = reinterpret_cast<int8_t *>(smem);
    float *ld = reinterpret_cast<float *>(smem + L.qbytes);
    int16_t *lbs = reinterpret_cast<int16_t *>(smem + L.qbytes + L.dbytes);
    int8_t *zero16 = reinterpret_cast<int8_t *>(smem + L.qbytes + L.dbytes + L.bbytes);
    float *red = reinterpret_cast<float *>(smem + L.qbytes + L.dbytes + L.bbytes + 16);

    // this wave's row group, matrix and K slice (wave-uniform)
    const int grp = min((int)blockIdx.x * RG + rg, a.ngroups - 1);
    int z = 0;
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (i < a.nmat && grp >= a.grp_start[i]) z = i;
    const uint8_t *wz = a.w[0];
    const float *bz = a.bias[0];
    float *oz = a.out[0];
    int nz = a.n_out[0];
#pragma unroll
    for (int i = 1; i < kMvMaxMats; ++i)
        if (z == i) {
            wz = a.w[i];
            bz = a.bias[i];
            oz = a.out[i];
            nz = a.n_out[i];
        }
    const int row0 = 32 * (grp - a.grp_start[z]);
    const int row = row0 + (lane & 31);
    const uint8_t *wrow = wz + (size_t)min(row, nz - 1) * a.row_bytes;
    const int per = (a.nb + KS - 1) / KS;
    const int sb0 = min(ks * per, a.nb), sb1 = min(sb0 + per, a.nb);

    // 1. the staging's first round of activation loads, then the first two
    //    super-blocks of weights (in this order: loads return in order)
    FusedArgs fa{};
    fa.K = a.K;
    fa.m = a.m;
    fa.nblk = a.nb;
    fa.x = a.x;
    float xs0[16], ys0[16];
    stage_q8_k_load<kMvThreads>(fa, 0, xs0);
    MvW wb[2];
    if (sb0 < sb1) mv_load(wrow, sb0, half, wb[0]);
    if (sb0 + 1 < sb1) mv_load(wrow, sb0 + 1, half, wb[1]);
    __builtin_amdgcn_sched_barrier(0);
    // 2. quantize the activation into LDS while the weights stream in
    stage_q8_k<kMvThreads, 0>(fa, xs0, ys0, lq, ld, lbs);
    if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(zero16)[threadIdx.x] = 0u;
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int k = 0; k < M; ++k) acc[k] = 0.0f;
    // 3. the slice, two super-blocks at a time, the next pair's loads issued
    //    before this pair's arithmetic
    for (int sb = sb0; sb < sb1; sb += 2) {
        mv_superblock<M>(wb[0], sb, lq, ld, lbs, zero16, a.K, a.nb, lane, acc);
        if (sb + 2 < sb1) mv_load(wrow, sb + 2, half, wb[0]);
        if (sb + 1 < sb1) {
            mv_superblock<M>(wb[1], sb + 1, lq, ld, lbs, zero16, a.K, a.nb, lane, acc);
            if (sb + 3 < sb1) mv_load(wrow, sb + 3, half, wb[1]);
        }
    }

    // 4. the K slices meet in LDS; the slice-0 wave adds them in order, the
    //    bias after the whole dot (the reference's b + dot), and stores
    if (KS > 1) {
        if (lane < 32) {
#pragma unroll
            for (int k = 0; k < M; ++k) red[(wave * M + k) * 32 + lane] = acc[k];
        }
        __syncthreads();
        if (ks != 0) return;
        if (lane < 32) {
            for (int s = 1; s < KS; ++s)
#pragma unroll
                for (int k = 0; k < M; ++k) acc[k] += red[((wave + s) * M + k) * 32 + lane];
        }
    }
    if (lane < 32 && row < nz && (int)blockIdx.x * RG + rg < a.ngroups) {
        const float b = bz != nullptr ? bz[row] : 0.0f;
#pragma unroll
        for (int k = 0; k < M; ++k)
            if (k < a.m) oz[(size_t)k * nz + row] = b + acc[k];
    }
}

}  // namespace exq

using namespace exq;

// Q4_K rows of K (a multiple of 256, at most 16384 elements) for 1..4 tokens.
bool gemv_mfma_supported(int type, int K, int m) {
    return type == kTypeQ4_K && K % kQKK == 0 && K > 0 && K <= 16384 && m >= 1 && m <= 4;
}

hipError_t launch_gemv_mfma(int type, int nmat, const uint8_t *const *w, const int *n_out, const float *const *bias,
                            float *const *out, size_t row_bytes, int K, int m, const float *x, hipStream_t st) {
    if (!gemv_mfma_supported(type, K, m) || nmat < 1 || nmat > kMvMaxMats || ((uintptr_t)x & 15u) != 0)
        return hipErrorInvalidValue;
    MvArgs a{};
    a.nmat = nmat;
    int g = 0;
    for (int z = 0; z < nmat; ++z) {
        if (n_out[z] < 1 || ((uintptr_t)w[z] & 15u) != 0) return hipErrorInvalidValue;
        a.w[z] = w[z];
        a.bias[z] = bias != nullptr ? bias[z] : nullptr;
        a.out[z] = out[z];
        a.n_out[z] = n_out[z];
        a.grp_start[z] = g;
        g += (n_out[z] + 31) / 32;
    }
    a.grp_start[nmat] = g;
    a.ngroups = g;
    a.row_bytes = row_bytes;
    a.K = K;
    a.nb = K / kQKK;
    a.m = m;
    a.x = x;
    // K slices from K alone (so a matrix's outputs do not depend on what it
    // is grouped with): up to 8, at least two super-blocks per slice
    int ks = 1;
    while (ks < kMvWaves && a.nb >= 4 * ks) ks *= 2;
    a.KS = ks;
    const int rg = kMvWaves / ks;
    const unsigned grid = (unsigned)((g + rg - 1) / rg);
    const FusedLds L(m, K, a.nb, true, 1, 1, 1, true);
    const size_t lds = L.qbytes + L.dbytes + L.bbytes + 16 + (size_t)kMvWaves * 4 * 32 * sizeof(float);
    switch (m) {
        case 1: hipLaunchKernelGGL(gemv_mfma_q4k_kernel<1>, dim3(grid), dim3(kMvThreads), lds, st, a); break;
        case 2: hipLaunchKernelGGL(gemv_mfma_q4k_kernel<2>, dim3(grid), dim3(kMvThreads), lds, st, a); break;
        case 3: hipLaunchKernelGGL(gemv_mfma_q4k_kernel<3>, dim3(grid), dim3(kMvThreads), lds, st, a); break;
        default: hipLaunchKernelGGL(gemv_mfma_q4k_kernel<4>, dim3(grid), dim3(kMvThreads), lds, st, a); break;
    }
    return hipGetLastError();
}
