// Prefill GEMM (m >= 16 tokens) of the quantized-weight path on the matrix
// cores, every block integer exact:
//   out[t][o] = bias[o] + sum_sb dx[t][sb] * (d[o][sb] * sumi - dmin[o][sb] * summ)
// for Q4_K weights against Q8_K activations -- edgexpu_cpu_linear_quant_batch
// (src/cpu_kernel.c:605-631) with dot_q4_k_q8_k's per-super-block integers
// (src/gguf_dot_q8.c:603-666):
//   sumi = sum_j sc_j * sum_{32} q4 * q8     summ = sum_j m_j * (bsum_2j + bsum_2j+1)
//
// Exact integers on fp16 matrix cores (v_mfma_f32_32x32x16_f16).  The weight
// operand is the integer sc_j * q4 <= 63 * 15 = 945 and the activation operand
// the integer code q8 in [-127, 127]; both are exact in fp16, every product is
// exact in fp32, and every partial sum is an integer.  One MFMA chain sums a
// super-block's 256 products; while every partial sum stays below 2^24 in
// magnitude the chain is exact whatever order the hardware adds in.  The
// activation packer stores each token's sum |q8| per super-block, so the
// workgroup knows the bound max_t sum|q8| * 945 before it starts a
// super-block: at most 17753 (the Q8_K codes of N(0,1) activations sum to
// ~9000) keeps the chain exact; otherwise the super-block runs as two chains
// of 128 products (15.4 M at most each), combined separately.  The min term
// is one more MFMA per tile: the 16 bsums (|bsum| <= 2032, exact in fp16)
// against m_j (<= 63).  The fp32 combination happens once per super-block:
//   acc += dx * (sumi * d - summ * dmin)
// (three VALU instructions per output and super-block).  Results agree with
// the reference within its fp32 summation-order bound (not bit-identical: the
// reference sums in 8-lane FMA order).
//
// Weight operand from the Q4_K bytes, per lane and K-step (8 fp16 values):
// u = 4 bytes of qs; (u & 0x000F000F) | 0x64006400 is the fp16 pair
// 1024 + q of the low nibbles of bytes 0 and 2, (u & 0x00F000F0) | 0x64006400
// the pair 1024 + 16 q of their high nibbles, and the same on u >> 8 for
// bytes 1 and 3.  One packed fp16 FMA per pair, (1024 + q) * sc - 1024 * sc
// or (1024 + 16 q) * (sc / 16) - 64 * sc, gives sc * q exactly (every
// constant is exact in fp16 and the result is rounded once).  Since K order
// is free when both operands use the same permutation, the activation packer
// writes the Q8_K codes as fp16 in exactly this order:
//   MFMA lane L = token + 32 h covers qs bytes 64 h .. 64 h + 63 of every row
//   (sub-blocks 4h .. 4h+3), K-step s the 4 bytes 64 h + 4 s .. + 3, and its
//   8 K slots hold [lo b0, lo b2, hi b0, hi b2, lo b1, lo b3, hi b1, hi b3].
// So a lane needs the scales of 4 sub-blocks, the B operand costs 9 VALU
// instructions per 8 weights, and each A operand is one conflict-free
// ds_read_b128 (the pack is already in lane order).
//
// Budget that shapes the tiling (measured on MI355X): a 32x32x16 fp16 MFMA
// occupies its SIMD for 32 cycles and hides only ~4 independent VALU
// instructions; every VALU instruction beyond that adds its own 4 cycles.
// LDS serves ~155 B per clock per CU.  So every dequantized weight operand
// (9 VALU) must feed several MFMAs, and every 1 KB activation operand read
// from LDS more than one:
//   * a workgroup of 8 waves (two per SIMD) computes 256 rows x 128 tokens;
//     wave w owns 64 rows (row group w % 4) for 64 tokens (token half w / 4):
//     4 MFMA tiles, each weight operand and each activation operand feeding
//     2 MFMAs, the combination 48 VALU per tile and super-block;
//   * every main-loop load is an LDS DMA; the activation pack of a half
//     super-block (128 tokens x 128 K, 32 KiB) one step ahead, its 5 KiB of
//     bsums, d and sum |q8| per super-block, the weight bytes two steps
//     ahead (the GEMM section below has the rings); one barrier per half
//     super-block.
// Shapes whose tiles cannot fill the chip split K over up to 4 workgroups
// per tile; each writes its partial tile, and the last to arrive (counted
// with a device-scope atomic) adds the partials in split order and the bias,
// so the result does not depend on which workgroup finishes last, and
// resets the counter for the next launch.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane l supplies row l % 32
// of A (a token) and column l % 32 of B (a weight row), K slots
// 8 (l / 32) .. + 7; accumulator register r of lane l holds
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], C[token][row].
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "gemm_common.h"
#include "q8k.h"

namespace exq {

constexpr int kRowsB = 32 * kWaves;  // 256 weight rows per workgroup
// largest sum |q8| of a token for which one chain of 256 products is exact:
// 17753 * 945 < 2^24
constexpr int kExactSqMax = 16777215 / 945;
constexpr int kMaxSplit = 4;

// --------------------------------------------------------------- packing

constexpr int kPackWaves = 8;  // workgroup of the pack kernels
constexpr int kPackThreads = 64 * kPackWaves;
constexpr int kPackF32Tokens = 4;  // tokens per wavefront of the f32 pack

// Code vectors of the pack: the 16-byte vector of (half hf, K-step s, lane
// half h) holds elements 64 j + 4 s .. + 3 (the low nibble positions of qs
// bytes 32 j + 4 s .. + 3) and 64 j + 32 + 4 s .. + 3 (their high nibbles)
// with j = 2 h + hf, as fp16 [lo 0, lo 2, hi 0, hi 2, lo 1, lo 3, hi 1, hi 3].
// Tokens past m get zero codes and d = 0.

// The f32 pack kernel: one wavefront per (super-block, 4 consecutive
// tokens), 8 wavefronts (32 tokens, one MFMA token tile) per workgroup,
// everything in registers.  The 16 lanes 16 t4 + 4 j + q of token t4 hold
// its elements 64 j + 8 q .. + 7 and 64 j + 32 + 8 q .. + 7: the code vectors
// of K-steps 2 q and 2 q + 1 of half j & 1, lane half j >> 1, with no
// exchange.  The Q8_K quantization (src/gguf_dot_q8.c:360-412) runs over a
// 16-lane row: the largest |x| (zeros and NaN never enter) by a row max,
// then iscale = -127 / max|x| and each code as quantize_q8_k_kernel forms
// it.  The reference's max carries the sign of the first element of largest
// |x|; where that is negative, this block is the reference's with codes,
// bsums and d negated, which every product of the GEMM, dx * (C d - mn dmin)
// with C and mn integer sums of the codes, leaves word for word (sum |q| is
// the same either way).
__global__ __launch_bounds__(kPackThreads) void q8k_pack_f32_kernel(const float *__restrict__ x, int ldx, int m,
                                                                    int K, int ntb, uint8_t *__restrict__ pack) {
    const int nb = K / kQKK;
    const int sb = (int)blockIdx.x % nb, tg = (int)blockIdx.x / nb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t4 = lane >> 4, r = lane & 15, j = r >> 2, q = r & 3;
    const int t = (tg * kPackWaves + wave) * kPackF32Tokens + t4;
    // xs[i] = element 64 j + 8 q + i, xs[8 + i] = element 64 j + 32 + 8 q + i
    float xs[16];
    {
        float4 v[4] = {};
        if (t < m) {
            const float *src = x + (size_t)t * ldx + (size_t)sb * kQKK + 64 * j + 8 * q;
            v[0] = *reinterpret_cast<const float4 *>(src);
            v[1] = *reinterpret_cast<const float4 *>(src + 4);
            v[2] = *reinterpret_cast<const float4 *>(src + 32);
            v[3] = *reinterpret_cast<const float4 *>(src + 36);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            xs[4 * k] = v[k].x;
            xs[4 * k + 1] = v[k].y;
            xs[4 * k + 2] = v[k].z;
            xs[4 * k + 3] = v[k].w;
        }
    }
    uint32_t bb[16], amax_bits = 0u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float av = fabsf(xs[i]);
        bb[i] = av > 0.0f ? __float_as_uint(av) : 0u;  // non-negative floats order as their bits
        amax_bits = max(amax_bits, bb[i]);
    }
    amax_bits = row16_max_u32(amax_bits);
    const bool zero = amax_bits == 0u;
    const float iscale = -127.0f / __uint_as_float(amax_bits);
    int qv[16], lo8 = 0, hi8 = 0, sq = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float pv = iscale * xs[i];
        // lrintf: a NaN or infinite product gives LONG_MIN, whose low 32 bits are 0
        int c = fabsf(pv) < 2147483648.0f ? (int)rintf(pv) : 0;
        c = c > 127 ? 127 : (c < -127 ? -127 : c);
        c = zero ? 0 : c;
        qv[i] = c;
        if (i < 8)
            lo8 += c;
        else
            hi8 += c;
        sq += abs(c);
    }
    const float d = zero ? 0.0f : 1.0f / iscale;
    // bsums: lanes q and q ^ 1 share the 16-element groups 4 j + q / 2 (low)
    // and 4 j + 2 + q / 2 (high); lane q = 0 then takes groups 4 j + 1 and
    // 4 j + 3 from lane q = 2
    lo8 += (int)dpp_u32<kDppXor1>((uint32_t)lo8);
    hi8 += (int)dpp_u32<kDppXor1>((uint32_t)hi8);
    const int lo_n = (int)dpp_u32<kDppXor2>((uint32_t)lo8), hi_n = (int)dpp_u32<kDppXor2>((uint32_t)hi8);
    sq += (int)dpp_u32<kDppXor1>((uint32_t)sq);
    sq += (int)dpp_u32<kDppXor2>((uint32_t)sq);
    sq += (int)dpp_u32<kDppHalfMirror>((uint32_t)sq);
    sq += (int)dpp_u32<kDppMirror>((uint32_t)sq);

    const int tb = t / kTokB, tt = (t % kTokB) / 32, tl = t % 32;
    const int h = j >> 1, hf = j & 1;
    uint8_t *blk = pack + ((size_t)sb * ntb + tb) * kPkBlk;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int s = 2 * q + u;
        v4u o;
        o[0] = h2_bits(qv[4 * u], qv[4 * u + 2]);
        o[1] = h2_bits(qv[8 + 4 * u], qv[8 + 4 * u + 2]);
        o[2] = h2_bits(qv[4 * u + 1], qv[4 * u + 3]);
        o[3] = h2_bits(qv[8 + 4 * u + 1], qv[8 + 4 * u + 3]);
        *reinterpret_cast<v4u *>(blk + hf * kPkHalf + (s * kTiles + tt) * 1024 + (tl + 32 * h) * 16) = o;
    }
    // min-term vector of lane half h: bsums 8 h .. 8 h + 7 as fp16 pairs; this
    // row's groups 4 j .. 4 j + 3 are its bytes 8 hf .. 8 hf + 7
    if (q == 0) {
        uint2 o;
        o.x = h2_bits(lo8, lo_n);
        o.y = h2_bits(hi8, hi_n);
        *reinterpret_cast<uint2 *>(blk + kPkCodes + tt * 1024 + (tl + 32 * h) * 16 + 8 * hf) = o;
    }
    if (r == 0) {
        *reinterpret_cast<float *>(blk + kPkCodes + kPkMn + 4 * (32 * tt + tl)) = d;
        *reinterpret_cast<int *>(blk + kPkCodes + kPkMn + kPkDx + 4 * (32 * tt + tl)) = sq;
    }
}

// The Q8_K-block pack kernel: one wavefront per (super-block, token), 8
// wavefronts (8 consecutive tokens, whose 16-byte vectors fill 128-byte
// lines) per workgroup.  Lane l reads the codes of elements 4 l .. 4 l + 3,
// so lane 16 j + s writes the code vector of K-step s of half j & 1, lane
// half j >> 1 after one exchange with lane 16 j + s + 8.
__global__ __launch_bounds__(kPackThreads) void q8k_pack_blocks_kernel(const uint8_t *__restrict__ xq,
                                                                       size_t xq_stride, int m, int K, int ntb,
                                                                       uint8_t *__restrict__ pack) {
    const int nb = K / kQKK;
    const int sb = (int)blockIdx.x % nb, tg = (int)blockIdx.x / nb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = tg * kPackWaves + wave;
    uint32_t word = 0u, dw = 0u, bw = 0u;
    if (t < m) {
        const uint8_t *blk = xq + (size_t)t * xq_stride + (size_t)sb * kBytesQ8_K;
        word = ldg4(blk + 4 + 4 * lane);
        dw = ldg4(blk);
        bw = ldg4(blk + 260 + 4 * (lane >> 3));  // bsums 2k, 2k+1 of k = lane >> 2
    }
    const int j = lane >> 4, s8 = lane & 7;
    const int h = j >> 1, hf = j & 1;
    const int tb = t / kTokB, tt = (t % kTokB) / 32, tl = t % 32;
    uint8_t *blk = pack + ((size_t)sb * ntb + tb) * kPkBlk;
    int q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = sbyte(word, e);
    const float d = __uint_as_float(dw);
    const int bsum = (int)(int16_t)((bw >> (16 * ((lane >> 2) & 1))) & 0xffffu);
    const int sq = wave_sum(abs(q[0]) + abs(q[1]) + abs(q[2]) + abs(q[3]));
    const uint32_t hiw = (uint32_t)__shfl_xor((int)word, 8, 64);
    if ((lane & 8) == 0) {
        v4u o;
        o[0] = h2_bits(sbyte(word, 0), sbyte(word, 2));
        o[1] = h2_bits(sbyte(hiw, 0), sbyte(hiw, 2));
        o[2] = h2_bits(sbyte(word, 1), sbyte(word, 3));
        o[3] = h2_bits(sbyte(hiw, 1), sbyte(hiw, 3));
        *reinterpret_cast<v4u *>(blk + hf * kPkHalf + (s8 * kTiles + tt) * 1024 + (tl + 32 * h) * 16) = o;
    }
    // min-term vector of lane half hh = lane (lanes 0, 1): bsums 8 hh .. 8 hh + 7,
    // held by lanes 32 hh + 4 k
    int bv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) bv[k] = __shfl(bsum, 32 * (lane & 1) + 4 * k, 64);
    if (lane < 2) {
        v4u o;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = h2_bits(bv[2 * k], bv[2 * k + 1]);
        *reinterpret_cast<v4u *>(blk + kPkCodes + tt * 1024 + (tl + 32 * lane) * 16) = o;
    }
    if (lane == 0) {
        *reinterpret_cast<float *>(blk + kPkCodes + kPkMn + 4 * (32 * tt + tl)) = d;
        *reinterpret_cast<int *>(blk + kPkCodes + kPkMn + kPkDx + 4 * (32 * tt + tl)) = sq;
    }
}

// ------------------------------------------------------------------ GEMM
//
// Wave tiles: wave w owns row group g = w % 4 (64 rows: 2 halves of 32) and
// token half th = w / 4 (64 tokens: 2 MFMA tiles).  Per K-step it builds 2
// weight operands (9 VALU each), reads 2 activation operands (1 KiB each)
// and issues 4 MFMAs, so LDS serves 0.5 KiB per MFMA -- reading one
// activation operand per MFMA (32 rows x 128 tokens per wave) saturates the
// LDS at ~42 % of the matrix-core peak.
//
// Every global load of the main loop is an LDS DMA (buffer_load ... lds)
// written as inline assembly, and every wait for one is an explicit
// s_waitcnt: the compiler then has no loads of its own in the loop and no
// reason to drain the DMA queue before LDS reads it cannot tell apart from
// the slots in flight.  The weights come from HBM (first touch) and are
// requested two steps ahead; the codes are L2 hits (every row block reads
// them) and one step ahead is enough.  LDS (135 KiB of the 160):
//   codes    2 slots x 32 KiB  half super-block of activation codes, one step ahead
//   extras   2 slots x 5 KiB   bsums / d / sum |q8| of a super-block
//   weights  3 slots x 20 KiB  per row group 5 KiB: qs pieces of both row
//                              halves and the 64 headers; two steps ahead
constexpr int kCodeSlots = 2;
constexpr int kWSlots = 3;
constexpr int kWGrp = 5 * 1024;
constexpr int kWSlot = 4 * kWGrp;
constexpr int kLdsCodes = 0;
constexpr int kLdsEx = kLdsCodes + kCodeSlots * kPkHalf;
constexpr int kLdsW = kLdsEx + 2 * kPkExtra;
constexpr int kLdsLast = kLdsW + kWSlots * kWSlot;
constexpr int kLdsBytes = kLdsLast + 16;
static_assert(kLdsBytes <= 160 * 1024, "the LDS rings fit the gfx950 LDS");

struct GmArgs {
    const uint8_t *w;     // [n_out][row_bytes] Q4_K
    size_t row_bytes;
    const uint8_t *pack;  // [nblk][ntb][kPkBlk]
    uint32_t pack_bytes;  // < 4 GiB (checked at launch)
    int ntb;              // 128-token blocks in the pack
    const float *bias;    // [n_out] or null
    float *out;           // [m][ldo]
    int ldo, m, n_out, nblk;
    int nrb;              // row blocks of kRowsB
    int ntiles;           // nrb * ntb
    int nsplit;           // workgroups per tile along K (1 .. kMaxSplit)
    float *part;          // [nsplit][ntiles][16][kThreads] float4 partial tiles (nsplit > 1)
    unsigned *cnt;        // [ntiles] arrival counters, zero between launches
};

// Constants of one super-block for one row and sub-blocks 4h .. 4h+3
// (get_scale_min_k4, src/gguf_quant.c:212-220, for four sub-blocks at once):
// the four 6-bit scales, the min operand, d and -dmin.
struct WConst {
    uint32_t sc4;
    v8h bmn;
    float dd, ndm;
};

__device__ __forceinline__ WConst w_const(const v4u hd, int h) {
    const uint32_t w0 = hd[1], w1 = hd[2], w2 = hd[3];
    const uint32_t sel = 0u - (uint32_t)h;  // all ones for sub-blocks 4..7
    const uint32_t m4 = ((w1 & 0x3f3f3f3fu) & ~sel) | ((((w2 >> 4) & 0x0f0f0f0fu) | ((w1 >> 2) & 0x30303030u)) & sel);
    WConst c;
    c.sc4 = ((w0 & 0x3f3f3f3fu) & ~sel) | (((w2 & 0x0f0f0f0fu) | ((w0 >> 2) & 0x30303030u)) & sel);
    c.dd = f16_bits_to_f32(hd[0] & 0xffffu);
    c.ndm = -f16_bits_to_f32(hd[0] >> 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const _Float16 mv = (_Float16)(float)((m4 >> (8 * k)) & 0xffu);
        c.bmn[2 * k] = mv;
        c.bmn[2 * k + 1] = mv;
    }
    return c;
}

// The packed-FMA multipliers / addends of half p of the super-block: the
// low- and high-nibble weights of sub-blocks 4h + 2p and 4h + 2p + 1.
struct HalfConst {
    h2 mlo, alo, mhi, ahi;
};

__device__ __forceinline__ HalfConst half_const(uint32_t sc4, int p) {
    const float lo = (float)((sc4 >> (16 * p)) & 0xffu), hi = (float)((sc4 >> (16 * p + 8)) & 0xffu);
    const _Float16 ml = (_Float16)lo, al = (_Float16)(-1024.0f * lo);
    const _Float16 mh = (_Float16)(0.0625f * hi), ah = (_Float16)(-64.0f * hi);
    return HalfConst{h2{ml, ml}, h2{al, al}, h2{mh, mh}, h2{ah, ah}};
}

struct NibMasks {
    uint32_t lo, hi, bias;  // 0x000F000F, 0x00F000F0, 0x64006400, held in VGPRs
};

// Weight operand of one K-step from its 4 qs bytes u (the lane's qs dword).
__device__ __forceinline__ v8h w_operand(uint32_t u, const HalfConst &c, const NibMasks &k) {
    const uint32_t u8 = u >> 8;
    const h2 y0 = __builtin_bit_cast(h2, (u & k.lo) | k.bias);
    const h2 y1 = __builtin_bit_cast(h2, (u & k.hi) | k.bias);
    const h2 y2 = __builtin_bit_cast(h2, (u8 & k.lo) | k.bias);
    const h2 y3 = __builtin_bit_cast(h2, (u8 & k.hi) | k.bias);
    const h2 b0 = __builtin_elementwise_fma(y0, c.mlo, c.alo);
    const h2 b1 = __builtin_elementwise_fma(y1, c.mhi, c.ahi);
    const h2 b2 = __builtin_elementwise_fma(y2, c.mlo, c.alo);
    const h2 b3 = __builtin_elementwise_fma(y3, c.mhi, c.ahi);
    return v8h{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

// C[g][tt]: the wave's 2 row halves x 2 token tiles.
typedef v16f Tiles[2][2];

// The 8 K-steps of half p: codes slot `cur` (this wave's two token tiles at
// `cur + tt * 1024`, stride 4 KiB per K-step), this row group's weight slot
// `wq` (qs pieces of row half g at wq + 2 KiB g).  Four accumulator chains
// advance together; each K-step reads 2 activation operands and issues 4
// MFMAs on 2 weight operands.  The weight operands of the next K-step (18
// VALU) are built while this K-step's MFMAs run, interleaved with them
// (an MFMA hides only a few VALU instructions issued behind it, and a block
// of VALU with no MFMA in flight leaves the matrix core idle).  FIRST: the
// chains start at zero.
template <int P, bool FIRST, int NT>
__device__ __forceinline__ void half_chains(const uint8_t *cur, const uint8_t *wq, int lane, const WConst (&wc)[2],
                                            const NibMasks &k, Tiles &C) {
    const HalfConst c0 = half_const(wc[0].sc4, P), c1 = half_const(wc[1].sc4, P);
    const v4u q00 = lds_v4u(wq + lane * 16), q01 = lds_v4u(wq + 1024 + lane * 16);
    const v4u q10 = lds_v4u(wq + 2048 + lane * 16), q11 = lds_v4u(wq + 3072 + lane * 16);
    v8h a[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) a[tt] = lds_v8h(cur + tt * 1024 + lane * 16);
    v8h b0 = w_operand(q00[0], c0, k), b1 = w_operand(q10[0], c1, k);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        v8h nb0 = b0, nb1 = b1;
        if (s + 1 < 8) {
            nb0 = w_operand(s + 1 < 4 ? q00[s + 1] : q01[s - 3], c0, k);
            nb1 = w_operand(s + 1 < 4 ? q10[s + 1] : q11[s - 3], c1, k);
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            C[0][tt] = mfma(a[tt], b0, (FIRST && s == 0) ? v16f{} : C[0][tt]);
            C[1][tt] = mfma(a[tt], b1, (FIRST && s == 0) ? v16f{} : C[1][tt]);
            if (s + 1 < 8) a[tt] = lds_v8h(cur + (s + 1) * 4096 + tt * 1024 + lane * 16);
        }
        if (NT == 2) {
            // MFMA, VALU x5, MFMA, DS read, VALU x4, MFMA, VALU x5, MFMA, DS read, VALU x4
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
        } else {
            // MFMA, VALU x9, DS read, MFMA, VALU x9
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        b0 = nb0;
        b1 = nb1;
    }
}

// acc += dx * (C * d - mn * dmin) for the wave's tiles (MN = false:
// acc += dx * C * d).  `ex` is the extras slot, `tq` the wave's first token
// tile in the workgroup (0 or 2).
template <bool MN, int NT>
__device__ __forceinline__ void combine(const uint8_t *ex, int tq, int lane, const WConst (&wc)[2], const Tiles &C,
                                        Tiles &acc) {
    const int h = lane >> 5;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        v16f mn[2] = {v16f{}, v16f{}};
        if (MN) {
            const v8h bs = lds_v8h(ex + (tq + tt) * 1024 + lane * 16);
            mn[0] = mfma(bs, wc[0].bmn, v16f{});
            mn[1] = mfma(bs, wc[1].bmn, v16f{});
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 dx = *reinterpret_cast<const float4 *>(ex + kPkMn + 4 * (32 * (tq + tt) + 8 * i + 4 * h));
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int g = 0; g < 2; ++g) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * i + e;
                    float v = C[g][tt][r] * wc[g].dd;
                    if (MN) v = __builtin_fmaf(mn[g][r], wc[g].ndm, v);
                    acc[g][tt][r] = __builtin_fmaf(v, dxs[e], acc[g][tt][r]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Per-wave state of the main loop.
struct GmLoop {
    v4u pack, rows;           // descriptors: the activation pack, this row group's 64 rows
    uint32_t pk0, pk_sb;      // pack offset of this token block, bytes per super-block
    uint32_t voff_q, voff_h;  // per lane: qs half of row 32 th + lane % 32 (+ 64 h), header of row lane
    uint32_t smem;            // LDS address of the workgroup's buffer
    NibMasks km;
    int lane, wave, grp, th, sb0, sblast;
    bool codes_on;            // the wave's code chunks (token tile wave % 4) hold a token below m
    bool ex_on;               // the wave's extras chunk: bsums of a live tile, or dx / sum |q8|
};

// Step s (half hf = s & 1 of super-block sb0 + s / 2) requests, in this
// order: the codes of step s + 1 (4 DMAs, a quarter of the half super-block),
// on odd steps the extras of the next super-block (1 DMA, waves 0..4), then
// the weights of step s + 2 (3 DMAs:
// qs pieces 0 and 1 of row half th of the wave's row group, the group's 64
// headers -- both token-half waves request them, the same bytes; rows past
// n_out read zeros).  Requests past the end of the K range re-request its
// last super-block into slots nobody reads again, so every step issues its
// weights last: a wait for vmcnt(3) at the start of step s + 1 leaves
// exactly the weights of step s + 2 in flight, however many code and extras
// chunks a wave skips (those of token tiles past the last token, which no
// wave reads).
constexpr int kWLoads = 3;

__device__ __forceinline__ void step_requests(const GmLoop &L, int s) {
    const uint32_t lv = (uint32_t)L.lane * 16;
    const int s1 = s + 1;
    const int sbc = min(L.sb0 + (s1 >> 1), L.sblast);
    const uint32_t cdst = L.smem + kLdsCodes + (uint32_t)(s1 % kCodeSlots) * kPkHalf;
    const uint32_t cso = L.pk0 + (uint32_t)sbc * L.pk_sb + (uint32_t)(s1 & 1) * kPkHalf;
    if (L.codes_on) {
#pragma unroll
        for (int i = 0; i < kHalfChunks / kWaves; ++i) {
            const uint32_t ch = (uint32_t)(kWaves * i + L.wave);
            dma16(cdst + ch * 1024, lv, L.pack, cso + ch * 1024);
        }
    }
    if ((s & 1) && L.ex_on) {  // extras of super-block sb0 + (s + 1) / 2
        const int je = s1 >> 1;
        const int sbe = min(L.sb0 + je, L.sblast);
        const uint32_t ch = (uint32_t)L.wave;
        dma16(L.smem + kLdsEx + (uint32_t)(je & 1) * kPkExtra + ch * 1024, lv, L.pack,
              L.pk0 + (uint32_t)sbe * L.pk_sb + kPkCodes + ch * 1024);
    }
    const int s2 = s + 2;
    const int sbw = min(L.sb0 + (s2 >> 1), L.sblast);
    const uint32_t wdst = L.smem + kLdsW + (uint32_t)(s2 % kWSlots) * kWSlot + (uint32_t)L.grp * kWGrp;
    const uint32_t wso = (uint32_t)sbw * kBytesQ4_K + 16 + 32 * (uint32_t)(s2 & 1);
    dma16(wdst + 2048 * L.th, L.voff_q, L.rows, wso);
    dma16(wdst + 2048 * L.th + 1024, L.voff_q, L.rows, wso + 16);
    dma16(wdst + 4096, L.voff_h, L.rows, (uint32_t)sbw * kBytesQ4_K);
}

// The main loop over the workgroup's super-blocks for a wave with NT live
// token tiles (NT = 0: the wave only moves data for the others).
template <int NT>
__device__ __forceinline__ void q4k_loop(const GmLoop &L, uint8_t *smem, int nsb, int tq, Tiles &C, Tiles &acc) {
    const int lane = L.lane, grp = L.grp, h = lane >> 5;
    for (int j = 0; j < nsb; ++j) {
        const int s = 2 * j;
        const uint8_t *ex = smem + kLdsEx + (j & 1) * kPkExtra;
        // even step: half 0 of super-block sb0 + j
        wait_dma<kWLoads>();
        __syncthreads();
        step_requests(L, s);
        if constexpr (NT > 0) {
            const uint8_t *wq0 = smem + kLdsW + (s % kWSlots) * kWSlot + grp * kWGrp;
            WConst wc[2];
#pragma unroll
            for (int g = 0; g < 2; ++g) wc[g] = w_const(lds_v4u(wq0 + 4096 + (32 * g + (lane & 31)) * 16), h);
            const int sq0 = *reinterpret_cast<const int *>(ex + kPkMn + kPkDx + 4 * lane);
            const int sq1 = *reinterpret_cast<const int *>(ex + kPkMn + kPkDx + 4 * (lane + 64));
            // the exactness bound of one chain over the workgroup's 128 tokens
            const bool split = wave_max_dpp(max(sq0, sq1)) > kExactSqMax;
            const uint8_t *cur0 = smem + kLdsCodes + tq * 1024;  // even steps use code slot 0
            half_chains<0, true, NT>(cur0, wq0, lane, wc, L.km, C);
            if (split) combine<false, NT>(ex, tq, lane, wc, C, acc);
            // odd step: half 1
            wait_dma<kWLoads>();
            __syncthreads();
            step_requests(L, s + 1);
            const uint8_t *wq1 = smem + kLdsW + ((s + 1) % kWSlots) * kWSlot + grp * kWGrp;
            const uint8_t *cur1 = smem + kLdsCodes + kPkHalf + tq * 1024;
            if (split)
                half_chains<1, true, NT>(cur1, wq1, lane, wc, L.km, C);
            else
                half_chains<1, false, NT>(cur1, wq1, lane, wc, L.km, C);
            combine<true, NT>(ex, tq, lane, wc, C, acc);
        } else {
            wait_dma<kWLoads>();
            __syncthreads();
            step_requests(L, s + 1);
        }
    }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_q4k_kernel(GmArgs a) {
    __shared__ __align__(16) uint8_t smem[kLdsBytes];
    int *s_last = reinterpret_cast<int *>(smem + kLdsLast);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int grp = wave & 3, th = wave >> 2;

    // workgroups sharing a row block are a multiple of nrb apart; with nrb a
    // multiple of 8 they land on one XCD and share its L2 copy of the weights
    const int tile = (int)blockIdx.x % a.ntiles, z = (int)blockIdx.x / a.ntiles;
    const int rb = tile % a.nrb, tb = tile / a.nrb;
    const int sb0 = (int)((long long)a.nblk * z / a.nsplit);
    const int sb1 = (int)((long long)a.nblk * (z + 1) / a.nsplit);
    const int nsb = sb1 - sb0;

    const int rowg = rb * kRowsB + 64 * grp;  // first row of the row group
    GmLoop L;
    L.lane = lane;
    L.wave = wave;
    L.grp = grp;
    L.th = th;
    L.sb0 = sb0;
    L.sblast = sb1 - 1;
    L.pk_sb = (uint32_t)a.ntb * kPkBlk;
    L.pk0 = (uint32_t)tb * kPkBlk;
    L.pack = rsrc_words(a.pack, a.pack_bytes);
    const int live_rows = min(64, a.n_out - rowg);  // rows past n_out lie past the descriptor (zeros)
    L.rows = rsrc_words(a.w + (size_t)min(rowg, a.n_out - 1) * a.row_bytes,
                        live_rows > 0 ? (uint32_t)live_rows * (uint32_t)a.row_bytes : 0u);
    L.voff_h = (uint32_t)lane * (uint32_t)a.row_bytes;
    L.voff_q = (uint32_t)(32 * th + (lane & 31)) * (uint32_t)a.row_bytes + 64u * (uint32_t)h;
    L.smem = lds_addr(smem);
    const int live_wg = min(kTiles, max(0, (a.m - kTokB * tb + 31) / 32));  // token tiles holding a token
    L.codes_on = (wave & 3) < live_wg;
    L.ex_on = wave < kTiles ? wave < live_wg : wave == kTiles;  // chunk 4: dx and sum |q8|
    L.km = NibMasks{0x000F000Fu, 0x00F000F0u, 0x64006400u};
    asm volatile("" : "+v"(L.km.lo), "+v"(L.km.hi), "+v"(L.km.bias));

    Tiles acc, C;
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[g][tt] = v16f{};

    // the first super-block: codes of step 0, its extras, weights of steps 0
    // and 1 (then each step's requests continue the pattern)
    {
        const uint32_t lv = (uint32_t)lane * 16;
        const uint32_t cso = L.pk0 + (uint32_t)sb0 * L.pk_sb;
        if (L.codes_on) {
#pragma unroll
            for (int i = 0; i < kHalfChunks / kWaves; ++i) {
                const uint32_t c = (uint32_t)(kWaves * i + wave);
                dma16(L.smem + kLdsCodes + c * 1024, lv, L.pack, cso + c * 1024);
            }
        }
        if (L.ex_on)
            dma16(L.smem + kLdsEx + (uint32_t)wave * 1024, lv, L.pack, cso + kPkCodes + (uint32_t)wave * 1024);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint32_t wdst = L.smem + kLdsW + (uint32_t)hf * kWSlot + (uint32_t)grp * kWGrp;
            const uint32_t wso = (uint32_t)sb0 * kBytesQ4_K;
            dma16(wdst + 2048 * th, L.voff_q, L.rows, wso + 16 + 32 * hf);
            dma16(wdst + 2048 * th + 1024, L.voff_q, L.rows, wso + 32 + 32 * hf);
            dma16(wdst + 4096, L.voff_h, L.rows, wso);
        }
    }

    const int tq = 2 * th;  // the wave's first token tile
    const int live = min(2, max(0, live_wg - tq));  // of its two tiles, those holding a token
    // one instance of the loop per live-tile count, so that neither carries
    // the other's registers
    if (live == 2)
        q4k_loop<2>(L, smem, nsb, tq, C, acc);
    else if (live == 1)
        q4k_loop<1>(L, smem, nsb, tq, C, acc);
    else
        q4k_loop<0>(L, smem, nsb, tq, C, acc);
    wait_dma<0>();  // the requests past the end have landed before the LDS is released

    if (a.nsplit > 1) {
        // the wave's four tiles in the order (row half, token tile)
        v16f(&flat)[4] = reinterpret_cast<v16f(&)[4]>(acc);
        if (!split_reduce<4>(flat, a.part, a.cnt, a.nsplit, a.ntiles, tile, z, s_last)) return;
    }

    // bias after the whole dot (the reference's b + dot), then the store
    const int t0 = kTokB * tb + 64 * th;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const int o = rowg + 32 * g + (lane & 31);
        if (o >= a.n_out) continue;
        const float b = a.bias != nullptr ? a.bias[o] : 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + 32 * tt + 8 * (r >> 2) + 4 * h + (r & 3);
                if (t < a.m) a.out[(size_t)t * a.ldo + o] = b + acc[g][tt][r];
            }
        }
    }
}

}  // namespace exq

using namespace exq;

bool gemm_q8_supported(int type, int n_out, int K, int m) {
    return type == kTypeQ4_K && K % kQKK == 0 && n_out > 0 && m >= 1;
}

size_t gemm_q4k_pack_bytes(int m, int K) { return (size_t)(K / kQKK) * pack_tblocks(m) * kPkBlk; }

static int gemm_split(int ntiles, int nblk) {
    static const int max_split = tuning_knob("EXQ_GEMM_SPLIT", kMaxSplit);  // sweep builds only
    return gemm_split_for(ntiles, nblk, max_split < 1 ? 1 : (max_split > kMaxSplit ? kMaxSplit : max_split));
}

static int gemm_tiles(int m, int n_out) { return ((n_out + kRowsB - 1) / kRowsB) * pack_tblocks(m); }

// Partial tiles of the K split (bytes), and the counters' size.
size_t gemm_q4k_part_bytes(int m, int n_out, int K) {
    const int nt = gemm_tiles(m, n_out);
    const int s = gemm_split(nt, K / kQKK);
    return s > 1 ? (size_t)s * nt * kTokB * kRowsB * sizeof(float) : 0;
}
size_t gemm_q4k_counter_bytes() { return kGemmCounters * sizeof(unsigned); }

hipError_t launch_q8k_pack_f32(const float *x, int m, int K, int ldx, uint8_t *pack, hipStream_t st) {
    const int ntb = pack_tblocks(m);
    const unsigned grid = (unsigned)((K / kQKK) * ntb * (kTokB / (kPackWaves * kPackF32Tokens)));
    hipLaunchKernelGGL(q8k_pack_f32_kernel, dim3(grid), dim3(kPackThreads), 0, st, x, ldx, m, K, ntb, pack);
    return hipGetLastError();
}

hipError_t launch_q8k_pack_q8k(const uint8_t *xq, size_t xq_stride, int m, int K, uint8_t *pack, hipStream_t st) {
    const int ntb = pack_tblocks(m);
    const unsigned grid = (unsigned)((K / kQKK) * ntb * (kTokB / kPackWaves));
    hipLaunchKernelGGL(q8k_pack_blocks_kernel, dim3(grid), dim3(kPackThreads), 0, st, xq, xq_stride, m, K, ntb, pack);
    return hipGetLastError();
}

// out = bias + W x over a packed activation (launch_q8k_pack_*); part holds
// gemm_q4k_part_bytes and cnt gemm_q4k_counter_bytes, zero-filled once.
hipError_t launch_gemm_q4k(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *pack,
                           float *part, unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st) {
    if (!gemm_q8_supported(kTypeQ4_K, n_out, K, m)) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)pack & 15u) != 0)
        return hipErrorInvalidValue;
    GmArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.pack = pack;
    a.ntb = pack_tblocks(m);
    const size_t pb = gemm_q4k_pack_bytes(m, K);
    if (pb >= ((size_t)1 << 32) || (size_t)32 * row_bytes >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.pack_bytes = (uint32_t)pb;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.nblk = K / kQKK;
    a.nrb = (n_out + kRowsB - 1) / kRowsB;
    a.ntiles = gemm_tiles(m, n_out);
    a.nsplit = gemm_split(a.ntiles, a.nblk);
    a.part = part;
    a.cnt = cnt;
    if (a.nsplit > 1 && (part == nullptr || cnt == nullptr)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_q4k_kernel, dim3((unsigned)(a.ntiles * a.nsplit)), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
