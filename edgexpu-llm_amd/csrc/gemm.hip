// Prefill GEMM (m >= 64 tokens) of the quantized-weight path on the matrix
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
// Tiling: a workgroup of 8 waves (two per SIMD) computes 128 tokens x 128
// rows; wave w owns rows 32 (w % 4) .. + 31 for tokens 64 (w / 4) .. + 63 (2
// tiles of 32 x 32), and the two chains advance together, each weight
// operand feeding both.  The activation pack of a super-block (69 KiB for the
// 128 tokens) goes global -> LDS with buffer_load ... lds (no registers, no
// address arithmetic) into one of two stages while the other is computed;
// the weight bytes go straight to registers, one super-block ahead.  The two
// stages are distinct LDS objects and the loop names them statically, so the
// compiler sees that a super-block's reads never touch the stage in flight
// (otherwise it waits for every outstanding load before the first read).
// Two waves per SIMD double the LDS read rate a single wave sustains and
// let one wave's VALU work run beside the other's MFMAs.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane l supplies row l % 32
// of A (a token) and column l % 32 of B (a weight row), K slots
// 8 (l / 32) .. + 7; accumulator register r of lane l holds
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], C[token][row].
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "q8k.h"

namespace exq {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource over [base, base + bytes): loads past the end read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Activation pack: per (super-block, tile of 32 tokens) one block of
constexpr int kPkA = 16 * 64 * 16;                      // fp16 codes [K-step][MFMA lane][8]
constexpr int kPkMn = 64 * 16;                          // fp16 bsums [MFMA lane][8]
constexpr int kPkDx = 32 * 4;                           // f32 d per token
constexpr int kPkSq = 32 * 4;                           // int32 sum |q8| per token
constexpr int kPkTile = kPkA + kPkMn + kPkDx + kPkSq;  // 17664 bytes
constexpr int kGmTiles = 4;                             // token tiles per workgroup (128 tokens)
constexpr int kWvTiles = 2;                             // token tiles per wave (64 tokens)
constexpr int kGmRows = 128;                            // rows per workgroup (4 row quarters of 32)
constexpr int kGmThreads = 512;                         // 8 waves: 4 row quarters x 2 token halves
constexpr int kGmStage = kGmTiles * kPkTile;            // 70656 bytes = 69 KiB
constexpr int kGmChunks = kGmStage / 1024;              // 1 KiB DMA chunks per stage
constexpr int kGmLds = 2 * kGmStage;                    // 141312 bytes
static_assert(kGmStage % 1024 == 0, "whole 1 KiB DMA chunks");
static_assert(kGmLds <= 160 * 1024, "two activation stages in the gfx950 LDS");
// largest sum |q8| of a token for which one chain of 256 products is exact:
// 17753 * 945 < 2^24
constexpr int kExactSqMax = 16777215 / 945;

// --------------------------------------------------------------- packing

// Writes one token's super-block into the pack from the codes a lane owns
// (elements 4l .. 4l+3), its 16-element sum (lanes 4i), d and sum |q8|.
__device__ __forceinline__ uint32_t h2_bits(int lo, int hi) {
    const _Float16 l = (_Float16)(float)lo, h = (_Float16)(float)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

__device__ __forceinline__ void pack_store(uint8_t *tile, int tl, int lane, const int q[4], int bsum, float d,
                                           int sq) {
    const int j = lane >> 4;                  // 64-element chunk = 32-byte qs group
    const int nib = (lane >> 3) & 1;          // elements 32..63 of the chunk: high nibbles
    const int s = 8 * (j & 1) + (lane & 7);   // K-step
    const int L = tl + 32 * (j >> 1);         // MFMA lane
    uint8_t *dst = tile + s * 1024 + L * 16;
    *reinterpret_cast<uint32_t *>(dst + 4 * nib) = h2_bits(q[0], q[2]);
    *reinterpret_cast<uint32_t *>(dst + 8 + 4 * nib) = h2_bits(q[1], q[3]);
    if ((lane & 3) == 0) {
        const int i = lane >> 2;  // bsum index
        const _Float16 b = (_Float16)(float)bsum;
        *reinterpret_cast<uint16_t *>(tile + kPkA + (tl + 32 * (i >> 3)) * 16 + (i & 7) * 2) =
            __builtin_bit_cast(uint16_t, b);
    }
    if (lane == 0) {
        *reinterpret_cast<float *>(tile + kPkA + kPkMn + 4 * tl) = d;
        *reinterpret_cast<int *>(tile + kPkA + kPkMn + kPkDx + 4 * tl) = sq;
    }
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One wavefront per (token, super-block) of the padded token range: the
// Q8_K quantization (bit-identical to quantize_q8_k_kernel) written in pack
// order; tokens past m get zero codes and d = 0.
__global__ __launch_bounds__(256) void q8k_pack_f32_kernel(const float *__restrict__ x, int m, int K, int ldx,
                                                           int mp, uint8_t *__restrict__ pack) {
    const int nb = K / kQKK;
    const int lane = threadIdx.x & 63;
    const long long g = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (g >= (long long)mp * nb) return;  // wavefront-uniform
    const int t = (int)(g % mp), sb = (int)(g / mp);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < m) v = *reinterpret_cast<const float4 *>(x + (size_t)t * ldx + (size_t)sb * kQKK + lane * 4);
    const Q8KLane r = q8k_quantize_lane(v, lane);
    int bsum = r.sum4;
    bsum += __shfl_xor(bsum, 1, 64);
    bsum += __shfl_xor(bsum, 2, 64);
    const int sq = wave_sum(abs(r.q[0]) + abs(r.q[1]) + abs(r.q[2]) + abs(r.q[3]));
    uint8_t *tile = pack + ((size_t)sb * (mp / 32) + (t >> 5)) * kPkTile;
    pack_store(tile, t & 31, lane, r.q, bsum, r.d, sq);
}

// The same pack from Q8_K block bytes already in memory (token t at
// xq + t * xq_stride): the block's own d, codes and 16-element sums.
__global__ __launch_bounds__(256) void q8k_pack_q8k_kernel(const uint8_t *__restrict__ xq, size_t xq_stride, int m,
                                                           int K, int mp, uint8_t *__restrict__ pack) {
    const int nb = K / kQKK;
    const int lane = threadIdx.x & 63;
    const long long g = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (g >= (long long)mp * nb) return;
    const int t = (int)(g % mp), sb = (int)(g / mp);
    int q[4] = {0, 0, 0, 0};
    int bsum = 0;
    float d = 0.0f;
    if (t < m) {
        const uint8_t *blk = xq + (size_t)t * xq_stride + (size_t)sb * kBytesQ8_K;
        const uint32_t w = ldg4(blk + 4 + 4 * lane);
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = (int)(int8_t)((w >> (8 * e)) & 0xffu);
        d = __uint_as_float(ldg4(blk));
        const int i = lane >> 2;  // this lane group's 16-element sum (int16 at 260 + 2i)
        if ((lane & 3) == 0) bsum = (int)(int16_t)((ldg4(blk + 260 + 4 * (i >> 1)) >> (16 * (i & 1))) & 0xffffu);
    }
    const int sq = wave_sum(abs(q[0]) + abs(q[1]) + abs(q[2]) + abs(q[3]));
    uint8_t *tile = pack + ((size_t)sb * (mp / 32) + (t >> 5)) * kPkTile;
    pack_store(tile, t & 31, lane, q, bsum, d, sq);
}

// ------------------------------------------------------------------ GEMM

struct GmArgs {
    const uint8_t *w;     // [n_out][row_bytes] Q4_K
    size_t row_bytes;
    const uint8_t *pack;  // [nblk][mtp][kPkTile]
    uint32_t pack_bytes;  // < 4 GiB (checked at launch)
    int mtp;              // token tiles in the pack (a multiple of kGmTiles)
    const float *bias;    // [n_out] or null
    float *out;           // [m][ldo]
    int ldo, m, n_out, nblk;
    int nrb;              // row blocks of kGmRows
    int ntiles;           // nrb * token blocks
};

// This lane's bytes of one super-block: the 16-byte header and its half
// (64 bytes) of the nibbles.
struct WRaw {
    v4u hd;
    v4u q[4];
};

// This lane's bytes of one super-block, global -> registers (rows past n_out
// lie past the resource and read as zeros): header at 0, nibbles at
// 16 + 64 h .. + 63 of the row's block.
__device__ __forceinline__ void load_w(__amdgpu_buffer_rsrc_t rows, uint32_t voff, int h, int sb, WRaw &r) {
    const uint32_t so = (uint32_t)sb * kBytesQ4_K;
    r.hd = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rows, voff, so, 0));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r.q[i] = __builtin_bit_cast(
            v4u, __builtin_amdgcn_raw_buffer_load_b128(rows, voff + 16 + 64 * h + 16 * i, so, 0));
}

// Constants of one super-block for this lane's row and sub-blocks 4h .. 4h+3:
// the packed-FMA multipliers / addends for the low- and high-nibble weights
// of sub-block pairs (4h, 4h+1) and (4h+2, 4h+3), the min operand, d, -dmin.
struct WConst {
    h2 mlo[2], alo[2], mhi[2], ahi[2];
    v8h bmn;
    float dd, ndm;
};

__device__ __forceinline__ WConst w_const(const v4u hd, int h) {
    // get_scale_min_k4 (src/gguf_quant.c:212-220) for four sub-blocks at once
    const uint32_t w0 = hd[1], w1 = hd[2], w2 = hd[3];
    const uint32_t sel = 0u - (uint32_t)h;  // all ones for sub-blocks 4..7
    const uint32_t sc4 = ((w0 & 0x3f3f3f3fu) & ~sel) | (((w2 & 0x0f0f0f0fu) | ((w0 >> 2) & 0x30303030u)) & sel);
    const uint32_t m4 = ((w1 & 0x3f3f3f3fu) & ~sel) | ((((w2 >> 4) & 0x0f0f0f0fu) | ((w1 >> 2) & 0x30303030u)) & sel);
    WConst c;
    c.dd = f16_bits_to_f32(hd[0] & 0xffffu);
    c.ndm = -f16_bits_to_f32(hd[0] >> 16);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const float lo = (float)((sc4 >> (16 * p)) & 0xffu), hi = (float)((sc4 >> (16 * p + 8)) & 0xffu);
        const _Float16 ml = (_Float16)lo, al = (_Float16)(-1024.0f * lo);
        const _Float16 mh = (_Float16)(0.0625f * hi), ah = (_Float16)(-64.0f * hi);
        c.mlo[p] = h2{ml, ml};
        c.alo[p] = h2{al, al};
        c.mhi[p] = h2{mh, mh};
        c.ahi[p] = h2{ah, ah};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const _Float16 mv = (_Float16)(float)((m4 >> (8 * k)) & 0xffu);
        c.bmn[2 * k] = mv;
        c.bmn[2 * k + 1] = mv;
    }
    return c;
}

// Weight operand of K-step s (qs dword s of this lane's 64 bytes; s is a
// constant once the K-step loops are unrolled).
struct NibMasks {
    uint32_t lo, hi, bias;  // 0x000F000F, 0x00F000F0, 0x64006400, held in VGPRs
};

__device__ __forceinline__ v8h w_operand(const WRaw &r, const WConst &c, const NibMasks &k, int s) {
    const int p = s >> 3;
    const uint32_t u = r.q[s >> 2][s & 3];
    const uint32_t u8 = u >> 8;
    const h2 y0 = __builtin_bit_cast(h2, (u & k.lo) | k.bias);
    const h2 y1 = __builtin_bit_cast(h2, (u & k.hi) | k.bias);
    const h2 y2 = __builtin_bit_cast(h2, (u8 & k.lo) | k.bias);
    const h2 y3 = __builtin_bit_cast(h2, (u8 & k.hi) | k.bias);
    const h2 b0 = __builtin_elementwise_fma(y0, c.mlo[p], c.alo[p]);
    const h2 b1 = __builtin_elementwise_fma(y1, c.mhi[p], c.ahi[p]);
    const h2 b2 = __builtin_elementwise_fma(y2, c.mlo[p], c.alo[p]);
    const h2 b3 = __builtin_elementwise_fma(y3, c.mhi[p], c.ahi[p]);
    return v8h{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

__device__ __forceinline__ v16f mfma(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v8h lds_v8h(const uint8_t *p) { return *reinterpret_cast<const v8h *>(p); }

// K-steps S0 .. S1-1 of one super-block for the wave's 2 token tiles: two
// independent accumulator chains advance together, so each K-step issues 2
// MFMAs behind one weight operand (built just in time) and the next K-step's
// activation operands are read while they run.
template <int S0, int S1>
__device__ __forceinline__ void sb_chains(const uint8_t *stage, int lane, const WRaw &r, const WConst &c,
                                          const NibMasks &k, v16f (&C)[kWvTiles]) {
    v8h a[kWvTiles];
#pragma unroll
    for (int tt = 0; tt < kWvTiles; ++tt) {
        C[tt] = v16f{};
        a[tt] = lds_v8h(stage + tt * kPkTile + S0 * 1024 + lane * 16);
    }
#pragma unroll
    for (int s = S0; s < S1; ++s) {
        const v8h b = w_operand(r, c, k, s);
        v8h an[kWvTiles];
        if (s + 1 < S1) {
#pragma unroll
            for (int tt = 0; tt < kWvTiles; ++tt) an[tt] = lds_v8h(stage + tt * kPkTile + (s + 1) * 1024 + lane * 16);
        }
#pragma unroll
        for (int tt = 0; tt < kWvTiles; ++tt) C[tt] = mfma(a[tt], b, C[tt]);
        if (s + 1 < S1) {
#pragma unroll
            for (int tt = 0; tt < kWvTiles; ++tt) a[tt] = an[tt];
        }
        // one K-step per scheduling region: the next step's operand reads
        // stay one step ahead instead of being hoisted (and held) further
        __builtin_amdgcn_sched_barrier(0);
    }
}

// acc += dx * (C * d - mn * dmin) for the wave's tiles (MN = false: acc += dx * C * d);
// the next tile's min-term MFMA is issued before this tile's VALU work.
template <bool MN>
__device__ __forceinline__ void sb_combine(const uint8_t *stage, int lane, const WConst &c, const v16f (&C)[kWvTiles],
                                           v16f (&acc)[kWvTiles]) {
    const int h = lane >> 5;
    v16f mn{};
    if (MN) mn = mfma(lds_v8h(stage + kPkA + lane * 16), c.bmn, v16f{});
#pragma unroll
    for (int tt = 0; tt < kWvTiles; ++tt) {
        const uint8_t *tile = stage + tt * kPkTile;
        v16f mn_next{};
        if (MN && tt + 1 < kWvTiles) mn_next = mfma(lds_v8h(tile + kPkTile + kPkA + lane * 16), c.bmn, v16f{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 dx = *reinterpret_cast<const float4 *>(tile + kPkA + kPkMn + 4 * (8 * i + 4 * h));
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * i + e;
                float v = C[tt][r] * c.dd;
                if (MN) v = __builtin_fmaf(mn[r], c.ndm, v);
                acc[tt][r] = __builtin_fmaf(v, dxs[e], acc[tt][r]);
            }
        }
        if (MN) mn = mn_next;
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Wavefront maximum through DPP row shifts and broadcasts (no LDS round trips).
__device__ __forceinline__ int wave_max_dpp(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));  // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));  // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// The workgroup's activation pack of one super-block (at byte soff of the
// pack), global -> LDS.
__device__ __forceinline__ void stage_pack(__amdgpu_buffer_rsrc_t pack, uint32_t soff, uint8_t *dst, int wave,
                                           int lane) {
    static_assert(kGmChunks == 8 * 8 + 5, "8 chunks per wave and one more for waves 0..4");
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int ch = 8 * i + wave;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(pack, (lds_void *)(dst + ch * 1024), 16, lane * 16,
                                                 soff + ch * 1024, 0, 0);
    }
    if (wave < 5)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(pack, (lds_void *)(dst + (64 + wave) * 1024), 16, lane * 16,
                                                 soff + (64 + wave) * 1024, 0, 0);
}


// Per-wave state of the main loop.
struct GmLoop {
    __amdgpu_buffer_rsrc_t pack, rows;
    uint32_t pk0, pk_sb, woff;
    NibMasks km;
    int lane, wave, h, th;
};

// One super-block from stage `cur` while the next one (if `more`) is
// requested into `nxt` and the next weights into wn.  cur and nxt are
// distinct LDS objects, so the compiler sees that the requests in flight do
// not touch what this super-block reads and needs no wait for them.
__device__ __forceinline__ void sb_step(const GmLoop &L, int sb, bool more, const uint8_t *cur, uint8_t *nxt,
                                        const WRaw &wr, WRaw &wn, v16f (&acc)[kWvTiles]) {
    if (more) {
        stage_pack(L.pack, L.pk0 + (uint32_t)(sb + 1) * L.pk_sb, nxt, L.wave, L.lane);
        load_w(L.rows, L.woff, L.h, sb + 1, wn);
    }
    const uint8_t *mine = cur + (kWvTiles * L.th) * kPkTile;  // this wave's two token tiles
    const WConst c = w_const(wr.hd, L.h);
    // the exactness bound of one chain over the wave's 64 tokens
    const int sq = *reinterpret_cast<const int *>(mine + (L.lane >> 5) * kPkTile + kPkA + kPkMn + kPkDx +
                                                   4 * (L.lane & 31));
    const int sqmax = wave_max_dpp(sq);
    v16f C[kWvTiles];
    if (sqmax <= kExactSqMax) {
        sb_chains<0, 16>(mine, L.lane, wr, c, L.km, C);
        sb_combine<true>(mine, L.lane, c, C, acc);
    } else {
        sb_chains<0, 8>(mine, L.lane, wr, c, L.km, C);
        sb_combine<true>(mine, L.lane, c, C, acc);
        sb_chains<8, 16>(mine, L.lane, wr, c, L.km, C);
        sb_combine<false>(mine, L.lane, c, C, acc);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the next stage and weights have landed
    __syncthreads();                // and every wave is done with this stage
}

__global__ __launch_bounds__(kGmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_q4k_kernel(GmArgs a) {
    // two activation stages: kGmLds bytes of LDS
    __shared__ __align__(16) uint8_t stage0[kGmStage];
    __shared__ __align__(16) uint8_t stage1[kGmStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rq = wave & 3, th = wave >> 2;  // row quarter, token half
    const int h = lane >> 5;

    // workgroups sharing a row block are a multiple of nrb apart; with nrb a
    // multiple of 8 they land on one XCD and share its L2 copy of the weights
    const int rb = (int)blockIdx.x % a.nrb, tb = (int)blockIdx.x / a.nrb;
    const int sb0 = 0, sb1 = a.nblk;

    const int row0 = rb * kGmRows + 32 * rq;
    const int row = min(row0 + (lane & 31), a.n_out - 1);
    GmLoop L;
    L.lane = lane;
    L.wave = wave;
    L.h = h;
    L.th = th;
    L.pk_sb = (uint32_t)a.mtp * kPkTile;
    L.pk0 = (uint32_t)(kGmTiles * tb) * kPkTile;
    L.pack = buffer_rsrc(a.pack, a.pack_bytes);
    const int live_rows = min(32, a.n_out - row0);  // rows past n_out lie past the resource (zeros)
    L.rows = buffer_rsrc(a.w + (size_t)min(row0, a.n_out - 1) * a.row_bytes,
                         live_rows > 0 ? (uint32_t)live_rows * (uint32_t)a.row_bytes : 0u);
    L.woff = (uint32_t)(lane & 31) * (uint32_t)a.row_bytes;
    L.km = NibMasks{0x000F000Fu, 0x00F000F0u, 0x64006400u};
    asm volatile("" : "+v"(L.km.lo), "+v"(L.km.hi), "+v"(L.km.bias));

    v16f acc[kWvTiles];
#pragma unroll
    for (int tt = 0; tt < kWvTiles; ++tt) acc[tt] = v16f{};

    WRaw w0, w1;
    stage_pack(L.pack, L.pk0 + (uint32_t)sb0 * L.pk_sb, stage0, wave, lane);
    load_w(L.rows, L.woff, h, sb0, w0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // two super-blocks per trip: each step names its stages and weight
    // registers statically
    for (int sb = sb0; sb < sb1; sb += 2) {
        sb_step(L, sb, sb + 1 < sb1, stage0, stage1, w0, w1, acc);
        if (sb + 1 >= sb1) break;
        sb_step(L, sb + 1, sb + 2 < sb1, stage1, stage0, w1, w0, acc);
    }

    // bias after the whole dot (the reference's b + dot), then the store
    const int o = row0 + (lane & 31);
    const float b = a.bias != nullptr ? a.bias[row] : 0.0f;
    if (o >= a.n_out) return;
#pragma unroll
    for (int tt = 0; tt < kWvTiles; ++tt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = kGmTiles * 32 * tb + 64 * th + 32 * tt + 8 * (r >> 2) + 4 * h + (r & 3);
            if (t < a.m) a.out[(size_t)t * a.ldo + o] = b + acc[tt][r];
        }
    }
}

}  // namespace exq

using namespace exq;

bool gemm_q8_supported(int type, int n_out, int K, int m) {
    return type == kTypeQ4_K && K % kQKK == 0 && n_out > 0 && m >= 1;
}

// Token tiles of the activation pack for m tokens (whole workgroup blocks).
static int pack_tiles(int m) { return (m + 32 * kGmTiles - 1) / (32 * kGmTiles) * kGmTiles; }

size_t gemm_q4k_pack_bytes(int m, int K) { return (size_t)(K / kQKK) * pack_tiles(m) * kPkTile; }

static int gemm_tiles(int m, int n_out) {
    return ((n_out + kGmRows - 1) / kGmRows) * (pack_tiles(m) / kGmTiles);
}

hipError_t launch_q8k_pack_f32(const float *x, int m, int K, int ldx, uint8_t *pack, hipStream_t st) {
    const int mp = pack_tiles(m) * 32;
    const long long threads = (long long)mp * (K / kQKK) * 64;
    hipLaunchKernelGGL(q8k_pack_f32_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, x, m, K, ldx,
                       mp, pack);
    return hipGetLastError();
}

hipError_t launch_q8k_pack_q8k(const uint8_t *xq, size_t xq_stride, int m, int K, uint8_t *pack, hipStream_t st) {
    const int mp = pack_tiles(m) * 32;
    const long long threads = (long long)mp * (K / kQKK) * 64;
    hipLaunchKernelGGL(q8k_pack_q8k_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, xq, xq_stride,
                       m, K, mp, pack);
    return hipGetLastError();
}

// out = bias + W x over a packed activation (launch_q8k_pack_*).
hipError_t launch_gemm_q4k(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *pack,
                           const float *bias, float *out, int ldo, hipStream_t st) {
    if (!gemm_q8_supported(kTypeQ4_K, n_out, K, m)) return hipErrorInvalidValue;
    if (((uintptr_t)w & 15u) != 0 || (row_bytes & 15u) != 0 || ((uintptr_t)pack & 15u) != 0)
        return hipErrorInvalidValue;
    GmArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.pack = pack;
    a.mtp = pack_tiles(m);
    const size_t pb = gemm_q4k_pack_bytes(m, K);
    if (pb >= ((size_t)1 << 32) || (size_t)kGmRows * row_bytes >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.pack_bytes = (uint32_t)pb;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.nblk = K / kQKK;
    a.nrb = (n_out + kGmRows - 1) / kGmRows;
    a.ntiles = gemm_tiles(m, n_out);
    hipLaunchKernelGGL(gemm_q4k_kernel, dim3((unsigned)a.ntiles), dim3(kGmThreads), 0, st, a);
    return hipGetLastError();
}
