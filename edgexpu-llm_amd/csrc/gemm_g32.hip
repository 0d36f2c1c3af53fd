// Prefill GEMM (m >= 16 tokens) of the 32-element-block formats Q8_0, Q4_0
// and Q5_0 against Q8_0 activations on the matrix cores, every block integer
// exact:
//   out[t][o] = bias[o] + sum_g dw[o][g] * dx[t][g] * sum_{32} q * q8
// -- edgexpu_cpu_linear_quant_batch (src/cpu_kernel.c:605-631) with the block
// dots dot_q8_0_q8_0 / dot_q4_0_q8_0 / dot_q5_0_q8_0 (src/gguf_dot_q8.c:
// 436-601; q = qs for Q8_0, nibble - 8 for Q4_0, nibble + 16 * qh bit - 16
// for Q5_0) and the activation quantizer edgexpu_gguf_quantize_q8_0
// (src/gguf_dot_q8.c:269-324).
//
// Exactness: |q| <= 128 and |q8| <= 128 are fp16 integers, so a block's 32
// products chained through two v_mfma_f32_32x32x16_f16 stay below
// 32 * 128 * 128 < 2^24: the block integer is exact.  Each block is then
// combined on its own, acc += (C * dw) * dx (two VALU instructions per output
// and block: the cost that bounds this kernel, not the matrix cores).
//
// Weights: Q8_0 / Q4_0 / Q5_0 blocks (34 / 18 / 22 B) are 2-byte aligned, so
// a per-call repack (g32_repack_kernel) rewrites every row as aligned
// records of 128 elements (4 blocks, a K step):
//   q   [lane half 2][K-step 8][8 B]  q + 128 of elements 16 s + 8 h .. + 7
//   dw  [4] f32                       the blocks' d (0 past the row's end)
// 144 B per 128 weights; the row is padded to whole records.  The activation
// pack (g32_pack_kernel) holds per (record, 128-token block) the Q8_0 codes
// as fp16 in the same K order, [K-step 8][token tile 4][MFMA lane 64][8 fp16]
// (32 KiB), then dx [block 4][token 128] f32 (2 KiB).
//
// Tiling and pipeline as the K-quant GEMM (gemm_kq.hip): 8 waves, 128 rows x
// 128 tokens per workgroup, wave w owns rows 32 (w % 4) .. + 31 for tokens
// 64 (w / 4) .. + 63; LDS DMA only, codes one step ahead (2 slots of 34 KiB),
// weights two steps ahead (3 slots of 24 KiB); one barrier per step.  Inside
// a step the block-g MFMAs run while block g-1 is combined.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "gemm_common.h"

namespace exq {

constexpr int kG32Rec = 144;           // repacked bytes per row and 128 weights
constexpr int kG32Step = 128;          // K elements per step
constexpr int kG32PkDx = 4 * kTokB * 4;           // 2 KiB
constexpr int kG32PkBlk = kPkHalf + kG32PkDx;     // 34 KiB per (step, token block)
constexpr int kG32RowsB = 128;
constexpr int kG32MaxSplit = 8;
constexpr int kG32GrpBytes = 6 * 1024;  // per row group and step: q 4 KiB, dw 2 x 1 KiB
constexpr int kG32WSlot = 4 * kG32GrpBytes;
constexpr int kG32WSlots = 3;
constexpr int kG32LdsCodes = 0;
constexpr int kG32LdsW = 2 * kG32PkBlk;
constexpr int kG32LdsLast = kG32LdsW + kG32WSlots * kG32WSlot;
constexpr int kG32LdsBytes = kG32LdsLast + 16;
static_assert(kG32LdsBytes <= 160 * 1024, "the LDS rings fit the gfx950 LDS");

__host__ __device__ constexpr int g32_steps(int K) { return (K + kG32Step - 1) / kG32Step; }

// ----------------------------------------------------------------- repack

// Bit b of the low 4 bits of x into byte b.
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
    return (x & 1u) | ((x & 2u) << 7) | ((x & 4u) << 14) | ((x & 8u) << 21);
}

constexpr int kG32RepackRecs = 32;  // records per workgroup, 8 threads each

// Thread t of a record writes q chunk t: block p = t % 4 of the record,
// lane half h = t / 4, elements 8 h .. 8 h + 7 and 16 + 8 h .. + 7 of the
// block (K-steps 2p and 2p + 1), biased by +128; thread 0 also the dw chunk.
template <int TYPE>
__global__ __launch_bounds__(256) void g32_repack_kernel(const uint8_t *__restrict__ w, int nb, int nst,
                                                         long long nrec, uint8_t *__restrict__ rw) {
    constexpr int kB = TYPE == kTypeQ8_0 ? kBytesQ8_0 : (TYPE == kTypeQ4_0 ? kBytesQ4_0 : kBytesQ5_0);
    const long long r = (long long)blockIdx.x * kG32RepackRecs + (threadIdx.x >> 3);
    if (r >= nrec) return;
    const int t = threadIdx.x & 7;
    const long long row = r / nst;
    const int st = (int)(r % nst);
    const int p = t & 3, h = t >> 2;
    const int blkno = 4 * st + p;
    const uint8_t *rowp = w + (size_t)row * nb * kB;
    uint8_t *dst = rw + (size_t)r * kG32Rec;
    uint2 lo = make_uint2(0x80808080u, 0x80808080u), hi = lo;
    if (blkno < nb) {
        const uint8_t *blk = rowp + (size_t)blkno * kB;
        if (TYPE == kTypeQ8_0) {
            const uint2 a = ldg8(blk + 2 + 8 * h), b = ldg8(blk + 18 + 8 * h);
            lo = make_uint2(a.x ^ 0x80808080u, a.y ^ 0x80808080u);
            hi = make_uint2(b.x ^ 0x80808080u, b.y ^ 0x80808080u);
        } else if (TYPE == kTypeQ4_0) {
            const uint2 v = ldg8(blk + 2 + 8 * h);  // elements 8h + b (lo nibble), 16 + 8h + b (hi)
            lo = make_uint2((v.x & 0x0F0F0F0Fu) + 0x78787878u, (v.y & 0x0F0F0F0Fu) + 0x78787878u);
            hi = make_uint2(((v.x >> 4) & 0x0F0F0F0Fu) + 0x78787878u, ((v.y >> 4) & 0x0F0F0F0Fu) + 0x78787878u);
        } else {
            const uint32_t qh = ldg4(blk + 2);
            const uint2 v = ldg8(blk + 6 + 8 * h);
            const uint32_t bl = qh >> (8 * h), bh = qh >> (16 + 8 * h);
            lo = make_uint2((v.x & 0x0F0F0F0Fu) + (spread4(bl) << 4) + 0x70707070u,
                            (v.y & 0x0F0F0F0Fu) + (spread4(bl >> 4) << 4) + 0x70707070u);
            hi = make_uint2(((v.x >> 4) & 0x0F0F0F0Fu) + (spread4(bh) << 4) + 0x70707070u,
                            ((v.y >> 4) & 0x0F0F0F0Fu) + (spread4(bh >> 4) << 4) + 0x70707070u);
        }
    }
    *reinterpret_cast<uint4 *>(dst + 64 * h + 16 * p) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    if (t == 0) {
        float d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 4 * st + i;
            d[i] = b < nb ? f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(rowp + (size_t)b * kB)) : 0.0f;
        }
        *reinterpret_cast<float4 *>(dst + 128) = make_float4(d[0], d[1], d[2], d[3]);
    }
}

// ------------------------------------------------------------------- pack

// One thread per (token, 4 elements): 8 threads hold a Q8_0 block, 32 a
// record's 128 elements, 8 tokens per workgroup.  F32IN: quantize exactly as
// quantize_q8_0_kernel (amax over the block, d = fp16(amax / 127), q =
// saturate(rint(x * 127 / amax))); otherwise read the Q8_0 block bytes.
// Tokens past m and elements past K get code 0 and dx 0.
template <bool F32IN>
__global__ __launch_bounds__(256) void g32_pack_kernel(const float *__restrict__ x, const uint8_t *__restrict__ xq,
                                                       size_t xq_stride, int m, int K, int nst, int ntb,
                                                       uint8_t *__restrict__ pack) {
    const int lt = threadIdx.x & 31;
    const long long tg = (long long)blockIdx.x * 8 + (threadIdx.x >> 5);  // (record, token) pairs
    const int tpad = ntb * kTokB;
    const int st = (int)(tg / tpad), t = (int)(tg % tpad);
    const int p = lt >> 3, part = lt & 7;
    const int e0 = kG32Step * st + 32 * p + 4 * part;
    const bool live = t < m && e0 < K;  // whole blocks: the 8 lanes of a block agree
    uint32_t word = 0;
    float dx = 0.0f;
    if (F32IN) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (live) v = *reinterpret_cast<const float4 *>(x + (size_t)t * K + e0);
        float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        dx = f16_bits_to_f32(f32_to_f16_rne(amax / 127.0f));
        const float xs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = rintf(xs[e] * id);
            int q = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT32_MIN;
            q = q < -128 ? -128 : (q > 127 ? 127 : q);
            word |= (uint32_t)(q & 0xff) << (8 * e);
        }
    } else if (live) {
        const uint8_t *blk = xq + (size_t)t * xq_stride + (size_t)(e0 >> 5) * kBytesQ8_0;
        word = ldg4(blk + 2 + 4 * part);
        dx = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
    }
    const int tb = t / kTokB, tt = (t % kTokB) / 32, tl = t % 32;
    uint8_t *blk = pack + ((size_t)st * ntb + tb) * kG32PkBlk;
    const int ee = 32 * p + 4 * part;  // element within the record
    const int s = ee >> 4, h = (ee >> 3) & 1, k = ee & 7;
    *reinterpret_cast<uint2 *>(blk + s * 4096 + tt * 1024 + (tl + 32 * h) * 16 + 2 * k) =
        make_uint2(h2_bits(sbyte(word, 0), sbyte(word, 1)), h2_bits(sbyte(word, 2), sbyte(word, 3)));
    if (part == 0) *reinterpret_cast<float *>(blk + kPkHalf + 4 * (kTokB * p + (t % kTokB))) = live ? dx : 0.0f;
}

// ------------------------------------------------------------------- GEMM

struct G32Args {
    const uint8_t *rw;    // [n_out][nst][kG32Rec]
    uint32_t rstride;
    const uint8_t *pack;  // [nst][ntb][kG32PkBlk]
    uint32_t pack_bytes;
    int ntb;
    const float *bias;
    float *out;
    int ldo, m, n_out, nst;
    int nrb, ntiles, nsplit;
    float *part;
    unsigned *cnt;
};

struct G32Loop {
    v4u pack, rows;
    uint32_t pk0, pk_st;
    uint32_t voff_q, voff_dw;
    uint32_t smem;
    int lane, wave, grp, th, st0, stlast;
    bool codes_on;
};

constexpr int kG32WLoads = 3;

// Step s requests the codes of step s + 1 (4 DMAs, waves whose token tile
// holds a token) and their dx (waves 0 and 1), then the weights of step
// s + 2 (3 DMAs: token-half 0 waves q pieces 0, 1 and the dw copy A, token-
// half 1 waves q pieces 2, 3 and dw copy B).  The weights are always the last
// 3, so a wait for vmcnt(3) covers everything else.
__device__ __forceinline__ void g32_step_requests(const G32Loop &L, int s) {
    const uint32_t lv = (uint32_t)L.lane * 16;
    const int s1 = s + 1;
    const int stc = min(L.st0 + s1, L.stlast);
    const uint32_t cdst = L.smem + kG32LdsCodes + (uint32_t)(s1 & 1) * kG32PkBlk;
    const uint32_t cso = L.pk0 + (uint32_t)stc * L.pk_st;
    if (L.codes_on) {
#pragma unroll
        for (int i = 0; i < kHalfChunks / kWaves; ++i) {
            const uint32_t ch = (uint32_t)(kWaves * i + L.wave);
            dma16(cdst + ch * 1024, lv, L.pack, cso + ch * 1024);
        }
    }
    if (L.wave < 2) dma16(cdst + kPkHalf + (uint32_t)L.wave * 1024, lv, L.pack, cso + kPkHalf + (uint32_t)L.wave * 1024);
    const int s2 = s + 2;
    const int stw = min(L.st0 + s2, L.stlast);
    const uint32_t wdst = L.smem + kG32LdsW + (uint32_t)(s2 % kG32WSlots) * kG32WSlot + (uint32_t)L.grp * kG32GrpBytes;
    const uint32_t wso = (uint32_t)stw * kG32Rec;
    dma16(wdst + 2048 * L.th, L.voff_q, L.rows, wso + 32 * L.th);
    dma16(wdst + 2048 * L.th + 1024, L.voff_q, L.rows, wso + 32 * L.th + 16);
    dma16(wdst + 4096 + 1024 * L.th, L.voff_dw, L.rows, wso + 128);
}

// Weight operand of one K-step from its 8 biased bytes: fp16 1024 + b, minus 1152.
__device__ __forceinline__ v8h g32_operand(uint32_t q0, uint32_t q1, uint32_t hi64) {
    h2 pa[2], pb[2];
    bytes_to_h2(q0, hi64, pa);
    bytes_to_h2(q1, hi64, pb);
    const h2 bias = h2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2 b0 = pa[0] + bias, b1 = pa[1] + bias, b2 = pb[0] + bias, b3 = pb[1] + bias;
    return v8h{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

// acc += (C * dw) * dx for block g of the step, the wave's first NT tiles.
template <int NT>
__device__ __forceinline__ void g32_combine(const uint8_t *dxb, int g, int tq, int lane, float dw, const v16f (&C)[2],
                                            v16f (&acc)[2]) {
    const int h = lane >> 5;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 dx = *reinterpret_cast<const float4 *>(dxb + 4 * (kTokB * g + 32 * (tq + tt) + 8 * i + 4 * h));
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * i + e;
                acc[tt][r] = __builtin_fmaf(C[tt][r] * dw, dxs[e], acc[tt][r]);
            }
        }
    }
}

// One step (4 blocks) for a wave with NT live token tiles: its codes at
// cur + tt * 1024 (4 KiB per K-step), the slot's dx at dxb, weight slot `wq`
// (q pieces at wq + 1024 p, the wave's dw copy at wq + 4096 + 1024 th).  Block g's two K-steps run on the
// matrix cores while block g - 1 is combined.
template <int NT>
__device__ __forceinline__ void g32_step(const uint8_t *cur, const uint8_t *dxb, const uint8_t *wq, int lane, int tq,
                                         int th, uint32_t hi64, v16f (&acc)[2]) {
    v4u q[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) q[p] = lds_v4u(wq + 1024 * p + lane * 16);
    const v4u dwv = lds_v4u(wq + 4096 + 1024 * th + lane * 16);
    v8h a[2][NT];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) a[k][tt] = lds_v8h(cur + k * 4096 + tt * 1024 + lane * 16);
    v8h b[2] = {g32_operand(q[0][0], q[0][1], hi64), g32_operand(q[0][2], q[0][3], hi64)};
    v16f C[2], P[2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            C[tt] = mfma(a[0][tt], b[0], v16f{});
            C[tt] = mfma(a[1][tt], b[1], C[tt]);
        }
        if (g + 1 < 4) {
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int tt = 0; tt < NT; ++tt)
                    a[k][tt] = lds_v8h(cur + (2 * (g + 1) + k) * 4096 + tt * 1024 + lane * 16);
            b[0] = g32_operand(q[g + 1][0], q[g + 1][1], hi64);
            b[1] = g32_operand(q[g + 1][2], q[g + 1][3], hi64);
        }
        if (g > 0) g32_combine<NT>(dxb, g - 1, tq, lane, __uint_as_float(dwv[g - 1]), P, acc);
        // per MFMA of the block: the share of the VALU work (the previous
        // block's combination, 32 NT, and the next operands, 16) and 3 DS reads
#pragma unroll
        for (int i = 0; i < 2 * NT; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, (32 * NT + 16) / (2 * NT), 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) P[tt] = C[tt];
    }
    g32_combine<NT>(dxb, 3, tq, lane, __uint_as_float(dwv[3]), P, acc);
}

template <int NT>
__device__ __forceinline__ void g32_loop(const G32Loop &L, uint8_t *smem, int nst, int tq, uint32_t hi64,
                                         v16f (&acc)[2]) {
    for (int j = 0; j < nst; ++j) {
        wait_dma<kG32WLoads>();
        __syncthreads();
        g32_step_requests(L, j);
        if constexpr (NT > 0) {
            const uint8_t *cur = smem + kG32LdsCodes + (j & 1) * kG32PkBlk;
            const uint8_t *wq = smem + kG32LdsW + (j % kG32WSlots) * kG32WSlot + L.grp * kG32GrpBytes;
            g32_step<NT>(cur + tq * 1024, cur + kPkHalf, wq, L.lane, tq, L.th, hi64, acc);
        }
    }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_g32_kernel(G32Args a) {
    __shared__ __align__(16) uint8_t smem[kG32LdsBytes];
    int *s_last = reinterpret_cast<int *>(smem + kG32LdsLast);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int grp = wave & 3, th = wave >> 2;

    const int tile = (int)blockIdx.x % a.ntiles, z = (int)blockIdx.x / a.ntiles;
    const int rb = tile % a.nrb, tb = tile / a.nrb;
    const int st0 = (int)((long long)a.nst * z / a.nsplit);
    const int st1 = (int)((long long)a.nst * (z + 1) / a.nsplit);

    const int rowg = rb * kG32RowsB + 32 * grp;
    G32Loop L;
    L.lane = lane;
    L.wave = wave;
    L.grp = grp;
    L.th = th;
    L.st0 = st0;
    L.stlast = st1 - 1;
    L.pk_st = (uint32_t)a.ntb * kG32PkBlk;
    L.pk0 = (uint32_t)tb * kG32PkBlk;
    L.pack = rsrc_words(a.pack, a.pack_bytes);
    const int live_rows = min(32, a.n_out - rowg);
    L.rows = rsrc_words(a.rw + (size_t)min(rowg, a.n_out - 1) * a.rstride,
                        live_rows > 0 ? (uint32_t)live_rows * a.rstride : 0u);
    L.voff_q = (uint32_t)(lane & 31) * a.rstride + 64u * (uint32_t)h;
    L.voff_dw = (uint32_t)(lane & 31) * a.rstride;
    L.smem = lds_addr(smem);
    const int live_wg = min(kTiles, max(0, (a.m - kTokB * tb + 31) / 32));
    L.codes_on = (wave & 3) < live_wg;
    uint32_t hi64 = 0x64646464u;
    asm volatile("" : "+v"(hi64));

    v16f acc[2];
    acc[0] = v16f{};
    acc[1] = v16f{};

    {
        const uint32_t lv = (uint32_t)lane * 16;
        const uint32_t cso = L.pk0 + (uint32_t)st0 * L.pk_st;
        if (L.codes_on) {
#pragma unroll
            for (int i = 0; i < kHalfChunks / kWaves; ++i) {
                const uint32_t c = (uint32_t)(kWaves * i + wave);
                dma16(L.smem + kG32LdsCodes + c * 1024, lv, L.pack, cso + c * 1024);
            }
        }
        if (wave < 2) dma16(L.smem + kG32LdsCodes + kPkHalf + (uint32_t)wave * 1024, lv, L.pack,
                            cso + kPkHalf + (uint32_t)wave * 1024);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int stw = min(st0 + k, L.stlast);
            const uint32_t wdst = L.smem + kG32LdsW + (uint32_t)k * kG32WSlot + (uint32_t)grp * kG32GrpBytes;
            const uint32_t wso = (uint32_t)stw * kG32Rec;
            dma16(wdst + 2048 * th, L.voff_q, L.rows, wso + 32 * th);
            dma16(wdst + 2048 * th + 1024, L.voff_q, L.rows, wso + 32 * th + 16);
            dma16(wdst + 4096 + 1024 * th, L.voff_dw, L.rows, wso + 128);
        }
    }

    const int tq = 2 * th;
    const int live = min(2, max(0, live_wg - tq));
    const int nst = st1 - st0;
    if (live == 2)
        g32_loop<2>(L, smem, nst, tq, hi64, acc);
    else if (live == 1)
        g32_loop<1>(L, smem, nst, tq, hi64, acc);
    else
        g32_loop<0>(L, smem, nst, tq, hi64, acc);
    wait_dma<0>();

    if (a.nsplit > 1 && !split_reduce<2>(acc, a.part, a.cnt, a.nsplit, a.ntiles, tile, z, s_last)) return;

    const int o = rowg + (lane & 31);
    if (o >= a.n_out) return;
    const float b = a.bias != nullptr ? a.bias[o] : 0.0f;
    const int t0 = kTokB * tb + 64 * th;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 32 * tt + 8 * (r >> 2) + 4 * h + (r & 3);
            if (t < a.m) a.out[(size_t)t * a.ldo + o] = b + acc[tt][r];
        }
    }
}

}  // namespace exq

using namespace exq;

bool gemm_g32_supported(int type, int n_out, int K, int m) {
    return (type == kTypeQ8_0 || type == kTypeQ4_0 || type == kTypeQ5_0) && K % kQK8_0 == 0 && K > 0 && n_out > 0 &&
           m >= 1;
}

size_t gemm_g32_repack_bytes(int n_out, int K) { return (size_t)n_out * g32_steps(K) * kG32Rec; }
size_t gemm_g32_pack_bytes(int m, int K) { return (size_t)g32_steps(K) * pack_tblocks(m) * kG32PkBlk; }

static int g32_tiles(int m, int n_out) { return ((n_out + kG32RowsB - 1) / kG32RowsB) * pack_tblocks(m); }

size_t gemm_g32_part_bytes(int m, int n_out, int K) {
    const int nt = g32_tiles(m, n_out);
    const int s = gemm_split_for(nt, g32_steps(K), kG32MaxSplit);
    return s > 1 ? (size_t)s * nt * kTokB * kG32RowsB * sizeof(float) : 0;
}

hipError_t launch_g32_repack(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, uint8_t *rw,
                             hipStream_t st) {
    if (!gemm_g32_supported(type, n_out, K, 1) || ((uintptr_t)rw & 15u) != 0 || ((uintptr_t)w & 1u) != 0)
        return hipErrorInvalidValue;
    const int nb = K / kQK8_0;
    const int kb = type == kTypeQ8_0 ? kBytesQ8_0 : (type == kTypeQ4_0 ? kBytesQ4_0 : kBytesQ5_0);
    if (row_bytes != (size_t)nb * kb) return hipErrorInvalidValue;  // rows are contiguous runs of blocks
    const int nst = g32_steps(K);
    const long long nrec = (long long)n_out * nst;
    const unsigned grid = (unsigned)((nrec + kG32RepackRecs - 1) / kG32RepackRecs);
    if (type == kTypeQ8_0)
        hipLaunchKernelGGL(g32_repack_kernel<kTypeQ8_0>, dim3(grid), dim3(256), 0, st, w, nb, nst, nrec, rw);
    else if (type == kTypeQ4_0)
        hipLaunchKernelGGL(g32_repack_kernel<kTypeQ4_0>, dim3(grid), dim3(256), 0, st, w, nb, nst, nrec, rw);
    else
        hipLaunchKernelGGL(g32_repack_kernel<kTypeQ5_0>, dim3(grid), dim3(256), 0, st, w, nb, nst, nrec, rw);
    return hipGetLastError();
}

// The activation pack from f32 rows (x, row stride K) or from Q8_0 blocks
// (xq, xq_stride bytes per token).
hipError_t launch_g32_pack(const float *x, const uint8_t *xq, size_t xq_stride, int m, int K, uint8_t *pack,
                           hipStream_t st) {
    if (K % kQK8_0 != 0 || m < 1 || ((uintptr_t)pack & 15u) != 0) return hipErrorInvalidValue;
    if (x != nullptr && ((uintptr_t)x & 15u) != 0) return hipErrorInvalidValue;
    const int nst = g32_steps(K), ntb = pack_tblocks(m);
    const unsigned grid = (unsigned)((long long)nst * ntb * kTokB / 8);
    if (x != nullptr)
        hipLaunchKernelGGL(g32_pack_kernel<true>, dim3(grid), dim3(256), 0, st, x, nullptr, (size_t)0, m, K, nst, ntb,
                           pack);
    else
        hipLaunchKernelGGL(g32_pack_kernel<false>, dim3(grid), dim3(256), 0, st, nullptr, xq, xq_stride, m, K, nst,
                           ntb, pack);
    return hipGetLastError();
}

hipError_t launch_gemm_g32(int type, const uint8_t *rw, int n_out, int K, int m, const uint8_t *pack, float *part,
                           unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st) {
    if (!gemm_g32_supported(type, n_out, K, m) || ((uintptr_t)rw & 15u) != 0 || ((uintptr_t)pack & 15u) != 0)
        return hipErrorInvalidValue;
    G32Args a{};
    const int nst = g32_steps(K);
    const size_t rstride = (size_t)nst * kG32Rec;
    const size_t pb = gemm_g32_pack_bytes(m, K);
    if (pb >= ((size_t)1 << 32) || 32 * rstride >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.rw = rw;
    a.rstride = (uint32_t)rstride;
    a.pack = pack;
    a.pack_bytes = (uint32_t)pb;
    a.ntb = pack_tblocks(m);
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.nst = nst;
    a.nrb = (n_out + kG32RowsB - 1) / kG32RowsB;
    a.ntiles = g32_tiles(m, n_out);
    a.nsplit = gemm_split_for(a.ntiles, nst, kG32MaxSplit);
    a.part = part;
    a.cnt = cnt;
    if (a.nsplit > 1 && (part == nullptr || cnt == nullptr)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_g32_kernel, dim3((unsigned)(a.ntiles * a.nsplit)), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
