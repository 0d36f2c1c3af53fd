// Prefill GEMM (m >= 16 tokens) of Q6_K and Q5_K weights against Q8_K
// activations on the matrix cores, every block integer exact:
//   out[t][o] = bias[o] + sum_sb dx[t][sb] * (d[o][sb] * sumi - dmin[o][sb] * summ)
// -- edgexpu_cpu_linear_quant_batch (src/cpu_kernel.c:605-631) with the
// per-super-block integers of dot_q6_k_q8_k (src/gguf_dot_q8.c:897-1002,
// sumi = sum_j sc_j * sum_{16} q * q8 with q = q6 - 32, no min term) and
// dot_q5_k_q8_k (src/gguf_dot_q8.c:764-895, sumi = sum_j sc_j * sum_{32} q * q8
// with q = q5 in 0..31, summ = sum_j m_j * (bsum_2j + bsum_2j+1)).
//
// Exactness.  A weight sc * q is not always an fp16 integer here (Q6_K:
// |sc * q| <= 4096, and odd values above 2048 are not representable), so the
// scale is split, sc = 16 s1 + s0 with s0 = sc & 15 in 0..15 and s1 = sc >> 4
// in -8..7, and every K-step runs two MFMA chains over the same activation
// operand: C0 = sum q8 * (s0 q) and C1 = sum q8 * (s1 q).  |s0 q| <= 480 and
// |s1 q| <= 256, so over a whole super-block |C0| <= 256 * 127 * 480 < 2^24
// and |C1| < 2^24: both chains are exact whatever order the matrix core adds
// in, for every input.  Per super-block sumi = 16 C1 + C0 (one fma, rounded
// once like the reference's float(sumi)), then
//   acc += dx * (sumi * d - mn * dmin)
// with mn the min-term MFMA of the 16 bsums against m_j (Q5_K only).
//
// Weights.  Q6_K blocks (210 B) are 2-byte aligned, so a per-call repack
// (kq_repack_kernel) rewrites each row into an aligned record per
// super-block, in the K order of the Q8_K activation pack (gemm_common.h):
//   half hf (192 B):  q  [lane half 2][K-step 8][8 B]  q + 128, slot order
//                     c  [lane half 2][4 x (fp16 s0, fp16 s1)]  the scales of
//                        (lo, K-steps 0-3), (lo, 4-7), (hi, 0-3), (hi, 4-7)
//                     x  [lane half 2][16 B]  half 0: fp16 m(4h), m(4h),
//                        m(4h+1), m(4h+1), f32 d, f32 dmin; half 1: fp16
//                        m(4h+2), m(4h+2), m(4h+3), m(4h+3)
// 384 B per row and super-block (1.5 B per weight).  The weight operand of a
// K-step is then 2 v_perm (bytes to fp16 1152 + q) and 8 packed fp16 FMAs
// (s * (1152 + q) - 1152 s = s q, exact: one rounding of a representable
// integer), for 4 MFMAs.
//
// Tiling: a workgroup of 8 waves computes 128 rows x 128 tokens; wave w owns
// rows 32 (w % 4) .. + 31 for tokens 64 (w / 4) .. + 63 (2 token tiles x 2
// chains = 4 accumulator tiles).  The main loop is the Q4_K GEMM's: LDS DMA
// only (inline assembly, explicit waits), codes one step ahead in 2 slots,
// extras (bsums / dx) per super-block in 2 slots, weights two steps ahead in
// 3 slots; one barrier per step.  LDS: 64 + 10 + 72 KiB.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "gemm_common.h"

namespace exq {

constexpr int kKqRec = 384;        // repacked bytes per row and super-block
constexpr int kKqHalfRec = 192;
constexpr int kKqRowsB = 128;      // rows per workgroup
constexpr int kKqMaxSplit = 8;
constexpr int kKqGrpBytes = 6 * 1024;  // per row group and step: q 4 KiB, c 1 KiB, x 1 KiB
constexpr int kKqWSlot = 4 * kKqGrpBytes;
constexpr int kKqWSlots = 3;
constexpr int kKqLdsCodes = 0;
constexpr int kKqLdsEx = kKqLdsCodes + 2 * kPkHalf;
constexpr int kKqLdsW = kKqLdsEx + 2 * kPkExtra;
constexpr int kKqLdsLast = kKqLdsW + kKqWSlots * kKqWSlot;
constexpr int kKqLdsBytes = kKqLdsLast + 16;
static_assert(kKqLdsBytes <= 160 * 1024, "the LDS rings fit the gfx950 LDS");

// ----------------------------------------------------------------- repack

// The slot order of one K-step, [lo b0, lo b2, hi b0, hi b2] and
// [lo b1, lo b3, hi b1, hi b3], from the four biased codes of the lo group
// (elements 64 j + 4 s + b) and of the hi group (64 j + 32 + 4 s + b).
__device__ __forceinline__ uint2 slot_order(uint32_t lo4, uint32_t hi4) {
    return make_uint2(__builtin_amdgcn_perm(hi4, lo4, 0x06040200u), __builtin_amdgcn_perm(hi4, lo4, 0x07050301u));
}

// Q6_K codes (src/gguf_dot_q8.c:971-983, q = ql nibble | qh 2 bits << 4,
// minus 32) of K-step s in half hf, lane half h, biased by +128: element
// 64 j + 4 s + b + 32 hi (j = 2 h + hf) is ql byte 64 h + 32 hi + 4 s + b,
// nibble hf, and bits 4 hf + 2 hi of qh byte 32 h + 4 s + b; four bytes at
// once per 32-bit word.
__device__ __forceinline__ uint2 q6k_step(uint32_t ql_lo, uint32_t ql_hi, uint32_t qh, int hf) {
    const int sh = 4 * hf;
    const uint32_t lo = ((ql_lo >> sh) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
    const uint32_t hi = ((ql_hi >> sh) & 0x0F0F0F0Fu) | (((qh >> (sh + 2)) & 0x03030303u) << 4);
    return slot_order(lo + 0x60606060u, hi + 0x60606060u);  // q6 - 32 + 128
}

// Q5_K codes (dequant_q5_k, src/gguf_quant.c:305-345, q = qs nibble + 16 *
// qh bit) of K-step s in half hf, lane half h, biased by +128: element
// 64 j + 4 s + b + 32 hi is nibble hi of qs byte 32 j + 4 s + b and bit
// 2 j + hi of qh byte 4 s + b.
__device__ __forceinline__ uint2 q5k_step(uint32_t qs, uint32_t qh, int j) {
    const uint32_t lo = (qs & 0x0F0F0F0Fu) | (((qh >> (2 * j)) & 0x01010101u) << 4);
    const uint32_t hi = ((qs >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * j + 1)) & 0x01010101u) << 4);
    return slot_order(lo + 0x80808080u, hi + 0x80808080u);
}

// get_scale_min_k4 (src/gguf_quant.c:212-220) on the 12 scale bytes held as
// three words (w0: bytes 0..3, w1: 4..7, w2: 8..11), for a sub-block j that
// may differ between lanes: shifts and one select, no indexed memory.
__device__ __forceinline__ void k4_scale_min(uint32_t w0, uint32_t w1, uint32_t w2, int j, int &sc, int &m) {
    const int sh = 8 * (j & 3);
    const uint32_t a = w0 >> sh, b = w1 >> sh, c = w2 >> sh;
    const bool lo = j < 4;
    sc = (int)(lo ? (a & 63u) : ((c & 0xFu) | (((a >> 6) & 3u) << 4)));
    m = (int)(lo ? (b & 63u) : (((c >> 4) & 0xFu) | (((b >> 6) & 3u) << 4)));
}

__device__ __forceinline__ uint32_t f16_pair(float lo, float hi) {
    const _Float16 l = (_Float16)lo, h = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

constexpr int kRepackRecs = 16;  // (row, super-block) records per workgroup

// 16 threads per record (rows are contiguous runs of blocks, so record r is
// the block at w + r * block bytes): thread t writes q chunk t (16 B: half
// t / 8, lane half (t / 4) % 2, K-steps 2 (t % 4) and + 1) from three 8-byte
// loads of its block, threads 0..3 the c chunks and 4..7 the x chunks of
// (half (t / 2) % 2, lane half t % 2).  Q6_K blocks are 2-byte aligned; gfx950 global memory
// runs in unaligned-access mode, so the loads stay plain dwordx2 loads.
template <int TYPE>
__global__ __launch_bounds__(256) void kq_repack_kernel(const uint8_t *__restrict__ w, long long nrec,
                                                        uint8_t *__restrict__ rw) {
    constexpr int kB = TYPE == kTypeQ6_K ? kBytesQ6_K : kBytesQ5_K;
    const long long r = (long long)blockIdx.x * kRepackRecs + (threadIdx.x >> 4);
    if (r >= nrec) return;
    const int t = threadIdx.x & 15;
    const uint8_t *blk = w + (size_t)r * kB;
    uint8_t *dst = rw + (size_t)r * kKqRec;
    {
        const int hf = t >> 3, h = (t >> 2) & 1, p = t & 3;
        uint2 a, b;
        if (TYPE == kTypeQ6_K) {
            const uint2 lo = ldg8(blk + 64 * h + 8 * p), hi = ldg8(blk + 64 * h + 32 + 8 * p);
            const uint2 qh = ldg8(blk + 128 + 32 * h + 8 * p);
            a = q6k_step(lo.x, hi.x, qh.x, hf);
            b = q6k_step(lo.y, hi.y, qh.y, hf);
        } else {
            const int j = 2 * h + hf;
            const uint2 qs = ldg8(blk + 48 + 32 * j + 8 * p), qh = ldg8(blk + 16 + 8 * p);
            a = q5k_step(qs.x, qh.x, j);
            b = q5k_step(qs.y, qh.y, j);
        }
        *reinterpret_cast<uint4 *>(dst + hf * kKqHalfRec + 64 * h + 16 * p) = make_uint4(a.x, a.y, b.x, b.y);
    }
    if (t < 8) {  // threads 0..3: the c chunk, 4..7: the x chunk of (half (t >> 1) & 1, lane half t & 1)
        const int hf = (t >> 1) & 1, h = t & 1, j = 2 * h + hf;
        uint32_t o[4];
        if (TYPE == kTypeQ6_K) {
            if (t < 4) {
                const uint32_t s4 = ldg4(blk + 192 + 4 * j);  // int8 scales of 16-element sub-blocks 4j .. 4j + 3
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    const int v = (int)(int8_t)(s4 >> (8 * kc));
                    o[kc] = f16_pair((float)(v & 15), (float)(v >> 4));
                }
            } else {
                const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk + 208));
                o[0] = o[1] = 0u;  // no min term
                o[2] = hf == 0 ? __float_as_uint(d) : 0u;
                o[3] = 0u;
            }
        } else {
            const uint32_t w0 = ldg4(blk + 4), w1 = ldg4(blk + 8), w2 = ldg4(blk + 12);
            if (t < 4) {
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    int v, m;
                    k4_scale_min(w0, w1, w2, 2 * j + (kc >> 1), v, m);  // lo: sub-block 2j, hi: 2j + 1
                    o[kc] = f16_pair((float)(v & 15), (float)(v >> 4));
                }
            } else {
                // half 0 carries m(4h), m(4h+1), d and dmin; half 1 m(4h+2), m(4h+3)
                int v, m0, m1;
                k4_scale_min(w0, w1, w2, 4 * h + 2 * hf, v, m0);
                k4_scale_min(w0, w1, w2, 4 * h + 2 * hf + 1, v, m1);
                const uint32_t hd = ldg4(blk);
                o[0] = f16_pair((float)m0, (float)m0);
                o[1] = f16_pair((float)m1, (float)m1);
                o[2] = hf == 0 ? __float_as_uint(f16_bits_to_f32(hd & 0xffffu)) : 0u;
                o[3] = hf == 0 ? __float_as_uint(f16_bits_to_f32(hd >> 16)) : 0u;
            }
        }
        *reinterpret_cast<uint4 *>(dst + hf * kKqHalfRec + (t < 4 ? 128 : 160) + 16 * h) =
            make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// ------------------------------------------------------------------- GEMM

struct KqArgs {
    const uint8_t *rw;    // [n_out][nblk][kKqRec] repacked weights
    uint32_t rstride;     // bytes per repacked row
    const uint8_t *pack;  // [nblk][ntb][kPkBlk] Q8_K activation pack
    uint32_t pack_bytes;
    int ntb;
    const float *bias;
    float *out;
    int ldo, m, n_out, nblk;
    int nrb, ntiles, nsplit;
    float *part;
    unsigned *cnt;
};

struct KqLoop {
    v4u pack, rows;
    uint32_t pk0, pk_sb;
    uint32_t voff_q, voff_cx;  // lane's q record (row lane % 32, + 64 h) and c / x (+ 16 h)
    uint32_t smem;
    int lane, wave, grp, th, sb0, sblast;
    bool codes_on;  // the wave's code chunks (token tile wave % 4) hold a token below m
    bool ex_on;     // the wave's extras chunk is needed: bsums of a live tile (min term), or dx
};

constexpr int kKqWLoads = 3;

// Step s requests: codes of step s + 1 (4 DMAs), on odd steps the extras of
// the next super-block (1 DMA), then the weights of step s + 2 (3 DMAs:
// token-half 0 waves q pieces 0, 1 and c; token-half 1 waves q pieces 2, 3
// and x).  Past the end of the K range the last super-block is requested
// again into slots nobody reads, so the weights are always the last 3: a
// wait for vmcnt(3) covers everything before them however many code and
// extras chunks a wave skips (those of token tiles past the last token,
// which no wave reads).
__device__ __forceinline__ void kq_step_requests(const KqLoop &L, int s) {
    const uint32_t lv = (uint32_t)L.lane * 16;
    const int s1 = s + 1;
    const int sbc = min(L.sb0 + (s1 >> 1), L.sblast);
    const uint32_t cdst = L.smem + kKqLdsCodes + (uint32_t)(s1 & 1) * kPkHalf;
    const uint32_t cso = L.pk0 + (uint32_t)sbc * L.pk_sb + (uint32_t)(s1 & 1) * kPkHalf;
    if (L.codes_on) {
#pragma unroll
        for (int i = 0; i < kHalfChunks / kWaves; ++i) {
            const uint32_t ch = (uint32_t)(kWaves * i + L.wave);
            dma16(cdst + ch * 1024, lv, L.pack, cso + ch * 1024);
        }
    }
    if ((s & 1) && L.ex_on) {
        const int je = s1 >> 1;
        const int sbe = min(L.sb0 + je, L.sblast);
        const uint32_t ch = (uint32_t)L.wave;
        dma16(L.smem + kKqLdsEx + (uint32_t)(je & 1) * kPkExtra + ch * 1024, lv, L.pack,
              L.pk0 + (uint32_t)sbe * L.pk_sb + kPkCodes + ch * 1024);
    }
    const int s2 = s + 2;
    const int sbw = min(L.sb0 + (s2 >> 1), L.sblast);
    const uint32_t wdst = L.smem + kKqLdsW + (uint32_t)(s2 % kKqWSlots) * kKqWSlot + (uint32_t)L.grp * kKqGrpBytes;
    const uint32_t wso = (uint32_t)sbw * kKqRec + (uint32_t)(s2 & 1) * kKqHalfRec;
    dma16(wdst + 2048 * L.th, L.voff_q, L.rows, wso + 32 * L.th);
    dma16(wdst + 2048 * L.th + 1024, L.voff_q, L.rows, wso + 32 * L.th + 16);
    dma16(wdst + 4096 + 1024 * L.th, L.voff_cx, L.rows, wso + 128 + 32 * L.th);
}

// Multipliers and addends of the half's four scales: m[kc] = {s0, s1},
// a[kc] = {-1152 s0, -1152 s1}.
struct KqConst {
    h2 m[4], a[4];
};

__device__ __forceinline__ KqConst kq_const(v4u c) {
    KqConst k;
    const h2 na = h2{(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        // through a scalar: a bit_cast whose operand is a vector element
        // reads element 0 with this compiler
        const uint32_t ck = c[kc];
        k.m[kc] = __builtin_bit_cast(h2, ck);
        k.a[kc] = k.m[kc] * na;
    }
    return k;
}

// Weight operands of chains 0 and 1 from the K-step's 8 biased q bytes.
__device__ __forceinline__ void kq_operands(uint32_t q0, uint32_t q1, const KqConst &k, int klo, int khi,
                                            uint32_t hi64, v8h &w0, v8h &w1) {
    h2 pa[2], pb[2];
    bytes_to_h2(q0, hi64, pa);
    bytes_to_h2(q1, hi64, pb);
    const h2 p[4] = {pa[0], pa[1], pb[0], pb[1]};
    const h2 ml0 = h2{k.m[klo].x, k.m[klo].x}, al0 = h2{k.a[klo].x, k.a[klo].x};
    const h2 mh0 = h2{k.m[khi].x, k.m[khi].x}, ah0 = h2{k.a[khi].x, k.a[khi].x};
    const h2 ml1 = h2{k.m[klo].y, k.m[klo].y}, al1 = h2{k.a[klo].y, k.a[klo].y};
    const h2 mh1 = h2{k.m[khi].y, k.m[khi].y}, ah1 = h2{k.a[khi].y, k.a[khi].y};
    const h2 b0 = __builtin_elementwise_fma(p[0], ml0, al0), b1 = __builtin_elementwise_fma(p[1], mh0, ah0);
    const h2 b2 = __builtin_elementwise_fma(p[2], ml0, al0), b3 = __builtin_elementwise_fma(p[3], mh0, ah0);
    const h2 c0 = __builtin_elementwise_fma(p[0], ml1, al1), c1 = __builtin_elementwise_fma(p[1], mh1, ah1);
    const h2 c2 = __builtin_elementwise_fma(p[2], ml1, al1), c3 = __builtin_elementwise_fma(p[3], mh1, ah1);
    w0 = v8h{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
    w1 = v8h{c0.x, c0.y, c1.x, c1.y, c2.x, c2.y, c3.x, c3.y};
}

// C[chain][token tile]
typedef v16f KqTiles[2][2];

// The 8 K-steps of one half for the wave's first NT token tiles: codes
// slot `cur` (token tiles at cur + tt * 1024, 4 KiB per K-step), weight slot
// `wq` (q pieces at wq + 1024 p, c at wq + 4096).  The operands of the next
// K-step are built while this K-step's MFMAs run.  NT < 2 when the wave's
// second token tile lies entirely past the last token.
template <bool FIRST, int NT>
__device__ __forceinline__ void kq_half(const uint8_t *cur, const uint8_t *wq, int lane, uint32_t hi64, KqTiles &C) {
    const KqConst k = kq_const(lds_v4u(wq + 4096 + lane * 16));
    v4u q[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) q[p] = lds_v4u(wq + 1024 * p + lane * 16);
    v8h a[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) a[tt] = lds_v8h(cur + tt * 1024 + lane * 16);
    v8h w0, w1;
    kq_operands(q[0][0], q[0][1], k, 0, 2, hi64, w0, w1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        v8h nw0 = w0, nw1 = w1;
        if (s + 1 < 8) {
            const int n = s + 1;
            kq_operands(q[n >> 1][2 * (n & 1)], q[n >> 1][2 * (n & 1) + 1], k, n >= 4 ? 1 : 0, n >= 4 ? 3 : 2, hi64,
                        nw0, nw1);
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            C[0][tt] = mfma(a[tt], w0, (FIRST && s == 0) ? v16f{} : C[0][tt]);
            C[1][tt] = mfma(a[tt], w1, (FIRST && s == 0) ? v16f{} : C[1][tt]);
            if (s + 1 < 8) a[tt] = lds_v8h(cur + (s + 1) * 4096 + tt * 1024 + lane * 16);
        }
        if (NT == 2) {
            // MFMA, VALU x3, MFMA, DS read, VALU x2, MFMA, VALU x3, MFMA, DS read, VALU x2
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
        } else {
            // MFMA, VALU x6, DS read, MFMA, VALU x6
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        w0 = nw0;
        w1 = nw1;
    }
}

// acc += dx * ((16 C1 + C0) * d - mn * dmin) for the wave's first NT token
// tiles (extras slot `ex`, the wave's first token tile tq).
template <bool MIN, int NT>
__device__ __forceinline__ void kq_combine(const uint8_t *ex, int tq, int lane, float dd, float ndm, v8h bmn,
                                           const KqTiles &C, v16f (&acc)[2]) {
    const int h = lane >> 5;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        v16f mn = v16f{};
        if (MIN) mn = mfma(lds_v8h(ex + (tq + tt) * 1024 + lane * 16), bmn, v16f{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 dx = *reinterpret_cast<const float4 *>(ex + kPkMn + 4 * (32 * (tq + tt) + 8 * i + 4 * h));
            const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * i + e;
                float v = __builtin_fmaf(C[1][tt][r], 16.0f, C[0][tt][r]) * dd;
                if (MIN) v = __builtin_fmaf(mn[r], ndm, v);
                acc[tt][r] = __builtin_fmaf(v, dxs[e], acc[tt][r]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The main loop over the workgroup's super-blocks for a wave with NT live
// token tiles (NT = 0: the wave only moves data for the others).
template <bool MIN, int NT>
__device__ __forceinline__ void kq_loop(const KqLoop &L, uint8_t *smem, int nsb, int tq, uint32_t hi64, KqTiles &C,
                                        v16f (&acc)[2]) {
    const int lane = L.lane, grp = L.grp;
    for (int j = 0; j < nsb; ++j) {
        const int s = 2 * j;
        const uint8_t *ex = smem + kKqLdsEx + (j & 1) * kPkExtra;
        // even step: half 0; its x chunk holds m(4h), m(4h+1), d and dmin
        wait_dma<kKqWLoads>();
        __syncthreads();
        kq_step_requests(L, s);
        if constexpr (NT > 0) {
            const uint8_t *wq0 = smem + kKqLdsW + (s % kKqWSlots) * kKqWSlot + grp * kKqGrpBytes;
            const v4u x0 = lds_v4u(wq0 + 5120 + lane * 16);
            kq_half<true, NT>(smem + kKqLdsCodes + tq * 1024, wq0, lane, hi64, C);
            // odd step: half 1, then the super-block's combination
            wait_dma<kKqWLoads>();
            __syncthreads();
            kq_step_requests(L, s + 1);
            const uint8_t *wq1 = smem + kKqLdsW + ((s + 1) % kKqWSlots) * kKqWSlot + grp * kKqGrpBytes;
            v4u x1 = v4u{0u, 0u, 0u, 0u};
            if (MIN) x1 = lds_v4u(wq1 + 5120 + lane * 16);
            kq_half<false, NT>(smem + kKqLdsCodes + kPkHalf + tq * 1024, wq1, lane, hi64, C);
            const float dd = __uint_as_float(x0[2]), ndm = -__uint_as_float(x0[3]);
            v8h bmn = v8h{};
            if (MIN) bmn = __builtin_bit_cast(v8h, v4u{x0[0], x0[1], x1[0], x1[1]});
            kq_combine<MIN, NT>(ex, tq, lane, dd, ndm, bmn, C, acc);
        } else {
            wait_dma<kKqWLoads>();
            __syncthreads();
            kq_step_requests(L, s + 1);
        }
    }
}

template <bool MIN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_kq_kernel(KqArgs a) {
    __shared__ __align__(16) uint8_t smem[kKqLdsBytes];
    int *s_last = reinterpret_cast<int *>(smem + kKqLdsLast);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int grp = wave & 3, th = wave >> 2;

    const int tile = (int)blockIdx.x % a.ntiles, z = (int)blockIdx.x / a.ntiles;
    const int rb = tile % a.nrb, tb = tile / a.nrb;
    const int sb0 = (int)((long long)a.nblk * z / a.nsplit);
    const int sb1 = (int)((long long)a.nblk * (z + 1) / a.nsplit);
    const int nsb = sb1 - sb0;

    const int rowg = rb * kKqRowsB + 32 * grp;
    KqLoop L;
    L.lane = lane;
    L.wave = wave;
    L.grp = grp;
    L.th = th;
    L.sb0 = sb0;
    L.sblast = sb1 - 1;
    L.pk_sb = (uint32_t)a.ntb * kPkBlk;
    L.pk0 = (uint32_t)tb * kPkBlk;
    L.pack = rsrc_words(a.pack, a.pack_bytes);
    const int live_rows = min(32, a.n_out - rowg);
    L.rows = rsrc_words(a.rw + (size_t)min(rowg, a.n_out - 1) * a.rstride,
                        live_rows > 0 ? (uint32_t)live_rows * a.rstride : 0u);
    L.voff_q = (uint32_t)(lane & 31) * a.rstride + 64u * (uint32_t)h;
    L.voff_cx = (uint32_t)(lane & 31) * a.rstride + 16u * (uint32_t)h;
    L.smem = lds_addr(smem);
    const int live_wg = min(kTiles, max(0, (a.m - kTokB * tb + 31) / 32));  // token tiles holding a token
    L.codes_on = (wave & 3) < live_wg;
    L.ex_on = wave < kTiles ? (MIN && wave < live_wg) : wave == kTiles;  // chunk 4: dx and sum |q8|
    uint32_t hi64 = 0x64646464u;
    asm volatile("" : "+v"(hi64));

    v16f acc[2];
    acc[0] = v16f{};
    acc[1] = v16f{};
    KqTiles C;

    {
        const uint32_t lv = (uint32_t)lane * 16;
        const uint32_t cso = L.pk0 + (uint32_t)sb0 * L.pk_sb;
        if (L.codes_on) {
#pragma unroll
            for (int i = 0; i < kHalfChunks / kWaves; ++i) {
                const uint32_t c = (uint32_t)(kWaves * i + wave);
                dma16(L.smem + kKqLdsCodes + c * 1024, lv, L.pack, cso + c * 1024);
            }
        }
        if (L.ex_on)
            dma16(L.smem + kKqLdsEx + (uint32_t)wave * 1024, lv, L.pack, cso + kPkCodes + (uint32_t)wave * 1024);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint32_t wdst = L.smem + kKqLdsW + (uint32_t)hf * kKqWSlot + (uint32_t)grp * kKqGrpBytes;
            const uint32_t wso = (uint32_t)sb0 * kKqRec + (uint32_t)hf * kKqHalfRec;
            dma16(wdst + 2048 * th, L.voff_q, L.rows, wso + 32 * th);
            dma16(wdst + 2048 * th + 1024, L.voff_q, L.rows, wso + 32 * th + 16);
            dma16(wdst + 4096 + 1024 * th, L.voff_cx, L.rows, wso + 128 + 32 * th);
        }
    }

    const int tq = 2 * th;
    // token tiles of this wave that hold at least one token below m; one
    // instance of the loop per count, so that neither carries the other's
    // registers
    const int live = min(2, max(0, live_wg - tq));
    if (live == 2)
        kq_loop<MIN, 2>(L, smem, nsb, tq, hi64, C, acc);
    else if (live == 1)
        kq_loop<MIN, 1>(L, smem, nsb, tq, hi64, C, acc);
    else
        kq_loop<MIN, 0>(L, smem, nsb, tq, hi64, C, acc);
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

bool gemm_kq_supported(int type, int n_out, int K, int m) {
    return (type == kTypeQ6_K || type == kTypeQ5_K) && K % kQKK == 0 && K > 0 && n_out > 0 && m >= 1;
}

size_t gemm_kq_repack_bytes(int n_out, int K) { return (size_t)n_out * (size_t)(K / kQKK) * kKqRec; }

static int kq_tiles(int m, int n_out) { return ((n_out + kKqRowsB - 1) / kKqRowsB) * pack_tblocks(m); }

size_t gemm_kq_part_bytes(int m, int n_out, int K) {
    const int nt = kq_tiles(m, n_out);
    const int s = gemm_split_for(nt, K / kQKK, kKqMaxSplit);
    return s > 1 ? (size_t)s * nt * kTokB * kKqRowsB * sizeof(float) : 0;
}

hipError_t launch_kq_repack(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, uint8_t *rw,
                            hipStream_t st) {
    if (!gemm_kq_supported(type, n_out, K, 1) || ((uintptr_t)rw & 15u) != 0 || ((uintptr_t)w & 1u) != 0)
        return hipErrorInvalidValue;
    const int nb = K / kQKK;
    // rows are contiguous runs of blocks (GGUF rows carry no padding)
    if (row_bytes != (size_t)nb * (type == kTypeQ6_K ? kBytesQ6_K : kBytesQ5_K)) return hipErrorInvalidValue;
    const long long nrec = (long long)n_out * nb;
    const unsigned grid = (unsigned)((nrec + kRepackRecs - 1) / kRepackRecs);
    if (type == kTypeQ6_K)
        hipLaunchKernelGGL(kq_repack_kernel<kTypeQ6_K>, dim3(grid), dim3(256), 0, st, w, nrec, rw);
    else
        hipLaunchKernelGGL(kq_repack_kernel<kTypeQ5_K>, dim3(grid), dim3(256), 0, st, w, nrec, rw);
    return hipGetLastError();
}

// out = bias + W x over the repacked weights (launch_kq_repack) and the Q8_K
// activation pack (launch_q8k_pack_*); part holds gemm_kq_part_bytes and cnt
// the zero-filled arrival counters.
hipError_t launch_gemm_kq(int type, const uint8_t *rw, int n_out, int K, int m, const uint8_t *pack,
                          float *part, unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st) {
    if (!gemm_kq_supported(type, n_out, K, m) || ((uintptr_t)rw & 15u) != 0 || ((uintptr_t)pack & 15u) != 0)
        return hipErrorInvalidValue;
    KqArgs a{};
    a.rw = rw;
    const size_t rstride = (size_t)(K / kQKK) * kKqRec;
    const size_t pb = (size_t)(K / kQKK) * pack_tblocks(m) * kPkBlk;
    if (pb >= ((size_t)1 << 32) || 32 * rstride >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.rstride = (uint32_t)rstride;
    a.pack = pack;
    a.pack_bytes = (uint32_t)pb;
    a.ntb = pack_tblocks(m);
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.m = m;
    a.n_out = n_out;
    a.nblk = K / kQKK;
    a.nrb = (n_out + kKqRowsB - 1) / kKqRowsB;
    a.ntiles = kq_tiles(m, n_out);
    a.nsplit = gemm_split_for(a.ntiles, a.nblk, kKqMaxSplit);
    a.part = part;
    a.cnt = cnt;
    if (a.nsplit > 1 && (part == nullptr || cnt == nullptr)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(a.ntiles * a.nsplit));
    if (type == kTypeQ5_K)
        hipLaunchKernelGGL(gemm_kq_kernel<true>, grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL(gemm_kq_kernel<false>, grid, dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
