// Streaming decode GEMV for one to four tokens of Q4_K or Q6_K rows:
// edgexpu_cpu_linear_quant_batch (src/cpu_kernel.c:545-644) at m <= 4 with
// the Q4_K x Q8_K and Q6_K x Q8_K block dots (dot_q4_k_q8_k,
// src/gguf_dot_q8.c:603-666; dot_q6_k_q8_k, 897-963), for the row lengths of
// the decode steps (Q4_K: K = 2560, 4096, 14336; Q6_K: 9728).
//
// Every weight row travels HBM -> LDS by DMA (buffer_load ... lds: no
// registers held while it is in flight), one row per wave step (two adjacent
// rows in long launches of rows of 2560, and of rows of 4096 at 2-4 tokens),
// into a per-wave ring of NB slots.  A slot is refilled as soon as its bytes are in
// registers, so NB rows per wave stay in flight while the wave computes.
// Lanes own fixed 64-element units of K (super-block i, quarter j): the
// activation slices of a lane stay in registers for every row (where the
// tokens' slices would take more than 160 registers, each row reads them
// from LDS), the Q4_K
// header's 6-bit scale/min pair is unpacked with lane-constant selectors
// (v_perm), integer block sums with sdot4 / sdot2, one fp32 combine per unit.
// A row's total is the fused kernel's butterfly over the lanes (so the two
// kernels' outputs are equal bit for bit), four rows at a time;
// step k's total is kept in lane k % 64 and every 64 steps one store per wave
// writes them with their bias (prefetched at the start), so the only vector
// memory operations inside the loop are the DMAs and every wait counts
// exactly the rows still in flight.
//
// The activation is quantized to Q8_K inside each workgroup with the
// fused kernel's staging (quantize_q8_k_group: the reference's
// quantize_row_q8_K, src/gguf_dot_q8.c:360-412, up to the sign of each
// block's codes and scale, which cancels in every dot), optionally after a
// staging prologue (RMSNorm, SiLU-mul; src/native.c:2529, 2576-2578), or read from
// Q8_K block bytes already in memory.  Epilogues: bias, residual
// (src/native.c:2571-2580), gate/up pairs with silu(gate) * up.
//
// The waits on the ring are explicit s_waitcnt counts over the DMAs this
// wave issued: vector memory loads of one wave complete in issue order, and
// the loop issues no other vector memory operation.  The staged inputs are
// read by inline-assembly loads issued before the ring's first rows, so the
// compiler inserts no wait of its own for them (its count would include the
// DMAs it cannot see); one explicit wait after the ring's first rows lets
// only those rows stay in flight.
#include <type_traits>
#include <utility>

#include "gemv_fused_kernel.h"

namespace exq {

namespace {

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));

constexpr int kStreamMaxMats = 4;
// Rows of 14336 elements take the streaming kernel in the size-based mode
// from this many weight bytes (2048 rows).
constexpr long long kStreamMinBytes14336 = 2048ll * 56 * kBytesQ4_K;

struct StreamArgs {
    int nmat;                              // matrices (pairs: 1, gate = w[0], up = w[1])
    const uint8_t *w[kStreamMaxMats];
    const float *bias[kStreamMaxMats];
    const float *resid[kStreamMaxMats];    // added after the bias (null: none)
    float *out[kStreamMaxMats];
    int n_out[kStreamMaxMats];
    int row_start[kStreamMaxMats + 1];     // first step of each matrix
    int nrows;                             // steps (rows, gate/up pairs or row pairs)
    const float *x;                        // f32 activation [m][K] (staged), or
    const uint8_t *xq;                     // its Q8_K block bytes
    const float *x2;                       // SiLU-mul: act = silu(x) * x2
    const float *nw;                       // RMSNorm: act = rmsnorm(x; nw, eps)
    float eps;
    unsigned long long *amax;              // argmax epilogue: one key per workgroup, at blockIdx.x
    int cu_major;                          // 1: wave w of workgroup g is wave w * G + g of the grid (G
                                           // workgroups), else g * NW + w
};

// flags: bits 0-1 prologue (1 RMSNorm, 2 SiLU-mul), 4 residual, 8 gate/up
// pairs, 16 activation already in Q8_K block bytes, 32 f32 activation (the
// f32-activation dot of the logits, not quantized), 64 greedy-argmax keys,
// 128 two adjacent rows of one matrix per step, 256 three adjacent rows per
// step (Q6_K f32 rows of 2560, their 120 units over two passes of 64 lanes)
constexpr int kSRes = 4, kSPair = 8, kSXq = 16, kSF32 = 32, kSArgmax = 64, kSRow2 = 128, kSRow3 = 256;

__device__ __forceinline__ v4u_t s_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return v4u_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// One LDS DMA: each lane's 16 bytes at base + soff + voff land at LDS byte
// address lds + 16 * lane (M0 saved and restored around it).  voff is the
// range-checked offset: past the buffer the lane reads zeros.
__device__ __forceinline__ void s_dma16(uint32_t lds, uint32_t voff, const v4u_t &rs, uint32_t soff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
        : "memory");
}
// The same with the non-temporal hint, for the weight rows, which are read
// once per launch: measured on the decode launches, 0.5 to 0.9 us less per
// launch ([4096 x 14336] 11.1 -> 10.1 us, [28672 x 4096] 14.5 -> 13.7,
// [4096 x 4096] 5.3 -> 4.8) than rows that allocate in the caches like the
// activation, which every workgroup reads.
__device__ __forceinline__ void s_dma16_nt(uint32_t lds, uint32_t voff, const v4u_t &rs, uint32_t soff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
        : "memory");
}

// One LDS DMA of 4 bytes per lane (lane L's dword lands at lds + 4 * L), non-temporal.
__device__ __forceinline__ void s_dma4_nt(uint32_t lds, uint32_t voff, const v4u_t &rs, uint32_t soff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dword %2, %3, %4 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
        : "memory");
}

template <int N>
__device__ __forceinline__ void s_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ uint32_t s_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes at p (16-byte aligned global address) into registers, no wait.
__device__ __forceinline__ v4u_t s_load16(const void *p) {
    v4u_t r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}

template <int CTRL>
__device__ __forceinline__ float s_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Sum over the 64 lanes, every lane gets it, as group_reduce (common.h)
// sums a 64-lane group: partners l ^ 32, ^ 16, ^ 8, ^ 4, ^ 2, ^ 1 in that
// order (bpermute, swizzle, DPP rotation by 8, swizzle, quad DPP).  Each pair
// adds the same two values, so every lane holds the same total, bit for bit
// the fused kernel's total for the same lane partials.
__device__ __forceinline__ float s_wave_total(float a) {
    a += __shfl_xor(a, 32, 64);
    a += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x401f));  // ^ 16
    a += s_dpp<0x128>(a);  // ^ 8 (row_ror:8)
    a += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x101f));  // ^ 4
    a += s_dpp<0x4E>(a);   // ^ 2
    a += s_dpp<0xB1>(a);   // ^ 1
    return a;
}

// Four values per lane summed over the wave with the same tree, the first
// two levels transposed (as group_reduce does for V = 4): level ^32 leaves
// rows {0,1} on lanes 0-31 and {2,3} on 32-63, level ^16 one row per lane;
// every row's pairs (and the order within each pair) are those of
// s_wave_total, so each total is its s_wave_total bit for bit.  Row r ends on the lanes with bit 5 = r / 2 and
// bit 4 = r % 2, e.g. lane 16 r.
__device__ __forceinline__ float s_wave_total4(const float (&v)[4]) {
    const int lane = threadIdx.x & 63;
    const bool u32 = (lane & 32) != 0;
    const float s0 = u32 ? v[0] : v[2], k0 = u32 ? v[2] : v[0];
    const float s1 = u32 ? v[1] : v[3], k1 = u32 ? v[3] : v[1];
    const float b0 = k0 + __shfl_xor(s0, 32, 64), b1 = k1 + __shfl_xor(s1, 32, 64);
    const bool u16 = (lane & 16) != 0;
    const float s = u16 ? b0 : b1, k = u16 ? b1 : b0;
    float a = k + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s), 0x401f));
    a += s_dpp<0x128>(a);  // ^ 8
    a += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x101f));  // ^ 4
    a += s_dpp<0x4E>(a);   // ^ 2
    a += s_dpp<0xB1>(a);   // ^ 1
    return a;
}

// The row total of 33-48 units as the fused kernel's f32-activation launches
// form it (16-lane slots over three waves, src/native.c:445-462 rows of
// 2112-3072): lanes 16k..16k+15 summed by the last four levels of
// s_wave_total (^ 8, ^ 4, ^ 2, ^ 1), then the three group totals added in
// order from 0, as the fused kernel adds its waves' partials.
__device__ __forceinline__ float s_wave_total_3x16(float a) {
    a += s_dpp<0x128>(a);  // ^ 8 (row_ror:8)
    a += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x101f));  // ^ 4
    a += s_dpp<0x4E>(a);   // ^ 2
    a += s_dpp<0xB1>(a);   // ^ 1
    float t = 0.0f;
    t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
    t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 16));
    t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 32));
    return t;
}

// Value of lane `src` (wave-uniform) in every lane.
__device__ __forceinline__ float s_lane(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// Per-lane selectors of the 6-bit scale/min pair of sub-blocks 2j, 2j+1
// (get_scale_min_k4, src/gguf_dot_q8.c:112-124): header words y = scales
// 0..3, z = 4..7, w = 8..11; for j < 2 sc = y[b..b+1] & 63, m = z[b..b+1] & 63;
// for j >= 2 sc = (w[b..] & 15) | ((y[b..] >> 6) << 4),
// m = (w[b..] >> 4) | ((z[b..] >> 6) << 4), b = 2 (j & 1).
struct ScaleSel {
    uint32_t sel, mT, sU;
};
__device__ __forceinline__ ScaleSel scale_sel(int j) {
    const uint32_t b = 2u * (uint32_t)(j & 1);
    return ScaleSel{b | ((b + 1u) << 8) | ((b + 4u) << 16) | ((b + 5u) << 24), j < 2 ? 0u : 0x0f0f0f0fu,
                    j < 2 ? 0u : 2u};
}

// One unit's contribution, with the roundings of FmtQ4K::dot1: fma(dx*d, isum)
// then fma(-dx*dmin, imin) (so a row's total is the fused kernel's bit for
// bit).  |dlo|, |dhi| <= 32 * 15 * 128 < 2^23: the scale products are 24-bit.
__device__ __forceinline__ float q4k_unit(v4u_t h, v4u_t q0, v4u_t q1, const FmtQ4K::Act &x, const ScaleSel &c) {
    const uint32_t T = __builtin_amdgcn_perm(h.w >> 4, h.w, c.sel);
    const uint32_t U = __builtin_amdgcn_perm(h.z, h.y, c.sel);
    const uint32_t res = ((T & c.mT) | ((U >> c.sU) & ~c.mT)) & 0x3f3f3f3fu;  // sc0, sc1, m0, m1
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int dlo = 0, dhi = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        dlo = sdot4(qw[k] & 0x0f0f0f0fu, x.q[k], dlo);
        dhi = sdot4((qw[k] >> 4) & 0x0f0f0f0fu, x.q[8 + k], dhi);
    }
    const int sc0 = (int)(res & 0xffu), sc1 = (int)((res >> 8) & 0xffu);
    const int isum = ((dlo << 8) >> 8) * sc0 + ((dhi << 8) >> 8) * sc1;
    const int imin = sdot2(__builtin_amdgcn_perm(0u, res, 0x0c030c02u), x.spair, 0);
    const float dd = x.dx * f16_bits_to_f32(h.x), dm = x.dx * f16_bits_to_f32(h.x >> 16);
    return fmaf(-dm, (float)imin, fmaf(dd, (float)isum, 0.0f));
}

// The activation slice of unit u from Q8_K block bytes (292 B per block) in LDS.
__device__ __forceinline__ void act_from_blocks(const uint8_t *raw, int unit, FmtQ4K::Act &x) {
    const int i = unit >> 2, j = unit & 3;
    const uint8_t *blk = raw + (size_t)i * kBytesQ8_K;
#pragma unroll
    for (int v = 0; v < 16; ++v) x.q[v] = *reinterpret_cast<const uint32_t *>(blk + 4 + 64 * j + 4 * v);
    x.dx = *reinterpret_cast<const float *>(blk);
    const uint32_t b0 = *reinterpret_cast<const uint32_t *>(blk + 260 + 8 * j);
    const uint32_t b1 = *reinterpret_cast<const uint32_t *>(blk + 264 + 8 * j);
    const int s0 = (int)(int16_t)(b0 & 0xffffu) + (int)(int16_t)(b0 >> 16);
    const int s1 = (int)(int16_t)(b1 & 0xffffu) + (int)(int16_t)(b1 >> 16);
    x.spair = ((uint32_t)s0 & 0xffffu) | ((uint32_t)s1 << 16);
}

// Q6_K rows in LDS: a row of 210-byte super-blocks starts 4-byte aligned in
// its slot, so a super-block starts 2 mod 4 when its index is odd.  The
// fields of a unit (16-byte quarter-rows A, B of the low nibbles, H of the
// high bits, the 8 scale bytes of its half, d) share that offset.  Reads
// take aligned dwords and join them with v_alignbyte (sh = 0 or 2 bytes).
__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ v4u_t lds16_a2(const uint8_t *q, uint32_t sh) {  // q 4-byte aligned
    const uint32_t w0 = lds_u32(q), w1 = lds_u32(q + 4), w2 = lds_u32(q + 8), w3 = lds_u32(q + 12),
                   w4 = lds_u32(q + 16);
    return v4u_t{__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                 __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh)};
}

// One Q6_K unit's contribution with the roundings of FmtQ6K::dot1 from a
// zero accumulator: fma(dx * d, isum, 0), isum = sum_k sc_k (dot_k - 32
// bsum_k) exact in int32 (src/gguf_dot_q8.c:897-963).
__device__ __forceinline__ float q6k_unit(v4u_t A4, v4u_t B4, v4u_t H4, uint32_t scx, uint32_t scy, uint32_t dbits,
                                          int p, const FmtQ6K::Act &xa) {
    const float d = f16_bits_to_f32(dbits);
    int sc[4];
    sc[0] = (int)(int8_t)((scx >> (8 * p)) & 0xffu);
    sc[1] = (int)(int8_t)((scx >> (8 * (2 + p))) & 0xffu);
    sc[2] = (int)(int8_t)((scy >> (8 * p)) & 0xffu);
    sc[3] = (int)(int8_t)((scy >> (8 * (2 + p))) & 0xffu);
    const uint32_t A[4] = {A4.x, A4.y, A4.z, A4.w};
    const uint32_t B[4] = {B4.x, B4.y, B4.z, B4.w};
    const uint32_t H[4] = {H4.x, H4.y, H4.z, H4.w};
    uint32_t c[4][4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        c[0][v] = (A[v] & 0x0f0f0f0fu) | ((H[v] << 4) & 0x30303030u);
        c[1][v] = (B[v] & 0x0f0f0f0fu) | ((H[v] << 2) & 0x30303030u);
        c[2][v] = ((A[v] >> 4) & 0x0f0f0f0fu) | (H[v] & 0x30303030u);
        c[3][v] = ((B[v] >> 4) & 0x0f0f0f0fu) | ((H[v] >> 2) & 0x30303030u);
    }
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int dk = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) dk = sdot4(c[k][v], xa.q[4 * k + v], dk);
        isum += sc[k] * (dk - xa.bs32[k]);
    }
    return fmaf(xa.dx * d, (float)isum, 0.0f);
}

template <int KSB, int NW, int NB, int FL, bool DEEP, int M = 1, int TYPE = kTypeQ4_K>
struct StreamGeom {
    static constexpr bool Q6 = TYPE == kTypeQ6_K;
    static constexpr int K = KSB * kQKK;
    static constexpr int U = 4 * KSB;                    // units per row
    static constexpr int R3 = (FL & kSRow3) ? 3 : 1;     // Q6_K f32 row triples: rows per step
    static constexpr int UT = R3 * U;                    // units per step
    static constexpr int T = (UT + 63) / 64;             // units per lane
    static constexpr int RB = KSB * (Q6 ? kBytesQ6_K : kBytesQ4_K);  // row bytes
    static constexpr int SPAN = R3 * RB;                 // bytes of a step's rows (Q6_K)
    static constexpr int RPS = (FL & (kSPair | kSRow2)) ? 2 : R3;  // rows per step
    // Q4_K rows are whole 16-byte transfers.  A Q6_K row starts s = 0, 4, 8
    // or 12 bytes past a 16-byte boundary: its slot takes the 16-byte
    // transfers from that boundary that end inside the row (F of them, F
    // depending on s), then 4-byte transfers of the rest; the row starts s
    // bytes into its slot.
    static constexpr int F_MIN = SPAN / 16, F_MAX = (SPAN + 12) / 16;
    static constexpr int SB = Q6 ? ((SPAN + 16 + 15) & ~15) : RPS * RB;  // slot bytes
    static constexpr int CH = (Q6 ? F_MIN * 16 : RB) / 1024;          // whole 1 KB chunks per row
    static constexpr int PL = (RB % 1024) / 16;          // Q4_K: lanes of the partial chunk
    static constexpr int NI = Q6 ? CH + 2 : RPS * (CH + (PL > 0 ? 1 : 0));  // DMA instructions per step
    static constexpr int NT = NW * 64;
    static constexpr bool F32 = (FL & kSF32) != 0;       // f32 activation slices, loaded by each lane
    static constexpr int ROUNDS = (FL & (kSXq | kSF32)) ? 0 : (M * KSB * 16 + NT - 1) / NT;  // staging rounds
    // the lane's activation slices (M tokens x T units) stay in registers when
    // they take at most 160 of them; otherwise each step reads them from LDS
    static constexpr int ACT_DW = F32 ? (Q6 ? 68 : 66) : Q6 ? 21 : 18;  // registers of one slice
    static constexpr bool XREG = M * T * ACT_DW <= 160;
    // staged activations of the M tokens: codes, block scales, 16-element sums
    static constexpr int QB = (M * K + 15) & ~15, DB = (M * KSB * 4 + 15) & ~15, BB = (M * (K / 16) * 2 + 15) & ~15;
    static constexpr int XQB = ((KSB * kBytesQ8_K + 1023) / 1024) * 1024;  // raw blocks, whole chunks
    static constexpr int AREA = (FL & kSXq) ? XQB : F32 ? 0 : QB + DB + BB;
    // ring slots: NB steps in flight, NS at the start (DEEP: twice NB)
    static constexpr int NS = DEEP ? 2 * NB : NB;
    static constexpr size_t lds() { return (size_t)AREA + (size_t)NW * NS * SB; }
    static_assert(Q6 ? (RB % 4 == 0 && F_MIN - 64 * CH >= 1 && F_MAX - 64 * CH <= 64)
                     : RB % 16 == 0,
                  "16-byte DMA lanes; Q6_K: one partial chunk of at least one lane");
    static_assert(!Q6 || (FL & (kSPair | kSXq)) == 0, "Q6_K rows: staged activations, no pairs");
    static_assert(AREA + (size_t)NW * NS * SB + 8 * NW <= 160 * 1024, "the ring and the staging fit the gfx950 LDS");
    static_assert(ROUNDS <= 8, "the staging loads of every round are in flight at the start");
    static_assert(NS * NI + 4 * ROUNDS * ((FL & 3) ? 2 : 1) + (F32 ? 16 * M * T : 0) <= 63, "vmcnt range");
    static_assert(!F32 || ((FL & ~(kSF32 | kSArgmax | kSRow3)) == 0 && XREG), "f32 activations: plain rows, slices in registers");
    static_assert(!(FL & kSRow3) || (Q6 && F32 && M == 1), "row triples: one token of Q6_K f32 logits");
    static_assert(!(FL & kSArgmax) || (F32 && M == 1), "argmax keys: one f32 token");
    static_assert(AREA % 16 == 0, "slot alignment");
    static_assert(M == 1 || (FL & ~(kSF32 | kSRow2)) == 0, "several tokens: plain projections");
    static_assert(XREG || (FL & kSXq) == 0, "Q8_K block input: the slices in registers");
    static_assert(!(FL & kSRow2) || ((FL & ~(kSRow2 | 1)) == 0 && !Q6),
                  "row pairs: Q4_K projections, RMSNorm prologue (one token) or none");
};

template <int KSB, int NW, int NB, int FL, bool DEEP, int M = 1, int TYPE = kTypeQ4_K>
__global__ __launch_bounds__(NW * 64) void gemv_stream_q4k(StreamArgs a) {
    using G = StreamGeom<KSB, NW, NB, FL, DEEP, M, TYPE>;
    constexpr bool Q6 = G::Q6;
    constexpr int PRO = FL & 3;
    constexpr bool kRes = (FL & kSRes) != 0, kPair = (FL & kSPair) != 0, kXq = (FL & kSXq) != 0;
    constexpr bool kF32 = G::F32, kArgmax = (FL & kSArgmax) != 0, kRow2 = (FL & kSRow2) != 0;
    constexpr bool kRow3 = (FL & kSRow3) != 0;
    constexpr int NS = G::NS;
    extern __shared__ __align__(16) uint8_t smem[];
    int8_t *lq = reinterpret_cast<int8_t *>(smem);
    float *ld = reinterpret_cast<float *>(smem + G::QB);
    int16_t *lbs = reinterpret_cast<int16_t *>(smem + G::QB + G::DB);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *ring = smem + G::AREA + wave * (NS * G::SB);
    const uint32_t ring_lds = s_lds_addr(ring);
    // the wave's index in the grid: workgroup-major (a workgroup takes NW
    // adjacent rows of each step) or wave-major (adjacent rows go to adjacent
    // workgroups, so the rows of a last partial step spread over every CU)
    const int gw = a.cu_major ? wave * (int)gridDim.x + (int)blockIdx.x : (int)blockIdx.x * NW + wave;
    const int TW = gridDim.x * NW;
    const int last = a.nrows;

    // the matrix of a step and its row (scalar selects over the arguments)
    struct Mat {
        const uint8_t *w;
        int n_out, row;
    };
    auto locate = [&](int step) {
        Mat m{a.w[0], a.n_out[0], step};
#pragma unroll
        for (int z = 1; z < kStreamMaxMats; ++z) {
            const bool in = !kPair && z < a.nmat && step >= a.row_start[z];
            m.w = in ? a.w[z] : m.w;
            m.n_out = in ? a.n_out[z] : m.n_out;
            m.row = in ? step - a.row_start[z] : m.row;
        }
        return m;
    };
    auto issue = [&](int b, int step) {
        const bool ok = step < last;
        const Mat m = locate(ok ? step : 0);
        // row pairs: step row r of the matrix is rows 2r and 2r + 1
        const uint32_t so = ok ? (uint32_t)m.row * (kRow2 ? 2u : 1u) * (uint32_t)G::SPAN : 0u;
        const uint32_t vo = ok ? (uint32_t)lane * 16u : 0x7ff00000u;
        if constexpr (Q6) {
            // every transfer lies inside the row or the rows before it
            const uint32_t sh = so & 15u, a0 = so - sh, end = sh + (uint32_t)G::SPAN;
            const int F = (int)(end >> 4), tail = (int)((end & 15u) >> 2);
            const v4u_t rs = s_rsrc(m.w, (uint32_t)m.n_out * G::RB);
            const uint32_t dst = ring_lds + b * G::SB;
            if constexpr (kRow3) {
                // the last triple may pass the matrix end: the offsets go in the
                // range-checked VGPR offset (bytes past n_out rows read 0)
                const uint32_t t0 = 16u * (uint32_t)F;
#pragma unroll
                for (int k = 0; k < G::CH; ++k)
                    s_dma16_nt(dst + k * 1024, ok ? a0 + k * 1024u + (uint32_t)lane * 16u : 0x7ff00000u, rs, 0u);
                if (lane < F - 64 * G::CH)
                    s_dma16_nt(dst + G::CH * 1024, ok ? a0 + G::CH * 1024u + (uint32_t)lane * 16u : 0x7ff00000u, rs, 0u);
                const uint32_t v4 = tail > 0 ? a0 + t0 + (uint32_t)lane * 4u : a0 + t0 - 4u;
                if (lane < (tail > 0 ? tail : 1)) s_dma4_nt(dst + t0, ok ? v4 : 0x7ff00000u, rs, 0u);
                return;
            }
#pragma unroll
            for (int k = 0; k < G::CH; ++k) s_dma16_nt(dst + k * 1024, vo, rs, a0 + k * 1024);
            if (lane < F - 64 * G::CH) s_dma16_nt(dst + G::CH * 1024, vo, rs, a0 + G::CH * 1024);
            // the row's last 0-12 bytes as dwords; none left: lane 0 reloads the
            // last dword of the 16-byte transfers past them (an issued
            // instruction either way, so every wait counts NI per step)
            const uint32_t t0 = 16u * (uint32_t)F;
            const uint32_t vo4 = ok ? (uint32_t)lane * 4u : 0x7ff00000u;
            if (lane < (tail > 0 ? tail : 1)) s_dma4_nt(dst + t0, vo4, rs, tail > 0 ? a0 + t0 : a0 + t0 - 4u);
            return;
        }
#pragma unroll
        for (int r = 0; r < G::RPS; ++r) {
            const v4u_t rs = s_rsrc(r == 0 || kRow2 ? m.w : a.w[1], (uint32_t)m.n_out * G::RB);
            const uint32_t dst = ring_lds + b * G::SB + r * G::RB;
            const uint32_t sr = so + (kRow2 ? (uint32_t)r * G::RB : 0u);
#pragma unroll
            for (int k = 0; k < G::CH; ++k) s_dma16_nt(dst + k * 1024, vo, rs, sr + k * 1024);
            if constexpr (G::PL > 0) {
                if (lane < G::PL) s_dma16_nt(dst + G::CH * 1024, vo, rs, sr + G::CH * 1024);
            }
        }
    };

    // 1. the inputs of the activation, then the ring's first rows
    const int tid = threadIdx.x, sub = tid & 15, bl = tid >> 4;
    constexpr int BPR = G::NT / 16;
    constexpr int RN = G::ROUNDS > 0 ? G::ROUNDS : 1;
    v4u_t xr[RN][4], yr[RN][4];
    // f32 activations: each lane's 64 floats of every unit pass and token
    // (Q4_K unit 4i+j: elements 256i+64j..+63; Q6_K unit (i, h, p): four
    // runs of 16 at 256i+128h+16p+32k, k = 0..3)
    v4u_t fr[kF32 ? M : 1][kF32 ? G::T : 1][16];
    if constexpr (kF32) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int t = 0; t < G::T; ++t) {
                const int uc = min(lane + 64 * t, G::UT - 1) % G::U;
                if constexpr (Q6) {
                    const float *px = a.x + (size_t)m * G::K + 256 * (uc >> 2) + 128 * ((uc >> 1) & 1) + 16 * (uc & 1);
#pragma unroll
                    for (int v = 0; v < 16; ++v) fr[m][t][v] = s_load16(px + 32 * (v >> 2) + 4 * (v & 3));
                } else {
                    const float *px = a.x + (size_t)m * G::K + 64 * uc;
#pragma unroll
                    for (int v = 0; v < 16; ++v) fr[m][t][v] = s_load16(px + 4 * v);
                }
            }
    } else if constexpr (kXq) {
        // Q8_K block bytes into LDS, 1 KB chunks over the waves
        const v4u_t rsx = s_rsrc(a.xq, (uint32_t)(KSB * kBytesQ8_K));
        constexpr int XCH = G::XQB / 1024;
        for (int c = wave; c < XCH; c += NW) s_dma16(s_lds_addr(smem) + c * 1024, lane * 16u, rsx, c * 1024u);
    } else {
#pragma unroll
        for (int r = 0; r < G::ROUNDS; ++r) {
            // block blk of the M tokens' [M][K] activation (token blk / KSB)
            const int blk = min(r * BPR + bl, M * KSB - 1);
            const float *px = a.x + blk * kQKK + 16 * sub;
#pragma unroll
            for (int k = 0; k < 4; ++k) xr[r][k] = s_load16(px + 4 * k);
            if constexpr (PRO != 0) {
                const float *py = PRO == 2 ? a.x2 + blk * kQKK + 16 * sub : a.nw + blk * kQKK + 16 * sub;
#pragma unroll
                for (int k = 0; k < 4; ++k) yr[r][k] = s_load16(py + 4 * k);
            }
        }
    }
    // every slot filled at the start: NS rows per wave in flight while the
    // activation is quantized, then NB once the steps begin
#pragma unroll
    for (int b = 0; b < NS; ++b) issue(b, gw + b * TW);
    s_wait_vm<NS * G::NI>();  // the activation inputs have arrived; the ring's rows may not have
    if constexpr (kXq) {
        __syncthreads();
    } else if constexpr (kF32) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int t = 0; t < G::T; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) asm volatile("" : "+v"(fr[m][t][v]));
    } else {
        // the loaded registers are complete only now: every use is ordered after the wait
#pragma unroll
        for (int r = 0; r < G::ROUNDS; ++r)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                asm volatile("" : "+v"(xr[r][k]));
                if constexpr (PRO != 0) asm volatile("" : "+v"(yr[r][k]));
            }
        // 2. Q8_K staging (quantize_q8_k_group), after the prologue
        float xs[RN][16], ys[RN][16];
#pragma unroll
        for (int r = 0; r < G::ROUNDS; ++r)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // whole-vector casts: a bit_cast of one ext-vector element reads element 0 in this clang
                const float4 f = __builtin_bit_cast(float4, xr[r][k]);
                xs[r][4 * k] = f.x; xs[r][4 * k + 1] = f.y; xs[r][4 * k + 2] = f.z; xs[r][4 * k + 3] = f.w;
                const float4 g = __builtin_bit_cast(float4, yr[r][k]);
                ys[r][4 * k] = g.x; ys[r][4 * k + 1] = g.y; ys[r][4 * k + 2] = g.z; ys[r][4 * k + 3] = g.w;
            }
        if constexpr (PRO == 2) {
#pragma unroll
            for (int r = 0; r < G::ROUNDS; ++r)
#pragma unroll
                for (int e = 0; e < 16; ++e) xs[r][e] = silu_f32(xs[r][e]) * ys[r][e];
        } else if constexpr (PRO == 1) {
            // RMSNorm (src/cpu_kernel.c:228-241): squares summed in double over the row (the
            // lanes of clamped past-the-end blocks add nothing), scale from the mean
            __shared__ double red[NW];
            double s = 0.0;
#pragma unroll
            for (int r = 0; r < G::ROUNDS; ++r) {
                double sr = 0.0;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const double v = (double)xs[r][e];
                    sr += v * v;
                }
                s += r * BPR + bl < KSB ? sr : 0.0;
            }
            s = wave_sum_f64(s);
            if (lane == 0) red[wave] = s;
            __syncthreads();
            double ss = 0.0;
#pragma unroll
            for (int w = 0; w < NW; ++w) ss += red[w];
            const float scale = rms_scale(ss, G::K, a.eps);
#pragma unroll
            for (int r = 0; r < G::ROUNDS; ++r)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float v = xs[r][e] * scale;
                    xs[r][e] = v * ys[r][e];
                }
        }
#pragma unroll
        for (int r = 0; r < G::ROUNDS; ++r)
            quantize_q8_k_group<G::NT>(xs[r], r * BPR + bl, M * KSB, KSB, G::K, sub, lq, ld, lbs);
        __syncthreads();
    }
    // the lane's activation slices, scale selectors and row offsets
    const ActLds act{lq, ld, lbs, G::K, KSB};
    using ActF32 = std::conditional_t<Q6, FmtQ6KF32::Act, FmtQ4KF32::Act>;
    using Act = std::conditional_t<kF32, ActF32, std::conditional_t<Q6, FmtQ6K::Act, FmtQ4K::Act>>;
    using Fmt = std::conditional_t<Q6, FmtQ6K, FmtQ4K>;
    Act xa[G::XREG ? M : 1][G::XREG ? G::T : 1];
    ScaleSel lc[G::T];
    uint32_t hoff[G::T], qoff[G::T];  // Q6_K: the unit's aligned byte offset, its shift (0 or 2)
    bool live[G::T];
    int unit[G::T], prow[G::T];  // the lane's unit of each pass and its row in the step
#pragma unroll
    for (int t = 0; t < G::T; ++t) {
        const int u = lane + 64 * t;
        live[t] = u < G::UT;
        const int gl = min(u, G::UT - 1);
        const int uc = gl % G::U;
        unit[t] = uc;
        prow[t] = gl / G::U;
        if constexpr (kXq) {
            act_from_blocks(smem, uc, xa[0][t]);
        } else if constexpr (kF32) {
            // the slice and sums of FmtQ4KF32::load_act / FmtQ6KF32::load_act
#pragma unroll
            for (int m = 0; m < M; ++m) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float4 f = __builtin_bit_cast(float4, fr[m][t][v]);
                    xa[m][t].x[4 * v] = f.x; xa[m][t].x[4 * v + 1] = f.y;
                    xa[m][t].x[4 * v + 2] = f.z; xa[m][t].x[4 * v + 3] = f.w;
                }
                if constexpr (Q6) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) xa[m][t].sx[k] = sum16(xa[m][t].x + 16 * k);
                } else {
                    xa[m][t].sx0 = sum16(xa[m][t].x) + sum16(xa[m][t].x + 16);
                    xa[m][t].sx1 = sum16(xa[m][t].x + 32) + sum16(xa[m][t].x + 48);
                }
            }
        } else if constexpr (G::XREG) {
#pragma unroll
            for (int m = 0; m < M; ++m) Fmt::load_act_lds(act, uc, m, xa[m][t]);
        }
        if constexpr (Q6) {
            // the unit's fields sit at sb + 4-byte multiples
            const uint32_t sb = (uint32_t)prow[t] * (uint32_t)G::RB + (uint32_t)(uc >> 2) * kBytesQ6_K;
            hoff[t] = sb & ~3u;
            qoff[t] = sb & 3u;  // v_alignbyte shift, bytes
        } else {
            lc[t] = scale_sel(uc & 3);
            hoff[t] = (uint32_t)(uc >> 2) * kBytesQ4_K;
            qoff[t] = hoff[t] + 16u + 32u * (uint32_t)(uc & 3);
        }
    }

    // token m's activation slice of unit pass t
    auto xslice = [&](int m, int t) -> Act {
        if constexpr (G::XREG) {
            return xa[m][t];
        } else {
            Act x;
            Fmt::load_act_lds(act, unit[t], m, x);
            return x;
        }
    };

    // 3. the epilogue words of the lane's step (step first + lane * TW), loaded ahead of use
    struct Epi {
        float b0, b1, r, b2;
    };
    auto lane_out = [&](int step, float *&out, int &row, const float *&bias, const float *&resid, int &n_out) {
        out = a.out[0];
        bias = a.bias[0];
        resid = a.resid[0];
        row = step;
        n_out = a.n_out[0];
#pragma unroll
        for (int z = 1; z < kStreamMaxMats; ++z) {
            const bool in = !kPair && z < a.nmat && step >= a.row_start[z];
            out = in ? a.out[z] : out;
            bias = in ? a.bias[z] : bias;
            resid = in ? a.resid[z] : resid;
            row = in ? step - a.row_start[z] : row;
            n_out = in ? a.n_out[z] : n_out;
        }
    };
    auto load_epi = [&](int first) {
        const int step = first + lane * TW;
        const bool ok = step < last;
        float *out;
        int row, n_out;
        const float *bias, *resid;
        lane_out(ok ? step : 0, out, row, bias, resid, n_out);
        Epi e{0.0f, 0.0f, 0.0f, 0.0f};
        if (ok) {
            if constexpr (kRow3) {
                e.b0 = bias != nullptr ? bias[3 * row] : 0.0f;
                e.b1 = bias != nullptr && 3 * row + 1 < n_out ? bias[3 * row + 1] : 0.0f;
                e.b2 = bias != nullptr && 3 * row + 2 < n_out ? bias[3 * row + 2] : 0.0f;
            } else if constexpr (kRow2) {
                e.b0 = bias != nullptr ? bias[2 * row] : 0.0f;
                e.b1 = bias != nullptr ? bias[2 * row + 1] : 0.0f;
            } else {
                e.b0 = bias != nullptr ? bias[row] : 0.0f;
            }
            if constexpr (kPair) e.b1 = a.bias[1] != nullptr ? a.bias[1][row] : 0.0f;
            if constexpr (kRes) e.r = resid != nullptr ? resid[row] : 0.0f;
        }
        return e;
    };
    // keep[m]: token m's total of step k (k % 64 = this lane); keep1[m]: the
    // step's second row (up of a pair, or the odd row of a row pair)
    float keep[M], keep1[M], keep2[M];
    unsigned long long best = 0ull;  // argmax: the lane's best key (score_key) so far
#pragma unroll
    for (int m = 0; m < M; ++m) keep[m] = keep1[m] = keep2[m] = 0.0f;
    auto flush = [&](int first, int n, const Epi &e) {
        const int step = first + lane * TW;
        float *out;
        int row, n_out;
        const float *bias, *resid;
        lane_out(step < last ? step : 0, out, row, bias, resid, n_out);
        if (lane < n && step < last) {
            // out = resid + (bias + dot) (src/native.c:2571-2580); pairs: silu(gate) * up
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = e.b0 + keep[m];
                float o = v;
                if constexpr (kRes) o = resid != nullptr ? e.r + v : v;
                if constexpr (kPair) o = silu_f32(v) * (e.b1 + keep1[m]);
                if constexpr (kRow2) {
                    out[(size_t)m * n_out + 2 * row] = o;
                    out[(size_t)m * n_out + 2 * row + 1] = e.b1 + keep1[m];
                    continue;
                }
                if constexpr (kRow3) {
                    const float o3[3] = {o, e.b1 + keep1[m], e.b2 + keep2[m]};
#pragma unroll
                    for (int r = 0; r < 3; ++r) {
                        const int ro = 3 * row + r;
                        if (ro < n_out) {
                            out[ro] = o3[r];
                            if constexpr (kArgmax) {
                                const unsigned long long key = score_key(o3[r], (unsigned)ro);
                                best = key > best ? key : best;
                            }
                        }
                    }
                    continue;
                }
                out[(size_t)m * n_out + row] = o;
                if constexpr (kArgmax) {
                    const unsigned long long key = score_key(o, (unsigned)row);
                    best = key > best ? key : best;
                }
            }
        }
    };
    Epi epi = load_epi(gw);

    // 4. one step (a row, or a gate/up pair) per ring slot.  Step k of the wave
    //    (row gw + k TW) sits in slot k % NS; once its bytes are in registers
    //    the slot of step k + NB - NS is free and takes step k + NB (before
    //    that, steps up to NS - 1 came with the start), then the lane partials
    //    of each row: per unit pass t, dead units 0.  WAIT: this wave's DMAs
    //    of later steps that may stay in flight.
    auto step_partials = [&](auto wait_c, int slot, int k, float (&p)[M][G::RPS][G::T]) {
        s_wait_vm<decltype(wait_c)::value>();
        if constexpr (Q6) {
            // the row starts (row * RB) & 15 bytes into its slot
            const int step = gw + k * TW;
            const Mat m = locate(step < last ? step : 0);
            const uint8_t *rb = ring + slot * G::SB + (((uint32_t)m.row * G::SPAN) & 15u);
            v4u_t A[G::T], B[G::T], H[G::T];
            uint32_t s0[G::T], s1[G::T], s2[G::T], dw[G::T];
#pragma unroll
            for (int t = 0; t < G::T; ++t) {
                const int u = unit[t], h = (u >> 1) & 1, pp = u & 1;
                const uint8_t *q = rb + hoff[t];
                A[t] = lds16_a2(q + 64 * h + 16 * pp, qoff[t]);
                B[t] = lds16_a2(q + 64 * h + 32 + 16 * pp, qoff[t]);
                H[t] = lds16_a2(q + 128 + 32 * h + 16 * pp, qoff[t]);
                s0[t] = lds_u32(q + 192 + 8 * h);
                s1[t] = lds_u32(q + 196 + 8 * h);
                s2[t] = lds_u32(q + 200 + 8 * h);
                dw[t] = lds_u32(q + 208);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (k + NB >= NS) issue((slot + NB) % NS, gw + (k + NB) * TW);  // uniform; slot == k % NS
#pragma unroll
            for (int t = 0; t < G::T; ++t) {
                const int u = unit[t];
                const uint32_t scx = __builtin_amdgcn_alignbyte(s1[t], s0[t], qoff[t]);
                const uint32_t scy = __builtin_amdgcn_alignbyte(s2[t], s1[t], qoff[t]);
                const uint32_t db = (dw[t] >> (8u * qoff[t])) & 0xffffu;
                if constexpr (kF32) {
                    // the f32-activation dot of every token, from a zero sum (as the fused kernel)
                    const FmtQ6K::W w{uint4{A[t][0], A[t][1], A[t][2], A[t][3]}, uint4{B[t][0], B[t][1], B[t][2], B[t][3]},
                                      uint4{H[t][0], H[t][1], H[t][2], H[t][3]}, uint2{scx, scy}, db};
                    Act xm[M];
                    float acc[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        xm[m] = xa[m][t];
                        acc[m] = 0.0f;
                    }
                    FmtQ6KF32::dotm<M>(w, u, xm, acc);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        p[m][0][t] = live[t] ? acc[m] : 0.0f;  // row triples: the rows are sorted out in finish
#pragma unroll
                        for (int r = 1; r < G::RPS; ++r) p[m][r][t] = 0.0f;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float v = q6k_unit(A[t], B[t], H[t], scx, scy, db, u & 1, xslice(m, t));
                        p[m][0][t] = live[t] ? v : 0.0f;
                    }
                }
            }
        } else {
            const uint8_t *sb = ring + slot * G::SB;
            v4u_t h[G::RPS][G::T], q0[G::RPS][G::T], q1[G::RPS][G::T];
#pragma unroll
            for (int r = 0; r < G::RPS; ++r)
#pragma unroll
                for (int t = 0; t < G::T; ++t) {
                    h[r][t] = *reinterpret_cast<const v4u_t *>(sb + r * G::RB + hoff[t]);
                    q0[r][t] = *reinterpret_cast<const v4u_t *>(sb + r * G::RB + qoff[t]);
                    q1[r][t] = *reinterpret_cast<const v4u_t *>(sb + r * G::RB + qoff[t] + 16);
                }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (k + NB >= NS) issue((slot + NB) % NS, gw + (k + NB) * TW);  // uniform; slot == k % NS
            if constexpr (kF32) {
                // the f32-activation dot of every token from one conversion of
                // the unit's weights, from a zero sum (as the fused kernel)
#pragma unroll
                for (int r = 0; r < G::RPS; ++r)
#pragma unroll
                    for (int t = 0; t < G::T; ++t) {
                        const FmtQ4K::W w{uint4{h[r][t][0], h[r][t][1], h[r][t][2], h[r][t][3]},
                                          uint4{q0[r][t][0], q0[r][t][1], q0[r][t][2], q0[r][t][3]},
                                          uint4{q1[r][t][0], q1[r][t][1], q1[r][t][2], q1[r][t][3]}};
                        Act xm[M];
                        float acc[M];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            xm[m] = xa[m][t];
                            acc[m] = 0.0f;
                        }
                        FmtQ4KF32::dotm<M>(w, min(lane + 64 * t, G::U - 1), xm, acc);
#pragma unroll
                        for (int m = 0; m < M; ++m) p[m][r][t] = live[t] ? acc[m] : 0.0f;
                    }
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int r = 0; r < G::RPS; ++r)
#pragma unroll
                        for (int t = 0; t < G::T; ++t) {
                            const float v = q4k_unit(h[r][t], q0[r][t], q1[r][t], xslice(m, t), lc[t]);
                            p[m][r][t] = live[t] ? v : 0.0f;
                        }
            }
        }
    };
    int k64 = 0, first = gw;
    auto advance = [&]() {
        if (++k64 == 64) {  // uniform
            s_wait_vm<0>();
            flush(first, 64, epi);
            first += 64 * TW;
            k64 = 0;
            epi = load_epi(first);
        }
    };
    // a row's total: per unit pass the wave's sum (the fused kernel's waves of
    // a split row), the passes added in order from 0
    auto finish = [&](float (&p)[M][G::RPS][G::T]) {
        float acc[M][G::RPS];
        if constexpr (M == 4 && G::T == 1) {
            // four tokens' rows in one tree (each total is its s_wave_total bit for bit)
#pragma unroll
            for (int r = 0; r < G::RPS; ++r) {
                const float v4[4] = {p[0][r][0], p[1][r][0], p[2][r][0], p[3][r][0]};
                const float tot = s_wave_total4(v4);
#pragma unroll
                for (int m = 0; m < 4; ++m) acc[m][r] = s_lane(tot, 16 * m);
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < G::RPS; ++r) {
                    if constexpr (kRow3) {
                        // unit j of each row to lane j (the lanes of pass 0 hold
                        // units 0-39 of row 0 and 0-23 of row 1, those of pass 1
                        // units 24-39 of row 1 and 0-39 of row 2), then the tree
                        // of one row of 40 units: the words of one row per step
                        const float a0 = p[m][0][0], a1 = p[m][0][1];
                        float v;
                        if (r == 0) {
                            v = lane < 40 ? a0 : 0.0f;
                        } else if (r == 1) {
                            const float x0 = __shfl(a0, (lane + 40) & 63, 64), x1 = __shfl(a1, (lane + 40) & 63, 64);
                            v = lane < 24 ? x0 : (lane < 40 ? x1 : 0.0f);
                        } else {
                            const float x2 = __shfl(a1, (lane + 16) & 63, 64);
                            v = lane < 40 ? x2 : 0.0f;
                        }
                        acc[m][r] = s_wave_total_3x16(v);
                    } else if constexpr (G::F32 && G::T == 1 && G::U > 32 && G::U <= 48) {
                        acc[m][r] = s_wave_total_3x16(p[m][r][0]);
                    } else if constexpr (G::T == 1) {
                        acc[m][r] = s_wave_total(p[m][r][0]);
                    } else if constexpr (G::T == 4) {
                        const float tot = s_wave_total4(p[m][r]);
                        float sum = 0.0f;
#pragma unroll
                        for (int t = 0; t < 4; ++t) sum += s_lane(tot, 16 * t);
                        acc[m][r] = sum;
                    } else {
                        float sum = 0.0f;
#pragma unroll
                        for (int t = 0; t < G::T; ++t) sum += s_wave_total(p[m][r][t]);
                        acc[m][r] = sum;
                    }
                }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) keep[m] = lane == k64 ? acc[m][0] : keep[m];
        if constexpr (kPair || kRow2 || kRow3) {
#pragma unroll
            for (int m = 0; m < M; ++m) keep1[m] = lane == k64 ? acc[m][1] : keep1[m];
        }
        if constexpr (kRow3) {
#pragma unroll
            for (int m = 0; m < M; ++m) keep2[m] = lane == k64 ? acc[m][2] : keep2[m];
        }
        advance();
    };
    // the first NS steps: their rows came with the start, so fewer stay in flight after each
    bool more = true;
    [&]<int... K>(std::integer_sequence<int, K...>) {
        ((more = more && gw + K * TW < last,
          more ? (void)([&] {
              float p[M][G::RPS][G::T];
              step_partials(std::integral_constant<int, (K < NS - NB ? NS - 1 - K : NB - 1) * G::NI>{}, K, K, p);
              finish(p);
          }())
               : (void)0),
         ...);
    }(std::make_integer_sequence<int, NS>{});
    // then NB in flight: one step per slot in turn (slot indices known at compile time)
    for (int k0 = NS; more; k0 += NS) {
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            more = more && gw + (k0 + b) * TW < last;
            if (more) {  // uniform
                float p[M][G::RPS][G::T];
                step_partials(std::integral_constant<int, (NB - 1) * G::NI>{}, b, k0 + b, p);
                finish(p);
            }
        }
    }
    s_wait_vm<0>();
    if (k64 > 0) flush(first, k64, epi);
    if constexpr (kArgmax) {
        // the workgroup's best key: each wave over its lanes, then the first
        // lane over the waves; one key per workgroup (at blockIdx.x)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        __shared__ unsigned long long wbest[NW];
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int k = 1; k < NW; ++k) best = wbest[k] > best ? wbest[k] : best;
            a.amax[blockIdx.x] = best;
        }
    }
}

template <int KSB, int NW, int NB, int FL, bool DEEP, int M, int TYPE>
hipError_t launch_stream_geom(const StreamArgs &a, hipStream_t st) {
    using G = StreamGeom<KSB, NW, NB, FL, DEEP, M, TYPE>;
    hipLaunchKernelGGL((gemv_stream_q4k<KSB, NW, NB, FL, DEEP, M, TYPE>), dim3(device_cus()), dim3(NW * 64), G::lds(),
                       st, a);
    return hipGetLastError();
}

template <int KSB, int NW, int NB, int FL, int M = 1, int TYPE = kTypeQ4_K>
hipError_t launch_stream(const StreamArgs &a, hipStream_t st) {
    // one workgroup per CU: the grid covers the chip once and every wave
    // strides over the rows.  Launches of at most three steps per wave fill
    // twice the ring at the start (measured: [4096 x 4096] 5.3 against
    // 5.5 us, [6144 x 2560] 5.5 against 6.1); longer ones keep NB in flight
    // from the start ([28672 x 4096] 14.5 against 14.7 us), and 8 KB rows
    // never take the deep start (12.4 against 11.0 us at [4096 x 14336];
    // measured again with the current staging: 10.8 against 9.6 us, and the
    // Q6_K [2560 x 9728] 9.8 against 8.9).
    const int grid = device_cus();
    const long long steps = ((long long)a.nrows + (long long)grid * NW - 1) / ((long long)grid * NW);
    if constexpr (KSB <= 16) {
        if (steps <= 3) return launch_stream_geom<KSB, NW, NB, FL, true, M, TYPE>(a, st);
    }
    return launch_stream_geom<KSB, NW, NB, FL, false, M, TYPE>(a, st);
}

// Q6_K rows: one token, staged activations; prologues and the residual as for Q4_K.
template <int KSB, int NW, int NB>
hipError_t launch_stream_q6k(int fl, const StreamArgs &a, hipStream_t st) {
    switch (fl) {
        case 0: return launch_stream<KSB, NW, NB, 0, 1, kTypeQ6_K>(a, st);
        case 1: return launch_stream<KSB, NW, NB, 1, 1, kTypeQ6_K>(a, st);
        case 2: return launch_stream<KSB, NW, NB, 2, 1, kTypeQ6_K>(a, st);
        case kSRes: return launch_stream<KSB, NW, NB, kSRes, 1, kTypeQ6_K>(a, st);
        case 2 | kSRes: return launch_stream<KSB, NW, NB, 2 | kSRes, 1, kTypeQ6_K>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// Plain projections of m = 2..4 staged tokens.  Rows of 4096 in launches
// of at most three steps per wave keep one row per wave in flight (measured,
// q+k+v [6144 x 4096] at 2 / 3 / 4 tokens: 6.5 / 7.9 / 8.5 us, against 7.3 /
// 8.1 / 9.1 with two slots filled twice at the start; o [4096 x 4096] 5.7 /
// 6.8 / 7.5 against 5.8 / 7.0 / 7.7); longer launches two.
template <int KSB, int NB, int TYPE = kTypeQ4_K, int FL = 0>
hipError_t launch_stream_tokens(int m, const StreamArgs &a, hipStream_t st) {
    if constexpr (KSB == 16 && NB == 2) {
        const long long per_gen = (long long)device_cus() * 8;
        if (((long long)a.nrows + per_gen - 1) / per_gen <= 3) {
            switch (m) {
                case 2: return launch_stream_geom<KSB, 8, 1, 0, false, 2, TYPE>(a, st);
                case 3: return launch_stream_geom<KSB, 8, 1, 0, false, 3, TYPE>(a, st);
                case 4: return launch_stream_geom<KSB, 8, 1, 0, false, 4, TYPE>(a, st);
                default: return hipErrorInvalidValue;
            }
        }
    }
    switch (m) {
        case 2: return launch_stream<KSB, 8, NB, FL, 2, TYPE>(a, st);
        case 3: return launch_stream<KSB, 8, NB, FL, 3, TYPE>(a, st);
        case 4: return launch_stream<KSB, 8, NB, FL, 4, TYPE>(a, st);
        default: return hipErrorInvalidValue;
    }
}

template <int KSB, int NW, int NB>
hipError_t launch_stream_flags(int fl, const StreamArgs &a, hipStream_t st) {
    switch (fl) {
        case 0: return launch_stream<KSB, NW, NB, 0>(a, st);
        case 1: return launch_stream<KSB, NW, NB, 1>(a, st);
        case 2: return launch_stream<KSB, NW, NB, 2>(a, st);
        case kSRes: return launch_stream<KSB, NW, NB, kSRes>(a, st);
        case 2 | kSRes: return launch_stream<KSB, NW, NB, 2 | kSRes>(a, st);
        case kSPair: return launch_stream<KSB, NW, NB, kSPair>(a, st);
        case 1 | kSPair: return launch_stream<KSB, NW, NB, 1 | kSPair>(a, st);
        case kSXq: return launch_stream<KSB, NW, NB, kSXq>(a, st);
        default: break;
    }
    if constexpr (KSB == 10 && NB == 1) {
        if (fl == kSRow2) return launch_stream<KSB, NW, NB, kSRow2>(a, st);
        if (fl == (1 | kSRow2)) return launch_stream<KSB, NW, NB, 1 | kSRow2>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Kernel choice for the launches this kernel covers (the
// library's edgexpu_hip_set_gemv_mode): 0 by launch size, 1 the fused kernel,
// 2 this one.  Both give the same outputs bit for bit.
static int g_gemv_mode = 0;
void set_gemv_stream_mode(int mode) { g_gemv_mode = mode; }
int gemv_stream_mode() { return g_gemv_mode; }

// True when the streaming GEMV can take (type, K, m).
// code: prologue (bits 0-1), residual (4), gate/up pairs (8); staged: f32
// tokens (not Q8_K block bytes).  Q4_K: one token of rows of 2560, 4096 or
// 14336, or plain projections of m = 2..4 staged tokens of those rows.
// Q6_K: staged tokens of rows of 9728 (the hybrid ~4B down projection), one
// (any variant but pairs) or two to four (plain projections).
bool gemv_stream_supported(int type, int K, int m, int code, bool staged) {
    if (type == kTypeQ4_K) {
        if (m == 1) return K == 2560 || K == 4096 || K == 14336;
        return m >= 2 && m <= 4 && staged && code == 0 && (K == 2560 || K == 4096 || K == 14336);
    }
    if (type == kTypeQ6_K) return K == 9728 && staged && (m == 1 ? (code & 8) == 0 : m <= 4 && code == 0);
    return false;
}

// True when the streaming GEMV runs a launch of `rows` rows (pairs: gate and
// up rows together) of (type, K, m).  By size, as measured on one MI355X
// (launch sweep over distinct weights, both kernels in one run): K = 2560
// and 4096 at every size swept, 1024 rows up (e.g. [28672 x 4096] 14.5
// against 16.0 us, [4096 x 4096] 5.2 against 5.7, [1024 x 4096] 4.4 against
// 5.0), K = 14336 from 2048 rows (7.7 against 7.0 us at 1024 rows, 8.8
// against 8.8 at 2048, 11.2 against 12.4 at 4096).
// The rows go to LDS as 16-byte DMA transfers from 16-byte-aligned
// addresses, so every matrix must start at one; others take the fused kernel.
bool gemv_stream_take(int type, int K, int m, long long rows, int nmat, const uint8_t *const *w, int code,
                      bool staged) {
    if (!gemv_stream_supported(type, K, m, code, staged) || g_gemv_mode == 1) return false;
    for (int z = 0; z < nmat; ++z)
        if (((uintptr_t)w[z] & 15u) != 0) return false;
    // a matrix's rows are addressed by 32-bit buffer offsets
    if (rows * (long long)(K / kQKK) * (type == kTypeQ6_K ? kBytesQ6_K : kBytesQ4_K) >= (1ll << 32)) return false;
    if (g_gemv_mode == 2) return true;
    // Q6_K rows of 9728 from 2048 rows (measured: 10.2 against 11.4 us at
    // 2560 rows, 18.9 against 25.1 at 9728; 7.4 against 6.5 at 1024; two /
    // three / four tokens of 2560 rows 12.8 / 15.6 / 18.2 against 17.9 /
    // 17.9 / 18.9 us for a quantize launch and the fused kernel)
    if (type == kTypeQ6_K) return rows >= 2048;
    // Q4_K rows of 14336 from 2048 rows (two / three tokens of 4096 rows:
    // 13.8 / 17.1 against 18.2 / 21.1 us), four tokens at any size (the other
    // path there is the generic GEMV: 15.0 against 22.5 us at 1024 rows)
    const long long bytes = rows * (long long)(K / kQKK) * kBytesQ4_K;
    return K != 14336 || bytes >= kStreamMinBytes14336 || m == 4;
}

// nmat Q4_K matrices against one token (m = 1) or the plain projection of
// m = 2..4 tokens ([m][K] f32 x; out[z] is [m][n_out[z]]): x f32 (quantized in the kernel, after
// the prologue pro: 1 RMSNorm with nw / eps, 2 SiLU-mul with x2) or xq (Q8_K
// block bytes); resid (per matrix, may be null) added after the bias; pair:
// nmat = 2 (gate, up), out[0] = silu(gate) * up.
hipError_t launch_gemv_stream(int type, int nmat, const uint8_t *const *w, const int *n_out,
                              const float *const *bias, const float *const *resid, float *const *out, int K, int m,
                              const float *x, const uint8_t *xq, const float *x2, const float *nw, float eps, int pro,
                              bool pair, hipStream_t st) {
    bool any_resid = false;
    for (int z = 0; z < nmat && resid != nullptr; ++z) any_resid = any_resid || resid[z] != nullptr;
    const int code = (pro & 3) | (any_resid ? kSRes : 0) | (pair ? kSPair : 0);
    if (!gemv_stream_supported(type, K, m, code, x != nullptr) || nmat < 1 || nmat > kStreamMaxMats)
        return hipErrorInvalidValue;
    if ((x == nullptr) == (xq == nullptr) || (xq != nullptr && (pro != 0 || pair))) return hipErrorInvalidValue;
    if (pair && (nmat != 2 || n_out[0] != n_out[1])) return hipErrorInvalidValue;
    const long long rb = (long long)(K / kQKK) * (type == kTypeQ6_K ? kBytesQ6_K : kBytesQ4_K);
    for (int z = 0; z < nmat; ++z)
        if (((uintptr_t)w[z] & 15u) != 0 || n_out[z] < 0 || (long long)n_out[z] * rb >= (1ll << 32))
            return hipErrorInvalidValue;
    // rows of 2560 (and rows of 4096 at 2-4 tokens), no residual, long
    // launches: two adjacent rows of a matrix per step (the steps and
    // row_start count row pairs) where every wave takes at least four pairs
    // and the longest wave takes no more rows than with single rows
    bool row2 = type == kTypeQ4_K && (K == 2560 || (K == 4096 && m > 1)) && !pair && !any_resid && xq == nullptr &&
                (pro & 3) <= 1;
    long long all_rows = 0;
    for (int z = 0; z < nmat; ++z) {
        row2 = row2 && n_out[z] % 2 == 0;
        all_rows += n_out[z];
    }
    if (row2) {
        const long long waves = (long long)device_cus() * 8, pairs = all_rows / 2;
        row2 = pairs >= 4 * waves && 2 * ((pairs + waves - 1) / waves) <= (all_rows + waves - 1) / waves;
    }
    StreamArgs a{};
    a.nmat = pair ? 1 : nmat;
    int rows = 0;
    bool any_res = false;
    for (int z = 0; z < nmat; ++z) {
        a.w[z] = w[z];
        a.bias[z] = bias != nullptr ? bias[z] : nullptr;
        a.resid[z] = resid != nullptr ? resid[z] : nullptr;
        a.out[z] = out[z];
        a.n_out[z] = n_out[z];
        any_res = any_res || a.resid[z] != nullptr;
    }
    for (int z = 0; z < a.nmat; ++z) {
        a.row_start[z] = rows;
        rows += row2 ? n_out[z] / 2 : n_out[z];
    }
    for (int z = a.nmat; z <= kStreamMaxMats; ++z) a.row_start[z] = rows;
    a.nrows = rows;
    // rows of 8 KB whose last step leaves waves idle: wave-major, so every
    // CU streams the same bytes ([2560 x 9728] Q6_K: 9.1 against 10.1 us;
    // shorter rows measured no faster: [1024 x 2560] 3.61 against 3.49,
    // [9728 x 2560] 6.3 against 6.15)
    a.cu_major = rb >= 4096 && rows % (device_cus() * 8) != 0;
    a.x = x;
    a.xq = xq;
    a.x2 = x2;
    a.nw = nw;
    a.eps = eps;
    if (any_res && pair) return hipErrorInvalidValue;
    const int fl = xq != nullptr ? kSXq : ((pro & 3) | (any_res ? kSRes : 0) | (pair ? kSPair : 0));
    // Q6_K rows of 9728 (8 KB): one slot per wave, no deep start (measured on
    // [2560 x 9728]: 10.2 us; a deep start 11.6, two slots 11.9, 12 waves
    // per CU 10.2 but 13.2 at 4096 rows)
    if (type == kTypeQ6_K)
        return m > 1 ? launch_stream_tokens<38, 1, kTypeQ6_K>(m, a, st) : launch_stream_q6k<38, 8, 1>(fl, a, st);
    if (m > 1) {
        switch (K) {
            case 2560:
                if (row2) return launch_stream_tokens<10, 1, kTypeQ4_K, kSRow2>(m, a, st);
                return launch_stream_tokens<10, 2>(m, a, st);
            case 4096:
                // row pairs: gate+up [28672 x 4096] at 2 / 4 tokens 14.7 / 18.5 -> 13.8 / 17.4 us
                if (row2) return launch_stream_tokens<16, 1, kTypeQ4_K, kSRow2>(m, a, st);
                return launch_stream_tokens<16, 2>(m, a, st);
            default: return launch_stream_tokens<56, 1>(m, a, st);
        }
    }
    // measured on the Llama-3-8B / hybrid decode shapes: 8 waves per CU, two
    // slots per wave, one slot where a row is 8 KB (K = 14336: two, 12.7
    // against 10.9 us at [4096 x 14336]).  Row pairs of 2560 (2880 bytes a
    // step) take one slot: gate+up [19456 x 2560] 8.07 against 8.9 us with
    // single rows (two slots of pairs 8.27, three 8.8); pairs of rows of
    // 4096 were no faster ([28672 x 4096] 12.8-13.1 against 12.8 us).
    switch (K) {
        case 2560:
            if (row2) return launch_stream_flags<10, 8, 1>(fl | kSRow2, a, st);
            return launch_stream_flags<10, 8, 2>(fl, a, st);
        case 4096: return launch_stream_flags<16, 8, 2>(fl, a, st);
        default: return launch_stream_flags<56, 8, 1>(fl, a, st);
    }
}

// True when the streaming GEMV runs the f32-activation product (the logits
// dot, src/native.c:445-462) of m tokens against the rows at w: Q4_K rows of
// 4096 or Q6_K rows of 2560, one or two tokens, the matrix 16-byte aligned.
// Measured on [128256 x 4096] Q4_K against the fused kernel: one token 57.6
// against 70.7 us (61.5 against 71.9 with the argmax keys and their
// reduction), two tokens 78.1 against 113.8; both kernels give the same
// words.
bool gemv_stream_f32_take(int type, int K, int m, const uint8_t *w, int n_out) {
    if (g_gemv_mode == 1 || m < 1 || m > 2) return false;
    if (!(type == kTypeQ4_K && K == 4096) && !(type == kTypeQ6_K && K == 2560)) return false;
    // rows addressed by 32-bit buffer offsets
    const long long rb = (long long)(K / kQKK) * (type == kTypeQ6_K ? kBytesQ6_K : kBytesQ4_K);
    return ((uintptr_t)w & 15u) == 0 && n_out >= 1 && (long long)n_out * rb < (1ll << 32);
}

// scores[t][row] = bias[row] + the f32-activation dot of token t (xf [m][K])
// with Q4_K row `row`; amax (one token): each workgroup's greedy-argmax key
// (score_key) at amax[blockIdx.x], *nparts keys.
hipError_t launch_gemv_stream_f32(int type, int K, int m, const uint8_t *w, int n_out, const float *bias,
                                  float *out, const float *xf, unsigned long long *amax, int *nparts, hipStream_t st) {
    if (!(type == kTypeQ4_K && K == 4096) && !(type == kTypeQ6_K && K == 2560)) return hipErrorInvalidValue;
    if (m < 1 || m > 2 || (amax != nullptr && m != 1) || ((uintptr_t)w & 15u) != 0 || n_out < 1 ||
        (long long)n_out * (K / kQKK) * (type == kTypeQ6_K ? kBytesQ6_K : kBytesQ4_K) >= (1ll << 32))
        return hipErrorInvalidValue;
    StreamArgs a{};
    a.nmat = 1;
    a.w[0] = w;
    a.bias[0] = bias;
    a.out[0] = out;
    a.n_out[0] = n_out;
    for (int z = 1; z <= kStreamMaxMats; ++z) a.row_start[z] = n_out;
    a.nrows = n_out;
    a.x = xf;
    a.amax = amax;
    if (nparts != nullptr) *nparts = device_cus();
    // one token: 16 waves per CU, one row each in flight (the f32 dot's
    // arithmetic wants the waves; measured 57.6 us against 59.2-65.0 with 8
    // waves and two to four slots); two tokens (two activation slices per
    // lane): 8 waves, three slots (78.1 against 81.2 with two)
    // Q6_K rows of 2560 ([151936 x 2560]) at one token: three rows per step,
    // their 120 units in two passes of 64 lanes (one row per step leaves 24
    // of 64 lanes idle on every row), 8 waves per CU (two activation slices
    // per lane); with the argmax keys one slot per wave, 69-72 against 84-86
    // us for 16 waves of one row per step; scores only two slots, 75-77
    // against 96-97 (one row per step: 77.8-80.5 against 86.5-87.5 fused in
    // the bench's step; it stays for a matrix whose last triple would pass
    // the 32-bit offset range).  Two tokens: 8 waves, two slots (108.9
    // against 147.9).
    const long long rb6 = (long long)(K / kQKK) * kBytesQ6_K;
    if (type == kTypeQ6_K && m == 1 && (long long)n_out * rb6 + 3 * rb6 < (1ll << 32)) {
        a.nrows = (n_out + 2) / 3;
        for (int z = 1; z <= kStreamMaxMats; ++z) a.row_start[z] = a.nrows;
        if (amax != nullptr) return launch_stream_geom<10, 8, 1, kSF32 | kSArgmax | kSRow3, false, 1, kTypeQ6_K>(a, st);
        return launch_stream_geom<10, 8, 2, kSF32 | kSRow3, false, 1, kTypeQ6_K>(a, st);
    }
    if (type == kTypeQ6_K) {
        if (amax != nullptr) return launch_stream_geom<10, 16, 1, kSF32 | kSArgmax, false, 1, kTypeQ6_K>(a, st);
        return m == 1 ? launch_stream_geom<10, 16, 1, kSF32, false, 1, kTypeQ6_K>(a, st)
                      : launch_stream_geom<10, 8, 2, kSF32, false, 2, kTypeQ6_K>(a, st);
    }
    if (amax != nullptr) return launch_stream_geom<16, 16, 1, kSF32 | kSArgmax, false, 1, kTypeQ4_K>(a, st);
    return m == 1 ? launch_stream_geom<16, 16, 1, kSF32, false, 1, kTypeQ4_K>(a, st)
                  : launch_stream<16, 8, 3, kSF32, 2>(a, st);
}

}  // namespace exq
