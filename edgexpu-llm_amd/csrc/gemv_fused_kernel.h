// Fused decode GEMV: edgexpu_cpu_linear_quant_batch (src/cpu_kernel.c:545-644)
// for m <= 4 tokens in ONE launch per group of projections that share an
// input.
//
//  * The activation quantizer runs inside the kernel: every workgroup turns
//    the f32 input into Q8_K (K-quant weights) or Q8_0 (Q8_0 weights) codes in
//    LDS with exactly the arithmetic of quantize.hip (bit-identical to
//    src/gguf_dot_q8.c:276-324,360-412), while the loads of its first weight
//    tile are already in flight.  No separate quantize launch.
//  * Lanes own fixed units of K (a unit is 64 elements of a super-block, or
//    one Q8_0 block), so each lane reads its activation slice from LDS once
//    and applies it to the R rows of its slot.  Long rows are split across
//    KS waves of the workgroup; the KS partial sums meet in LDS.
//  * One tile (S*R rows, S = 64/G slots per wave) per wave and no software
//    pipelining: the register budget stays near the generic kernel's, so
//    eight waves per SIMD stay resident and the whole matrix is requested in
//    one generation of workgroups; NW waves per workgroup share one staging.
//  * Up to 4 matrices with the same K and type (q/k/v, gate/up) are one
//    launch: tiles are numbered across the matrices.
#pragma once

#include <stdlib.h>

#include <type_traits>

#include "formats.h"

namespace exq {

constexpr int kFusedMaxMats = 4;

// Greedy-argmax keys one f32 logits launch writes at most (one per workgroup).
constexpr int kFusedArgmaxParts = 4096;

struct FusedArgs {
    int nmat;
    const uint8_t *w[kFusedMaxMats];
    const float *bias[kFusedMaxMats];
    float *out[kFusedMaxMats];       // [m][n_out[z]]
    int n_out[kFusedMaxMats];
    int tile_start[kFusedMaxMats + 1];
    size_t row_bytes;
    int K;
    int nblk;
    int U;       // units per row
    int G;       // lanes per row slot (16, 32 or 64)
    int KS;      // waves splitting a row's units (1, 2, 4 or 8; divides NW)
    int ntiles;  // total row tiles over all matrices (a tile is S*R rows)
    int m;
    const float *x;        // [m][K] f32 activations (staged kernels)
    const uint8_t *xq;     // or: activations already quantized, reference block bytes
    size_t xq_stride;      //     (Q8_0: 34 B per 32, Q8_K: 292 B per 256), token t at xq + t*xq_stride
    const float *xf;       // or (f32-activation formats): x [m][K] f32
    const float *resid[kFusedMaxMats];  // added to each output after its bias ([m][n_out[z]]; null: none)
    const float *x2;       // SiLU-mul prologue: the staged activation is silu(x) * x2
    const float *nw;       // RMSNorm prologue: the staged activation is rmsnorm(x; nw, eps)
    float eps;
    unsigned long long *amax;  // argmax epilogue: one key per workgroup, at blockIdx.x
    int amax_cap;              //     keys amax holds (the grid is clamped to it)
};

// Greedy-argmax key of a score (src/native.c:2355-2396): order-preserving
// score bits above ~index, so the largest key is the largest score at the
// lowest index; NaN and -inf give 0 and never win.
__device__ __forceinline__ unsigned long long score_key(float s, unsigned idx) {
    // selects only (no branch in the store path of the GEMV's epilogue);
    // -0.0 and +0.0 compare equal in the reference's `score > best`, so they
    // share one key (the lower index then wins)
    const uint32_t b = s == 0.0f ? 0u : __float_as_uint(s);
    const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const bool wins = s > -INFINITY;
    return ((unsigned long long)(wins ? u : 0u) << 32) | (unsigned long long)(wins ? ~idx : 0u);
}

struct WSrc {
    const uint8_t *w;
    size_t row_bytes;
};

// v_cvt_i32_f32 on a value already rounded to an integer: NaN gives 0,
// out-of-range values saturate (inline assembly: the hardware's result for
// every input, which a C conversion leaves undefined for NaN).
__device__ __forceinline__ int cvt_f32_i32(float v) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Q8_K quantization of x into LDS (src/gguf_dot_q8.c:360-412) for the
// GEMV's own use.  16 threads per 256-element block, each owning one
// 16-element group (so its int16 sum needs no reduction); NT/16 blocks per
// round, one round in registers at a time (the register budget of the
// staging decides the kernel's occupancy).
//
// The reference's scale is iscale = -127 / max with max the first element
// of largest |x|, sign included.  Here max is |max| for every block: a block
// whose first largest element is negative gets the negated codes, bsums and
// d of the reference's block (rint and the clamp are odd functions, and
// 1 / -iscale = -d), and every use of the block in a dot product is a
// product of d with an integer sum of codes (dot_q4_k_q8_k / dot_q6_k_q8_k
// and the other K-quant dots), unchanged word for word when both factors
// change sign.  So the outputs are the reference's; only the sign search
// (a compare and a select per element, a 16-lane minimum per block) is gone.
// quantize_q8_k_kernel, whose bytes leave the kernel, keeps the reference's
// signs.  With iscale finite every |iscale * x| is at most 127 (|x| <= amax)
// or NaN, so rint and the hardware conversion (NaN -> 0, as lrintf's
// LONG_MIN truncates to 0) give the codes with no clamp; with iscale
// infinite (amax below ~3.7e-37) every product is infinite or NaN and every
// code is 0.  Codes are packed four to a word with byte permutes and their
// sums taken with sdot4 against ones.
template <int NT>
__device__ __forceinline__ void quantize_q8_k_group(const float (&xs)[16], int blk, int total, int nb, int K,
                                                    int sub, int8_t *lq, float *ld, int16_t *lbs) {
    const bool valid = blk < total;  // uniform over each 16-thread group
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(xs[e]));
    const float amax = row16_max(am);
    if (!valid) return;
    const int tok = blk / nb, b = blk - tok * nb;
    const float iscale = -127.0f / amax;
    const bool codes = amax > 0.0f && fabsf(iscale) < INFINITY;  // uniform over the group
    uint32_t words[4];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = cvt_f32_i32(rintf(iscale * xs[4 * k + e]));
        // bytes q0..q3, low to high
        const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q[1], (uint32_t)q[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q[3], (uint32_t)q[2], 0x04000c0cu);
        words[k] = codes ? (lo | hi) : 0u;
        sum = __builtin_amdgcn_sdot4((int)words[k], 0x01010101, sum, false);
    }
    const float d = amax > 0.0f ? 1.0f / iscale : 0.0f;
    *reinterpret_cast<uint4 *>(lq + (size_t)tok * K + (size_t)b * kQKK + 16 * sub) =
        make_uint4(words[0], words[1], words[2], words[3]);
    lbs[(size_t)tok * (K / 16) + 16 * b + sub] = (int16_t)sum;
    if (sub == 0) ld[tok * nb + b] = d;
}

// This thread's 16 elements of the round starting at block blk0 (clamped:
// every thread issues the same loads) from src, whose tokens are tok_stride
// elements apart (the activation: K; the RMSNorm weights: 0).
template <int NT>
__device__ __forceinline__ void stage_q8_k_load_from(const float *src, size_t tok_stride, const FusedArgs &a,
                                                     int blk0, float (&xs)[16]) {
    const int tid = threadIdx.x, sub = tid & 15, bl = tid >> 4;
    const int nb = a.K / kQKK, total = a.m * nb;
    const int cb = min(blk0 + bl, total - 1);
    const int tok = cb / nb;
    const float4 *p =
        reinterpret_cast<const float4 *>(src + (size_t)tok * tok_stride + (size_t)(cb - tok * nb) * kQKK + 16 * sub);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 u = p[k];
        xs[4 * k] = u.x; xs[4 * k + 1] = u.y; xs[4 * k + 2] = u.z; xs[4 * k + 3] = u.w;
    }
}
template <int NT>
__device__ __forceinline__ void stage_q8_k_load(const FusedArgs &a, int blk0, float (&xs)[16]) {
    stage_q8_k_load_from<NT>(a.x, (size_t)a.K, a, blk0, xs);
}

// The prologue's second input for this thread's elements, loaded with the
// activation: x2 (SiLU-mul) or the RMSNorm weights.
template <int PRO, int NT>
__device__ __forceinline__ void stage_pro_load16(const FusedArgs &a, int blk0, float (&ys)[16]) {
    if constexpr (PRO == 2) stage_q8_k_load_from<NT>(a.x2, (size_t)a.K, a, blk0, ys);
    else if constexpr (PRO == 1) stage_q8_k_load_from<NT>(a.nw, 0, a, blk0, ys);
}

// The staging prologue on n elements of one thread (src/native.c:2529,
// 2576-2578): SiLU-mul, act = silu(x) * x2; RMSNorm (one token, every
// element of the row loaded in this round), act = (x * scale) * w with scale
// from the double sum of squares over the workgroup (lanes whose loads were
// clamped past the row's end contribute nothing).
template <int PRO, int NW, int N>
__device__ __forceinline__ void stage_pro_apply(const FusedArgs &a, float (&xs)[N], const float (&ys)[N], bool valid) {
    if constexpr (PRO == 2) {
#pragma unroll
        for (int e = 0; e < N; ++e) xs[e] = silu_f32(xs[e]) * ys[e];
    } else if constexpr (PRO == 1) {
        __shared__ double red[NW];
        double s = 0.0;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const double v = (double)xs[e];
            s += v * v;
        }
        s = wave_sum_f64(valid ? s : 0.0);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        double ss = 0.0;
#pragma unroll
        for (int w = 0; w < NW; ++w) ss += red[w];
        const float scale = rms_scale(ss, a.K, a.eps);
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float v = xs[e] * scale;
            xs[e] = v * ys[e];
        }
    }
}

// Q8_K quantization of x into LDS, 16 threads per 256-block; the first
// round's elements (xs0) were loaded by the caller before the first weight
// tile, so they do not queue behind it.
template <int NT, int PRO = 0>
__device__ void stage_q8_k(const FusedArgs &a, const float (&xs0)[16], const float (&ys0)[16], int8_t *lq,
                           float *ld, int16_t *lbs) {
    constexpr int BPR = NT / 16;  // blocks per round
    const int tid = threadIdx.x, sub = tid & 15, bl = tid >> 4;
    const int nb = a.K / kQKK, total = a.m * nb;
    {
        float xs[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) xs[e] = xs0[e];
        stage_pro_apply<PRO, NT / 64>(a, xs, ys0, bl < total);
        quantize_q8_k_group<NT>(xs, bl, total, nb, a.K, sub, lq, ld, lbs);
    }
    for (int blk0 = BPR; blk0 < total; blk0 += BPR) {  // RMSNorm prologue: never (one round)
        float xs[16], ys[16];
        stage_q8_k_load<NT>(a, blk0, xs);
        stage_pro_load16<PRO, NT>(a, blk0, ys);
        if constexpr (PRO == 2) stage_pro_apply<PRO, NT / 64>(a, xs, ys, true);
        quantize_q8_k_group<NT>(xs, blk0 + bl, total, nb, a.K, sub, lq, ld, lbs);
    }
}

// Q8_0 quantization of x into LDS (AVX2 variant, src/gguf_dot_q8.c:276-324):
// 8 threads per 32-element block, NT/8 blocks per round; same arithmetic as
// quantize_q8_0_kernel.
template <int NT>
__device__ __forceinline__ float4 stage_q8_0_load_from(const float *src, size_t tok_stride, const FusedArgs &a,
                                                      int blk0) {
    const int tid = threadIdx.x, part = tid & 7, bl = tid >> 3;
    const int nb = a.K / kQK8_0, total = a.m * nb;
    const int cb = min(blk0 + bl, total - 1);  // clamped: every thread issues the same loads
    const int tok = cb / nb, b = cb - tok * nb;
    return *reinterpret_cast<const float4 *>(src + (size_t)tok * tok_stride + (size_t)b * kQK8_0 + part * 4);
}
template <int NT>
__device__ __forceinline__ float4 stage_q8_0_load(const FusedArgs &a, int blk0) {
    return stage_q8_0_load_from<NT>(a.x, (size_t)a.K, a, blk0);
}
template <int PRO, int NT>
__device__ __forceinline__ float4 stage_pro_load4(const FusedArgs &a, int blk0) {
    if constexpr (PRO == 2) return stage_q8_0_load_from<NT>(a.x2, (size_t)a.K, a, blk0);
    else if constexpr (PRO == 1) return stage_q8_0_load_from<NT>(a.nw, 0, a, blk0);
    else return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// v0 / y0: this thread's elements of the first round (activation and the
// prologue's second input), loaded by the caller before the first weight
// tile.
template <int NT, int PRO = 0>
__device__ void stage_q8_0(const FusedArgs &a, float4 v0, float4 y0, int8_t *lq, float *ld) {
    constexpr int BPR = NT / 8;  // blocks per round
    const int tid = threadIdx.x, part = tid & 7, bl = tid >> 3;
    const int nb = a.K / kQK8_0, total = a.m * nb;
    for (int blk0 = 0; blk0 < total; blk0 += BPR) {  // RMSNorm prologue: one round
        const int blk = blk0 + bl;
        const int cb = min(blk, total - 1);
        const int tok = cb / nb, b = cb - tok * nb;
        float4 v = blk0 == 0 ? v0 : stage_q8_0_load<NT>(a, blk0);
        if constexpr (PRO != 0) {
            const float4 y = blk0 == 0 ? y0 : stage_pro_load4<PRO, NT>(a, blk0);
            float xv[4] = {v.x, v.y, v.z, v.w};
            const float yv[4] = {y.x, y.y, y.z, y.w};
            stage_pro_apply<PRO, NT / 64>(a, xv, yv, blk < total);
            v = make_float4(xv[0], xv[1], xv[2], xv[3]);
        }
        // the block's largest |x| over its 8 threads (half a DPP row)
        const float amax = row8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (blk >= total) continue;  // uniform within each 8-thread group
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const uint32_t dh = f32_to_f16_rne(d);
        const float xs[4] = {v.x, v.y, v.z, v.w};
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float q0 = rintf(xs[e] * id);
            int q = (q0 >= -2147483648.0f && q0 < 2147483648.0f) ? (int)q0 : INT32_MIN;
            q = q < -128 ? -128 : (q > 127 ? 127 : q);
            word |= (uint32_t)(q & 0xff) << (8 * e);
        }
        reinterpret_cast<uint32_t *>(lq + (size_t)tok * a.K + (size_t)b * kQK8_0)[part] = word;
        if (part == 0) ld[tok * nb + b] = f16_bits_to_f32(dh);
    }
}

// The matrix a row tile belongs to and the tile's first row.  The
// kernel-argument arrays are read at constant indices only and selected
// between, so their words are loaded once, before the tile loop, and stay in
// scalar registers; a dynamic index would reload them (a chain of dependent
// scalar loads) between one tile's data and the next tile's loads.
// Word 3 of a raw buffer descriptor for untyped dword access: DATA_FORMAT 32
// (bits 18:15 = 4; a zero format would drop every access), all else zero.
constexpr int kRawBufferWord3 = 0x00020000;
// A buffer offset beyond every output buffer: the store is dropped.
constexpr int kDeadOffset = 0x7ffffff0;

// A tile output's bias and residual words (zero where there is none).
struct Epi {
    float b, r;
};

struct TileMat {
    const uint8_t *w;
    const float *bias;
    const float *resid;
    float *out;
    int n_out;
    int row0;
};
__device__ __forceinline__ TileMat locate(const FusedArgs &a, int tile, int rows_per_tile) {
    TileMat t{a.w[0], a.bias[0], a.resid[0], a.out[0], a.n_out[0], 0};
    int start = 0;
#pragma unroll
    for (int k = 1; k < kFusedMaxMats; ++k) {
        const bool in = k < a.nmat && tile >= a.tile_start[k];
        t.w = in ? a.w[k] : t.w;
        t.bias = in ? a.bias[k] : t.bias;
        t.resid = in ? a.resid[k] : t.resid;
        t.out = in ? a.out[k] : t.out;
        t.n_out = in ? a.n_out[k] : t.n_out;
        start = in ? a.tile_start[k] : start;
    }
    t.row0 = (tile - start) * rows_per_tile;
    return t;
}

// LDS carve-up shared by the kernel and its launcher.
struct FusedLds {
    size_t qbytes, dbytes, bbytes, rbytes;
    __host__ __device__ FusedLds(int m, int K, int nblk, bool q8k, int NW, int S, int NV, bool staged = true) {
        if (!staged) m = 0;
        qbytes = ((size_t)m * K + 15) & ~(size_t)15;
        dbytes = (((size_t)m * nblk * 4) + 15) & ~(size_t)15;
        bbytes = q8k ? ((((size_t)m * (K / 16) * 2) + 15) & ~(size_t)15) : 0;
        rbytes = 2 * (size_t)NW * S * NV * sizeof(float);  // two buffers, alternating by tile
    }
    __host__ __device__ size_t total() const { return qbytes + dbytes + bbytes + rbytes; }
};

// Waves per SIMD the register allocator is held to: enough for the whole
// weight matrix to be requested by one generation of workgroups.  The
// figures for the wide Q6_K weight registers and the staging prologues are
// capped in fused_occupancy_pro so that no instantiation spills (under
// -Rpass-analysis=kernel-resource-usage every instantiation in this library
// reports 0 bytes of scratch).
template <class Fmt>
constexpr int fused_occupancy(int r, int m, int loop) {
    // f32-activation formats: the activation slice (32 to 68 floats) stays
    // in registers, one per token
    if (sizeof(typename Fmt::Act) >= 128) return m > 1 ? 2 : (r <= 1 ? 4 : 3);
    // two register buffers at 2-4 tokens: one 8-wave workgroup per CU, two
    // waves per SIMD
    if (loop == 1 && m > 1) return 2;
    return loop == 1 ? (r <= 1 ? (sizeof(typename Fmt::W) > 48 ? 4 : 5) : r <= 2 ? (sizeof(typename Fmt::W) > 48 ? 3 : 4) : 2)
           : loop == 2 ? (r <= 1 ? (sizeof(typename Fmt::W) > 48 ? 5 : 7)
                          : r <= 2 ? (sizeof(typename Fmt::W) > 48 ? 4 : 5)
                                   : (sizeof(typename Fmt::W) > 48 ? 3 : 4))
           : r * m <= 1 ? (sizeof(typename Fmt::W) > 48 ? 5 : 7)
           : r * m <= 2 ? (sizeof(typename Fmt::W) > 48 ? (m > 1 ? 4 : 5) : (m > 1 ? 5 : 6))
                        : (sizeof(typename Fmt::W) > 48 ? 3 : 4);
}

// STAGE: quantize a.x into LDS inside the kernel; otherwise read the codes
// of a.xq (quantized by an earlier launch) straight from global memory.
// A staging prologue holds its second input (16 more registers) and its
// arithmetic beside the first tile, the RMSNorm one its sums too.  Caps
// found with -Rpass-analysis=kernel-resource-usage, each the highest
// occupancy at which that shape spills nothing:
//   Q4_K rows, RMSNorm prologue: 4;  other prologues: 5;
//   Q6_K rows (56 bytes of weight registers per unit): 4 for one or two rows
//   per slot; four rows per slot: 2 under a prologue or a gate/up pair
//   (whose two rows per slot hold twice the weights).
// The Q4_K logits kernel with the argmax epilogue (f32 activation, two rows
// per slot) is held to 4, not the 3 of the other f32 shapes: at 3 its two
// workgroups per CU no longer fit (77.9 against 82.4 us for the [128256 x
// 4096] product, when it still needed 16 bytes of scratch per lane at 4;
// since the codes convert two at a time it fits 4 without any).
template <class Fmt>
constexpr int fused_occupancy_pro(int r, int m, int loop, int pro) {
    const bool wide = sizeof(typename Fmt::W) > 48;
    if ((pro & 16) != 0 && sizeof(typename Fmt::Act) >= 128 && !wide && m == 1 && r <= 2) return 4;
    int occ = fused_occupancy<Fmt>(r, m, loop);
    int cap = (pro & 3) == 1 ? 4 : (pro & 3) != 0 ? 5 : 8;
    if (wide) {
        cap = cap < 4 ? cap : 4;
        const int rows = r * ((pro & 8) != 0 ? 2 : 1);  // a pair's slot holds gate and up rows
        if (rows >= 4 && ((pro & 3) != 0 || (pro & 8) != 0)) cap = 2;
    }
    return occ > cap ? cap : occ;
}

// PRO bits 0-1: staging prologue (0 none, 1 RMSNorm, 2 SiLU-mul; STAGE
// kernels); bit 2: residual epilogue (outputs += resid).  Without bit 2 the
// kernel loads no residual word and holds no register for it.  Bit 4:
// greedy-argmax epilogue (one matrix, one token): every stored score also
// enters its lane's running best key, and each workgroup writes its best to
// a.amax at the end.
// Formats whose dotm<M> takes M tokens per conversion of the weights.
template <class F, class = void>
struct tokens_share_w : std::false_type {};
template <class F>
struct tokens_share_w<F, std::void_t<decltype(F::kTokensShareW)>> : std::bool_constant<F::kTokensShareW> {};

template <class Fmt, int M, int R, int NW, bool STAGE, int LOOP, int PRO = 0>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(fused_occupancy_pro<Fmt>(R, M, LOOP, PRO))))
void gemv_fused_kernel(FusedArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    // wave-uniform values go through readfirstlane so that the tile, matrix
    // and pointer selection below is scalar (kernel-argument arrays are read
    // with scalar loads)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int G = a.G, S = 64 / G, KS = a.KS, RG = NW / KS;
    const int rg = wave / KS, ks = wave - rg * KS;
    const int slot = lane / G, gl = lane & (G - 1);
    const int unit = gl + G * ks;
    const int u = min(unit, a.U - 1);
    // PRO bit 3: gate/up pairs (matrix 0 = gate, a.w[1] / a.bias[1] = up):
    // slot rows r = 2j and 2j+1 are row j of gate and of up, and the tile's
    // store writes silu(gate) * up (src/native.c:2576-2578) from the gate lane
    constexpr bool kPair = (PRO & 8) != 0;
    static_assert(!kPair || (M == 1 && R % 2 == 0), "pairs need one token and an even row count");
    const int rows_per_tile = S * (kPair ? R / 2 : R);
    constexpr int NV = R * M;
    constexpr int V = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : NV <= 8 ? 8 : 16;
    static_assert(NV <= 16, "too many partials per lane");

    constexpr bool kQ8K = Fmt::kUnitsPerBlock == 4;
    const FusedLds L(a.m, a.K, a.nblk, kQ8K, NW, S, NV, STAGE);
    int8_t *lq = reinterpret_cast<int8_t *>(smem);
    float *ld = reinterpret_cast<float *>(smem + L.qbytes);
    int16_t *lbs = reinterpret_cast<int16_t *>(smem + L.qbytes + L.dbytes);
    float *red = reinterpret_cast<float *>(smem + L.qbytes + L.dbytes + L.bbytes);  // [2][wave][slot][NV]

    // The one output value (if any) this lane stores: with G >= V the
    // reduction leaves each lane at most one value.  KS == 1: writer lanes of
    // every wave; KS > 1: the first S*NV lanes of the row group's first wave.
    static_assert(V <= 16, "group_reduce leaves one value per lane only for V <= G (G >= 16)");
    const int base = group_reduce_index(V, G, gl);
    const int spread = V < G ? G / V : 1;
    int o_slot, o_idx;
    bool o_live;
    if (KS == 1) {
        o_slot = slot;
        o_idx = base;
        o_live = (gl & (spread - 1)) == 0 && base < NV;
    } else {
        o_slot = lane / NV;
        o_idx = lane - o_slot * NV;
        o_live = ks == 0 && lane < S * NV;
    }
    const int o_r = o_idx / M, o_t = o_idx - (o_idx / M) * M;
    constexpr bool kArgmax = (PRO & 16) != 0;
    static_assert(!kArgmax || (M == 1 && (LOOP == 0 || LOOP == 2)), "the argmax epilogue: one token, one register buffer");
    // argmax epilogue: each lane's running best key lives in LDS for the
    // f32-activation formats (the logits kernels have no registers to
    // spare), in two registers otherwise
    constexpr bool kKeyLds = sizeof(typename Fmt::Act) >= 128;
    __shared__ unsigned long long lbest[kArgmax ? (kKeyLds ? NW * 64 : NW) : 1];
    unsigned long long best_reg = 0ull;
    if constexpr (kArgmax && kKeyLds) lbest[threadIdx.x] = 0ull;

    // Loads of one tile: weights (unconditional: clamped tile, row and unit,
    // so every path issues the same loads), the bias and the residual of
    // this lane's output.
    const int wg_tiles = (a.ntiles + RG - 1) / RG;
    constexpr bool kRes = (PRO & 4) != 0;
    // The bias (and residual) words are loaded unconditionally and selected
    // when used: a conditional write to the register of a load still in
    // flight would make the compiler wait for every outstanding load first,
    // which serialises the prefetch.  Where there is none the load reads the
    // first word of the lane's first weight row, a line its workgroup's
    // weight loads fetch anyway (one shared address for every lane of the
    // grid would queue them all on one L2 channel).
    auto issue_tile = [&](const TileMat &t_, Epi &e_, typename Fmt::W (&w_)[R]) {
        // bias and residual first: waiting for them then waits for no weight row
        const int orow = min(t_.row0 + o_slot + S * (kPair ? o_r >> 1 : o_r), t_.n_out - 1);
        const float *wf = reinterpret_cast<const float *>(t_.w + (size_t)min(t_.row0 + slot, t_.n_out - 1) * a.row_bytes);
        const float *bsel = kPair && (o_r & 1) ? a.bias[1] : t_.bias;
        e_.b = *(bsel != nullptr ? bsel + orow : wf);
        if constexpr (kRes) e_.r = *(t_.resid != nullptr ? t_.resid + (size_t)o_t * t_.n_out + orow : wf);
        else e_.r = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const WSrc src{kPair && (r & 1) ? a.w[1] : t_.w, a.row_bytes};
            Fmt::load_w(src, min(t_.row0 + slot + S * (kPair ? r >> 1 : r), t_.n_out - 1), u, w_[r]);
        }
    };
    auto load_tile = [&](int wt_, TileMat &t_, Epi &e_, typename Fmt::W (&w_)[R]) {
        t_ = locate(a, min(wt_ * RG + rg, a.ntiles - 1), rows_per_tile);
        issue_tile(t_, e_, w_);
    };
    auto bias_of = [&](const TileMat &t_, Epi raw) {
        const float *bsel = kPair && (o_r & 1) ? a.bias[1] : t_.bias;
        return Epi{bsel != nullptr ? raw.b : 0.0f, kRes && t_.resid != nullptr ? raw.r : 0.0f};
    };

    // 1. the activation's first staging round, then the first tile's
    //    weights: issued in this order, the activation does not wait behind
    //    the tile (loads of one wave return in order)
    float xs0[16], ys0[16];
    float4 v0, y0;
    if constexpr (STAGE) {
        if constexpr (kQ8K) {
            stage_q8_k_load<NW * 64>(a, 0, xs0);
            stage_pro_load16<PRO & 3, NW * 64>(a, 0, ys0);
        } else {
            v0 = stage_q8_0_load<NW * 64>(a, 0);
            y0 = stage_pro_load4<PRO & 3, NW * 64>(a, 0);
        }
    }
    int wt = blockIdx.x;
    TileMat tm;
    Epi bias;
    typename Fmt::W wa[R];
    load_tile(wt, tm, bias, wa);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the staging arithmetic

    // 2. quantize the activation into LDS once per workgroup while the tile
    //    streams in (the staging is shared by the NW waves; quantizing per
    //    lane in registers instead repeats it in every wave and measured
    //    slower)
    if constexpr (STAGE) {
        if constexpr (kQ8K) stage_q8_k<NW * 64, PRO & 3>(a, xs0, ys0, lq, ld, lbs);
        else stage_q8_0<NW * 64, PRO & 3>(a, v0, y0, lq, ld);
        __syncthreads();
    }
    const ActLds act{lq, ld, lbs, a.K, a.nblk};
    // the tokens' activation slices stay in registers for every tile
    typename Fmt::Act x1;
    if (M == 1) {
        if constexpr (STAGE) Fmt::load_act_lds(act, u, 0, x1);
        else Fmt::load_act(a, u, 0, x1);
    }
    typename Fmt::Act xr[M > 1 ? M : 1];
    if constexpr (M > 1) {
#pragma unroll
        for (int t = 0; t < M; ++t) {
            if constexpr (STAGE) Fmt::load_act_lds(act, u, t, xr[t]);
            else Fmt::load_act(a, u, t, xr[t]);
        }
    }

    // dot products of one tile's weights into vals
    // Every lane computes (u is clamped to a real unit) and the lanes past the
    // row's units drop their sums by a select: with no branch around it, every
    // path through the loop waits for the weights it consumes, so the next
    // tile's loads need not wait for the previous tile's store.
    const bool unit_live = unit < a.U;
    auto dot = [&](const typename Fmt::W (&w_)[R], float (&vals)[V]) {
#pragma unroll
        for (int k = 0; k < V; ++k) vals[k] = 0.0f;
        if constexpr (M > 1 && tokens_share_w<Fmt>::value) {
            // every token's dot from one conversion of the weights
#pragma unroll
            for (int r = 0; r < R; ++r) Fmt::template dotm<M>(w_[r], u, xr, &vals[r * M]);
        } else {
#pragma unroll
            for (int t = 0; t < M; ++t) {
                typename Fmt::Act x;
                if constexpr (M == 1) x = x1;
                else x = xr[t];
#pragma unroll
                for (int r = 0; r < R; ++r) Fmt::dot1(w_[r], u, x, vals[r * M + t]);
            }
        }
#pragma unroll
        for (int k = 0; k < V; ++k) vals[k] = unit_live ? vals[k] : 0.0f;
    };
    // lane reduction, K-split sum and store of one tile
    auto finish = [&](float (&vals)[V], int iter, bool have, const TileMat &ct, Epi ce) {
        group_reduce<V>(vals, G, lane);
        float result = vals[0];
        if (KS > 1) {
            // the KS waves of a row group add their partials in LDS, in wave
            // order; the buffer alternates by iteration, so one barrier per
            // iteration keeps the next write away from this read
            float *rb = red + (iter & 1) * (NW * S * NV);
            if ((gl & (spread - 1)) == 0 && base < NV) rb[(wave * S + slot) * NV + base] = vals[0];
            __syncthreads();
            result = 0.0f;
            if (o_live)
                for (int k2 = 0; k2 < KS; ++k2) result += rb[((rg * KS + k2) * S + o_slot) * NV + o_idx];
        }
        // One store instruction per tile on every path: a lane without an
        // output gets an offset past the end of the buffer, whose range check
        // drops the write.  With no branch around the store, the compiler
        // counts exactly one store after each tile's loads and waits for the
        // weights alone, not for the previous tile's store as well.
        const int row = ct.row0 + o_slot + S * (kPair ? o_r >> 1 : o_r);
        const bool live = have && o_live && row < ct.n_out && (!kPair || (o_r & 1) == 0);
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(ct.out, (short)0, a.m * ct.n_out * 4, kRawBufferWord3);
        // out = residual + (bias + dot): the reference's projection, then its
        // residual add (src/native.c:2571-2580)
        const float v = ce.b + result;
        float o = kRes && ct.resid != nullptr ? ce.r + v : v;
        if constexpr (kPair) {
            // the up value of the same row sits on the lane whose value index
            // differs in bit 0: lane bit G/V after the lane reduction, the next
            // lane after the K-split sum
            const float up = shfl_xor_f(v, KS > 1 ? 1 : G / V);
            o = silu_f32(v) * up;
        }
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), rs,
                                              live ? (o_t * ct.n_out + row) * 4 : kDeadOffset, 0, 0);
        if constexpr (kArgmax) {
            const unsigned long long k = live ? score_key(o, (unsigned)row) : 0ull;
            if constexpr (kKeyLds) {
                // the LDS unit keeps the maximum (ds_max_u64; each lane owns
                // its slot): no register holds the old key
                __hip_atomic_fetch_max(&lbest[threadIdx.x], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            } else {
                best_reg = k > best_reg ? k : best_reg;
            }
        }
    };

    // 3. grid-stride loop over workgroup tiles (a uniform trip count, so the
    //    barriers of the KS > 1 reduction line up).  A trip that has a next
    //    tile always loads it and the last trip leaves before loading: a
    //    conditional load would make the weight registers a merge of old and
    //    new values, which the register allocator resolves with copies that
    //    wait for the loads just issued.  The tile's bias is resolved before
    //    its dot, which frees its register for the next tile's bias without
    //    a copy.  A dropped store (an empty buffer) enters the loop the way
    //    its end re-enters it, with one store behind the tile's loads, so
    //    that no path's wait for a tile's last weights includes the store.
    __builtin_amdgcn_raw_buffer_store_b32(0u, __builtin_amdgcn_make_buffer_rsrc(tm.out, (short)0, 0, kRawBufferWord3),
                                          0, 0, 0);
    auto resolve_bias = [&](const TileMat &t_, Epi raw) {
        Epi e = bias_of(t_, raw);
        asm volatile("" : "+v"(e.b));  // the selects stay here, not at their use
        if constexpr (kRes) asm volatile("" : "+v"(e.r));
        __builtin_amdgcn_sched_barrier(0);
        return e;
    };
    if constexpr (LOOP == 1) {
        // Two register buffers in turn: the next tile's loads are issued
        // before the current tile is computed, so each wave keeps a tile in
        // flight while it works and the dot products overlap the stream.
        typename Fmt::W wb[R];
        for (int iter = 0;; iter += 2) {
            TileMat tmb;
            Epi biasb;
            float vals[V];
            const int wt1 = wt + (int)gridDim.x;
            const Epi ba = resolve_bias(tm, bias);
            if (wt1 >= wg_tiles) {  // uniform over the workgroup
                dot(wa, vals);
                finish(vals, iter, wt * RG + rg < a.ntiles, tm, ba);
                break;
            }
            load_tile(wt1, tmb, biasb, wb);
            dot(wa, vals);
            finish(vals, iter, wt * RG + rg < a.ntiles, tm, ba);
            const int wt2 = wt1 + (int)gridDim.x;
            const Epi bb = resolve_bias(tmb, biasb);
            if (wt2 >= wg_tiles) {
                dot(wb, vals);
                finish(vals, iter + 1, wt1 * RG + rg < a.ntiles, tmb, bb);
                break;
            }
            load_tile(wt2, tm, bias, wa);
            dot(wb, vals);
            finish(vals, iter + 1, wt1 * RG + rg < a.ntiles, tmb, bb);
            wt = wt2;
        }
    } else if constexpr (LOOP == 2) {
        // Balanced per-wave schedule (rows not split over waves): with W
        // waves in the grid, round 0 gives wave k of workgroup b tile
        // b*RG + k; round j >= 1 gives it tile j*W + k*nWG + b, so a partial
        // last round spreads over the workgroups and every workgroup (hence,
        // with the grid at the resident capacity, every CU) gets the same
        // number of tiles to within one.
        const int T = a.ntiles, nwg = (int)gridDim.x, W = nwg * RG;
        int cur = (int)blockIdx.x * RG + rg;
        for (int iter = 0;; ++iter) {
            const bool have = cur < T;
            const Epi cbias = resolve_bias(tm, bias);
            float vals[V];
            dot(wa, vals);
            const TileMat ct = tm;
            const int next = iter == 0 ? W + rg * nwg + (int)blockIdx.x : cur + W;
            if (next >= T) {  // uniform over the wave
                finish(vals, iter, have, ct, cbias);
                break;
            }
            tm = locate(a, next, rows_per_tile);
            issue_tile(tm, bias, wa);
            finish(vals, iter, have, ct, cbias);
            cur = next;
        }
    } else {
        // One buffer: the next tile's loads are issued as soon as the
        // current tile's weights have been consumed, so the lane reduction
        // and the store overlap them.
        for (int iter = 0;; ++iter) {
            const bool have = wt * RG + rg < a.ntiles;
            // resolved before the next tile's loads go out, so the store
            // below depends on no outstanding load
            const Epi cbias = resolve_bias(tm, bias);
            float vals[V];
            dot(wa, vals);
            const TileMat ct = tm;
            wt += gridDim.x;
            if (wt >= wg_tiles) {  // uniform over the workgroup
                finish(vals, iter, have, ct, cbias);
                break;
            }
            load_tile(wt, tm, bias, wa);
            finish(vals, iter, have, ct, cbias);
        }
    }
    if constexpr (kArgmax) {
        // the workgroup's best key: each wave over its 64 lanes, then the
        // first wave over the NW wave results; one key per workgroup
        unsigned long long best_key = kKeyLds ? lbest[threadIdx.x] : best_reg;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(best_key, off, 64);
            best_key = o > best_key ? o : best_key;
        }
        __syncthreads();  // every lane has read its own lbest entry
        if (lane == 0) lbest[wave] = best_key;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int k = 1; k < NW; ++k) best_key = lbest[k] > best_key ? lbest[k] : best_key;
            a.amax[blockIdx.x] = best_key;
        }
    }
}

// Compute units of the current device (256 if the query fails).
static int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

// Tuning knobs (tuning_knob): EXQ_FUSED_R (rows per slot at m = 1: 1, 2 or
// 4), EXQ_FUSED_NW (waves per workgroup: 4 or 8), EXQ_FUSED_GRID (multiple of
// the resident workgroup count), EXQ_FUSED_PER_CU (workgroups per CU at most),
// EXQ_FUSED_PIPE / EXQ_FUSED_DYN / EXQ_FUSED_BIG (tile schedule).

// Grid of the most recent launch_fused_fmt (the argmax epilogue's key count).
static inline int &fused_last_grid() {
    static int g = 0;
    return g;
}

// per_cu_cap > 0: at most that many workgroups per CU in the grid.
template <class Fmt, int M, int R, int NW, bool STAGE, int LOOP, int PRO = 0>
static hipError_t launch_fused_fmt(FusedArgs a, hipStream_t st, int per_cu_cap = 0) {
    const int S = 64 / a.G, RG = NW / a.KS;
    const int rows_per_tile = S * ((PRO & 8) != 0 ? R / 2 : R);
    int t = 0;
    for (int z = 0; z < a.nmat; ++z) {
        a.tile_start[z] = t;
        t += (a.n_out[z] + rows_per_tile - 1) / rows_per_tile;
    }
    for (int z = a.nmat; z <= kFusedMaxMats; ++z) a.tile_start[z] = t;
    a.ntiles = t;
    const FusedLds L(a.m, a.K, a.nblk, Fmt::kUnitsPerBlock == 4, NW, S, R * M, STAGE);
    const int wg_tiles = (t + RG - 1) / RG;
    // resident workgroups from the kernel's real occupancy (registers + LDS);
    // the grid takes at most that many, each looping over the same number of
    // tiles, so no second generation of workgroups forms a tail
    const int cus = device_cus();
    static size_t cached_lds = (size_t)-1;
    static int per_cu = 1;
    if (L.total() != cached_lds) {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_fused_kernel<Fmt, M, R, NW, STAGE, LOOP, PRO>, NW * 64,
                                                         L.total()) != hipSuccess ||
            v < 1)
            v = 1;
        per_cu = v;
        cached_lds = L.total();
    }
    static const int grid_scale = tuning_knob("EXQ_FUSED_GRID", 1);  // resident multiple
    static const int cu_cap_env = tuning_knob("EXQ_FUSED_PER_CU", 0);  // workgroups per CU
    const int cu_cap = cu_cap_env > 0 ? cu_cap_env : per_cu_cap;
    const int resident = (cu_cap > 0 && cu_cap < per_cu ? cu_cap : per_cu) * cus * (grid_scale > 0 ? grid_scale : 1);
    const int rounds = (wg_tiles + resident - 1) / resident;
    // workgroup-tile schedule: equal tile counts per workgroup; balanced
    // per-wave schedule: every resident slot (equal work per CU)
    int grid = LOOP == 2 ? (wg_tiles < resident ? wg_tiles : resident) : (wg_tiles + rounds - 1) / rounds;
    // argmax epilogue: one key per workgroup must fit a.amax (both schedules
    // that carry it stride over the tiles by the grid, so any grid is complete)
    if constexpr ((PRO & 16) != 0) {
        if (grid > a.amax_cap) grid = a.amax_cap;
    }
    fused_last_grid() = grid;
    hipLaunchKernelGGL((gemv_fused_kernel<Fmt, M, R, NW, STAGE, LOOP, PRO>), dim3(grid), dim3(NW * 64), L.total(), st, a);
    return hipGetLastError();
}


template <class Fmt, int NW, bool STAGE>
static hipError_t launch_fused_m(FusedArgs a, int r1, int loop, hipStream_t st) {
    switch (a.m) {
        case 1:
            // Launches with more than two workgroups' worth of wave tiles per
            // CU: two register buffers of 2-row tiles, one workgroup per CU
            // (EXQ_FUSED_BIG=0: the balanced single-buffer schedule).
            // Measured, gate+up [28672 x 4096] in the decode step: 14.4 us,
            // against 15.0-15.2 balanced and 15.7 with workgroup tiles; the
            // smaller launches (o [4096 x 4096]: 4.9 against 5.5 us) and the
            // row-split ones keep workgroup tiles at the resident grid.
            if (loop == 2 && a.KS == 1) {
                const int rows_per_tile = (64 / a.G) * r1;
                int tiles = 0;
                for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] + rows_per_tile - 1) / rows_per_tile;
                if (tiles <= 2 * device_cus() * NW) loop = 0;
                static const int big = tuning_knob("EXQ_FUSED_BIG", 1);
                if (loop == 2 && big != 0) return launch_fused_fmt<Fmt, 1, 2, NW, STAGE, 1>(a, st, 1);
            }
            if (loop == 2 && a.KS == 1) {
                if (r1 == 1) return launch_fused_fmt<Fmt, 1, 1, NW, STAGE, 2>(a, st);
                if (r1 == 4) return launch_fused_fmt<Fmt, 1, 4, NW, STAGE, 2>(a, st);
                return launch_fused_fmt<Fmt, 1, 2, NW, STAGE, 2>(a, st);
            }
            if (loop == 1) {
                if (r1 == 1) return launch_fused_fmt<Fmt, 1, 1, NW, STAGE, 1>(a, st);
                // two buffers of four Q6_K rows exceed the 256 registers a
                // wave of an 8-wave workgroup can hold: two rows instead
                if constexpr (sizeof(typename Fmt::W) <= 48)
                    if (r1 == 4) return launch_fused_fmt<Fmt, 1, 4, NW, STAGE, 1>(a, st);
                return launch_fused_fmt<Fmt, 1, 2, NW, STAGE, 1>(a, st);
            }
            if (r1 == 1) return launch_fused_fmt<Fmt, 1, 1, NW, STAGE, 0>(a, st);
            if (r1 == 4) return launch_fused_fmt<Fmt, 1, 4, NW, STAGE, 0>(a, st);
            return launch_fused_fmt<Fmt, 1, 2, NW, STAGE, 0>(a, st);
        case 2:
        case 3:
        case 4: {
            // 2-4 tokens (measured on the Llama-3-8B and hybrid ~4B decode
            // steps): mid-size unsplit launches (4096 < 1-row tiles <= 12288,
            // e.g. q+k+v [6144 x 4096]: 11.8 -> 10.1 us at m = 4) take two
            // register buffers at one workgroup per CU; otherwise workgroup
            // tiles, two rows per slot at m = 2 (gate+up [28672 x 4096]:
            // 17.5 -> 16.4 us) and one at m = 3, 4 (the registers hold every
            // token's activation slice).
            if constexpr (NW == 8 && STAGE) {
                int tiles = 0;
                for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] + (64 / a.G) - 1) / (64 / a.G);
                const int per_gen = device_cus() * NW;
                if (a.KS == 1 && tiles > 2 * per_gen && tiles <= 6 * per_gen) {
                    if (a.m == 2) return launch_fused_fmt<Fmt, 2, 1, NW, STAGE, 1>(a, st, 1);
                    if (a.m == 3) return launch_fused_fmt<Fmt, 3, 1, NW, STAGE, 1>(a, st, 1);
                    return launch_fused_fmt<Fmt, 4, 1, NW, STAGE, 1>(a, st, 1);
                }
                if (a.m == 2) return launch_fused_fmt<Fmt, 2, 2, NW, STAGE, 0>(a, st);
            }
            if (a.m == 2) return launch_fused_fmt<Fmt, 2, 1, NW, STAGE, 0>(a, st);
            if (a.m == 3) return launch_fused_fmt<Fmt, 3, 1, NW, STAGE, 0>(a, st);
            return launch_fused_fmt<Fmt, 4, 1, NW, STAGE, 0>(a, st);
        }
        default: return hipErrorInvalidValue;
    }
}

// Rows per slot of the 16-wave row-split launch: the largest R whose
// workgroup tiles fill the grid best (Q6_K at most 2); r_env overrides.
template <class Fmt>
static int pick_r16(const FusedArgs &a, int r_env) {
    constexpr int kRMax = sizeof(typename Fmt::W) > 48 ? 2 : 4;
    const int rg = 16 / a.KS, cus = device_cus();
    auto fill = [&](int r) {
        int tiles = 0;
        for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] + r - 1) / r;
        const int wg_tiles = (tiles + rg - 1) / rg, rounds = (wg_tiles + cus - 1) / cus;
        return (double)wg_tiles / (double)(rounds * cus);
    };
    int r16 = kRMax;
    if (kRMax == 4 && fill(2) > fill(r16) + 1e-9) r16 = 2;
    if (fill(1) > fill(r16) + 1e-9) r16 = 1;
    if (r_env == 1 || r_env == 2 || (r_env == 4 && kRMax == 4)) r16 = r_env;
    return r16;
}

// One token of a K-quant row split over three waves (12-wave workgroups,
// four row groups): rows per slot by grid fill as pick_r16.
template <class Fmt, int PRO = 0>
static hipError_t launch_fused_ks3(FusedArgs a, hipStream_t st) {
    constexpr bool kPair = (PRO & 8) != 0;
    constexpr int kRMax = sizeof(typename Fmt::W) > 48 ? 2 : 4;
    const int cus = device_cus();
    auto fill = [&](int r) {
        int tiles = 0;
        for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] * (kPair ? 2 : 1) + r - 1) / r;
        const int wg_tiles = (tiles + 3) / 4, rounds = (wg_tiles + cus - 1) / cus;
        return (double)wg_tiles / (double)(rounds * cus);
    };
    int r = kRMax;
    if (kRMax == 4 && fill(2) > fill(r) + 1e-9) r = 2;
    if (!kPair && fill(1) > fill(r) + 1e-9) r = 1;
    if constexpr (!kPair) {
        if (r == 1) return launch_fused_fmt<Fmt, 1, 1, 12, true, 0, PRO>(a, st);
    }
    if (r == 2) return launch_fused_fmt<Fmt, 1, 2, 12, true, 0, PRO>(a, st);
    if constexpr (kRMax == 4) return launch_fused_fmt<Fmt, 1, 4, 12, true, 0, PRO>(a, st);
    return hipErrorInvalidValue;
}

// One token with a staging prologue (PRO 1: RMSNorm, 2: SiLU-mul), a
// residual (bit 2) or gate/up pairs (bit 3): the default one-token schedules
// of launch_fused_nw, instantiated with them (pairs take an even row count
// per slot).
template <class Fmt, int PRO>
static hipError_t launch_fused_pro(FusedArgs a, hipStream_t st) {
    constexpr bool kPair = (PRO & 8) != 0;
    if (a.m != 1 || a.KS > 4) return hipErrorInvalidValue;
    if (a.KS > 1) {
        if constexpr (Fmt::kUnitsPerBlock == 4) {
            if (a.KS == 3) return launch_fused_ks3<Fmt, PRO>(a, st);
            int r16 = pick_r16<Fmt>(a, 0);
            if constexpr (kPair) {
                // pairs per slot 1 or 2: the count whose workgroup tiles fill the grid best
                const int rg = 16 / a.KS, cus = device_cus();
                auto fill = [&](int pairs) {
                    const int tiles = (a.n_out[0] + pairs - 1) / pairs;
                    const int wg_tiles = (tiles + rg - 1) / rg, rounds = (wg_tiles + cus - 1) / cus;
                    return (double)wg_tiles / (double)(rounds * cus);
                };
                r16 = sizeof(typename Fmt::W) <= 48 && fill(2) >= fill(1) ? 4 : 2;
            } else {
                if (r16 == 1) return launch_fused_fmt<Fmt, 1, 1, 16, true, 0, PRO>(a, st);
            }
            if (r16 == 2) return launch_fused_fmt<Fmt, 1, 2, 16, true, 0, PRO>(a, st);
            if constexpr (sizeof(typename Fmt::W) <= 48) return launch_fused_fmt<Fmt, 1, 4, 16, true, 0, PRO>(a, st);
            return hipErrorInvalidValue;
        } else {
            return launch_fused_fmt<Fmt, 1, 4, 8, true, 0, PRO>(a, st);
        }
    }
    int rows = 0;
    for (int z = 0; z < a.nmat; ++z) rows += a.n_out[z] * (kPair ? 2 : 1);
    const int r1 = rows <= 4096 ? 2 : 4;
    const int rows_per_tile = (64 / a.G) * r1;
    int tiles = 0;
    for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] * (kPair ? 2 : 1) + rows_per_tile - 1) / rows_per_tile;
    if (tiles > 2 * device_cus() * 8) return launch_fused_fmt<Fmt, 1, 2, 8, true, 1, PRO>(a, st, 1);
    return r1 == 2 ? launch_fused_fmt<Fmt, 1, 2, 8, true, 0, PRO>(a, st)
                   : launch_fused_fmt<Fmt, 1, 4, 8, true, 0, PRO>(a, st);
}

// Tile shape: 8 waves per workgroup; R = 4 rows per slot at m = 1 unless
// the launch is short and unsplit (<= 4096 rows), where R = 2 keeps more
// workgroups in flight.  (Measured on [1024..28672 x 4096] and
// [4096 x 14336] Q4_K.)  Knobs EXQ_FUSED_R / EXQ_FUSED_NW.
template <class Fmt>
static hipError_t launch_fused_nw(FusedArgs a, bool stage, hipStream_t st) {
    static const int r_env = tuning_knob("EXQ_FUSED_R", 0);
    static const int nw = tuning_knob("EXQ_FUSED_NW", 8);
    // 2: balanced per-wave schedule (m = 1, rows not split over waves); 1:
    // two register buffers; 0: workgroup tiles, grid-stride
    static const int loop = tuning_knob("EXQ_FUSED_PIPE", 0) != 0 ? 1 : (tuning_knob("EXQ_FUSED_DYN", 1) != 0 ? 2 : 0);
    if (a.KS > 4) return hipErrorInvalidValue;
    int rows = 0;
    for (int z = 0; z < a.nmat; ++z) rows += a.n_out[z];
    const int r1 = r_env > 0 ? r_env : (a.KS == 1 && rows <= 4096 ? 2 : 4);
    // Rows split over waves (more than 64 units) with the activation staged
    // in the kernel, one token: 16-wave workgroups (one per CU), whose 1024
    // threads quantize up to 16384 elements in one round (issued before the
    // first weight tile) and share it over twice the rows of an 8-wave
    // workgroup.  Rows per slot: the largest R whose workgroup tiles fill the
    // grid best (a partial last round leaves CUs idle).  Measured in the
    // decode steps: down [4096 x 14336] Q4_K 11.4 us (R = 4) against 12.6 us
    // for a quantize launch and 8-wave workgroups; down [2560 x 9728] Q6_K
    // 12.0 us (R = 1) against 13.7 us with R = 2; [1024 | 2048 x 14336] Q4_K
    // 6.9 | 8.4 us (R = 1) against 8.5 | 9.7 us (R = 4).  Q6_K has at most
    // two rows per slot: four exceed the 128 registers of such a workgroup.
    if constexpr (Fmt::kUnitsPerBlock == 4) {  // Q8_K activations (Q4_K, Q6_K rows)
        if (stage && a.m == 1 && a.KS == 3) return launch_fused_ks3<Fmt>(a, st);
        if (stage && a.m == 1 && a.KS > 1) {
            static const int r_env = tuning_knob("EXQ_FUSED_NW16_R", 0);  // rows per slot
            const int r16 = pick_r16<Fmt>(a, r_env);
            if (r16 == 1) return launch_fused_fmt<Fmt, 1, 1, 16, true, 0>(a, st);
            if (r16 == 2) return launch_fused_fmt<Fmt, 1, 2, 16, true, 0>(a, st);
            if constexpr (sizeof(typename Fmt::W) <= 48) return launch_fused_fmt<Fmt, 1, 4, 16, true, 0>(a, st);
        }
    }
    if (stage)
        return nw == 4 ? launch_fused_m<Fmt, 4, true>(a, r1, loop, st) : launch_fused_m<Fmt, 8, true>(a, r1, loop, st);
    return nw == 4 ? launch_fused_m<Fmt, 4, false>(a, r1, loop, st) : launch_fused_m<Fmt, 8, false>(a, r1, loop, st);
}

// Lanes per slot G and waves per row KS for U units so that every unit is
// covered in one pass (G * KS >= U) with the best lane use; KS <= 4 so that
// both workgroup sizes can hold a row group.  with3: KS = 3 too, for rows of
// more than 128 units (12-wave workgroups; one token of a K-quant row):
// measured on the Q6_K down [2560 x 9728] (152 units), 12.1 -> 10.0 us; the
// 40-unit rows of K = 2560 ran slower as 3 x 16 lanes than as 64.
static inline bool pick_fused_shape(int U, int &G, int &KS, bool with3 = false) {
    double best = -1.0;
    bool found = false;
    for (int ks = 1; ks <= 4; ++ks) {
        if (ks == 3 && (!with3 || U <= 128)) continue;  // only where four waves were the choice
        for (int g = 64; g >= 16; g >>= 1) {
            if (g * ks < U) continue;
            const double util = (double)U / (double)(g * ks);
            if (util > best + 1e-9) {
                best = util;
                G = g;
                KS = ks;
                found = true;
            }
        }
    }
    return found;
}

}  // namespace exq
