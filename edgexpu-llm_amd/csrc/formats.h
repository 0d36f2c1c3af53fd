// Per-format pieces of the decode GEMV kernels: how a lane loads its slice of
// a GGUF row ("unit") and of the activation, and the unit's contribution to
// the row dot.  Shared by the generic kernel (gemv.hip) and the fused,
// persistent kernel (gemv_fused.hip).
//
//   Q8_0 x Q8_0  -- dot_q8_0_q8_0  src/gguf_dot_q8.c:436-480
//   Q4_K x Q8_K  -- dot_q4_k_q8_k  src/gguf_dot_q8.c:603-762
//   Q6_K x Q8_K  -- dot_q6_k_q8_k  src/gguf_dot_q8.c:897-1002
//   Q4_K/Q6_K/Q8_0 x f32 -- dot_q4_k / dot_q6_k / dot_q8_0, src/gguf_quant.c:539-794
//   Q4_0 / Q5_0 x Q8_0 -- dot_q4_0_q8_0 / dot_q5_0_q8_0, src/gguf_dot_q8.c:482-601
//   Q5_K x Q8_K  -- dot_q5_k_q8_k  src/gguf_dot_q8.c:764-895
//   Q4_0/Q5_0/Q5_K/F16 x f32 -- dot_q4_0 / dot_q5_0 / dot_q5_k / dot_f16,
//                   src/gguf_quant.c:672-702, 796-892
//
// Integer block sums are exact (sdot4 on the int8 codes); their fp32
// combination differs from the reference only in summation order.
#pragma once

#include "common.h"

namespace exq {

struct GemvArgs {
    const uint8_t *w;        // n_out rows of row_bytes
    size_t row_bytes;
    int n_out;
    int K;                   // n_in
    int nblk;                // K / block elements (32 or 256)
    int U;                   // units per row
    int G;                   // lanes per slot (8, 16, 32 or 64)
    int T;                   // ceil(U / G)
    int m;                   // tokens in this launch (== M template)
    // quantized activations in the reference's block bytes (Q8_0: 34 B per
    // 32, Q8_K: 292 B per 256), token t at xq + t*xq_stride; or f32 activations
    const uint8_t *xq;
    size_t xq_stride;
    const float *xf;         // [m][K] f32 activations (f32 path)
    const float *bias;       // [n_out] or null
    float *out;              // [m][ldo]
    int ldo;
};

// Activation staged in LDS by the fused kernel (split layout, per token t):
//   q8  int8  [K]        at q + t*K
//   d   f32   [K/QK]     at d + t*nblk   (Q8_K d, or the fp16-rounded Q8_0 d)
//   bs  int16 [K/16]     at bs + t*K/16  (16-element code sums; Q8_K only)
struct ActLds {
    const int8_t *q;
    const float *d;
    const int16_t *bs;
    int K;
    int nblk;
};

// ------------------------------------------------------------------ Q4_K

struct FmtQ4K {
    static constexpr int kUnitsPerBlock = 4;  // (super-block i, 64-chunk j)
    struct Act {
        uint32_t q[16];   // codes of elements 64j..64j+63 of super-block i
        float dx;         // Q8_K block scale
        uint32_t spair;   // int16 pair: sums of sub-blocks 2j and 2j+1
    };
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const int i = unit >> 2, j = unit & 3;
        const uint8_t *blk = a.xq + (size_t)tk * a.xq_stride + (size_t)i * kBytesQ8_K;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 t = ldg16(blk + 4 + 64 * j + 16 * v);
            x.q[4 * v + 0] = t.x; x.q[4 * v + 1] = t.y; x.q[4 * v + 2] = t.z; x.q[4 * v + 3] = t.w;
        }
        x.dx = *reinterpret_cast<const float *>(blk);
        const uint2 bs = ldg8(blk + 260 + 8 * j);  // bsums 4j..4j+3
        const int s0 = (int)(int16_t)(bs.x & 0xffff) + (int)(int16_t)(bs.x >> 16);
        const int s1 = (int)(int16_t)(bs.y & 0xffff) + (int)(int16_t)(bs.y >> 16);
        x.spair = ((uint32_t)s0 & 0xffffu) | ((uint32_t)s1 << 16);
    }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) {
        const int i = unit >> 2, j = unit & 3;
        const uint4 *p = reinterpret_cast<const uint4 *>(s.q + (size_t)tk * s.K + 256 * i + 64 * j);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 t = p[v];
            x.q[4 * v + 0] = t.x; x.q[4 * v + 1] = t.y; x.q[4 * v + 2] = t.z; x.q[4 * v + 3] = t.w;
        }
        x.dx = s.d[tk * s.nblk + i];
        const uint2 bs = *reinterpret_cast<const uint2 *>(s.bs + (size_t)tk * (s.K / 16) + 16 * i + 4 * j);
        const int s0 = (int)(int16_t)(bs.x & 0xffff) + (int)(int16_t)(bs.x >> 16);
        const int s1 = (int)(int16_t)(bs.y & 0xffff) + (int)(int16_t)(bs.y >> 16);
        x.spair = ((uint32_t)s0 & 0xffffu) | ((uint32_t)s1 << 16);
    }
    struct W {
        uint4 h, q0, q1;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const int i = unit >> 2, j = unit & 3;
        const uint8_t *sb = a.w + (size_t)row * a.row_bytes + (size_t)i * kBytesQ4_K;
        w.h = *reinterpret_cast<const uint4 *>(sb);
        w.q0 = *reinterpret_cast<const uint4 *>(sb + 16 + 32 * j);
        w.q1 = *reinterpret_cast<const uint4 *>(sb + 32 + 32 * j);
    }
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        const int j = unit & 3;
        const float d = f16_bits_to_f32(w.h.x & 0xffffu);
        const float dmin = f16_bits_to_f32(w.h.x >> 16);
        // Six-bit scale/min pairs of sub-blocks 2j, 2j+1 (unpack_k4_scales,
        // src/gguf_dot_q8.c:112-124): bytes 0..3 hold sc0..3, 4..7 m0..3, and
        // 8..11 the low nibbles of sc4..7 / m4..7 with the top bits of 0..7.
        const int sh = 16 * (j & 1);
        uint32_t scp, mp;
        if (j < 2) {
            scp = (w.h.y >> sh) & 0x3f3fu;
            mp = (w.h.z >> sh) & 0x3f3fu;
        } else {
            scp = ((w.h.w >> sh) & 0x0f0fu) | (((w.h.y >> sh) >> 2) & 0x3030u);
            mp = (((w.h.w >> sh) >> 4) & 0x0f0fu) | (((w.h.z >> sh) >> 2) & 0x3030u);
        }
        const int sc0 = (int)(scp & 0xffu), sc1 = (int)(scp >> 8);
        const uint32_t mpair = (mp & 0xffu) | ((mp & 0xff00u) << 8);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            lo[k] = qw[k] & 0x0f0f0f0fu;
            hi[k] = (qw[k] >> 4) & 0x0f0f0f0fu;
        }
        {
            int dlo = 0, dhi = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                dlo = sdot4(lo[k], xa.q[k], dlo);
                dhi = sdot4(hi[k], xa.q[8 + k], dhi);
            }
            const int isum = sc0 * dlo + sc1 * dhi;
            const int imin = sdot2(mpair, xa.spair, 0);
            const float dd = xa.dx * d;
            const float dm = xa.dx * dmin;
            acc = fmaf(dd, (float)isum, acc);
            acc = fmaf(-dm, (float)imin, acc);
        }
    }
};

// ------------------------------------------------------------------ Q6_K

struct FmtQ6K {
    static constexpr int kUnitsPerBlock = 4;  // (super-block i, half h, l-half p)
    struct Act {
        uint32_t q[16];   // q8 of elements 128h+32k+16p..+15, k=0..3 (4 dwords each)
        float dx;
        int bs32[4];      // 32 * (16-element code sum) of sub-block 8h+2k+p
    };
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const int i = unit >> 2, h = (unit >> 1) & 1, p = unit & 1;
        const uint8_t *blk = a.xq + (size_t)tk * a.xq_stride + (size_t)i * kBytesQ8_K;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 t = ldg16(blk + 4 + 128 * h + 32 * k + 16 * p);
            x.q[4 * k + 0] = t.x; x.q[4 * k + 1] = t.y; x.q[4 * k + 2] = t.z; x.q[4 * k + 3] = t.w;
        }
        x.dx = *reinterpret_cast<const float *>(blk);
        const int16_t *bs = reinterpret_cast<const int16_t *>(blk + 260) + 8 * h + p;
#pragma unroll
        for (int k = 0; k < 4; ++k) x.bs32[k] = 32 * (int)bs[2 * k];
    }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) {
        const int i = unit >> 2, h = (unit >> 1) & 1, p = unit & 1;
        const int8_t *base = s.q + (size_t)tk * s.K + 256 * i + 128 * h + 16 * p;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 t = *reinterpret_cast<const uint4 *>(base + 32 * k);
            x.q[4 * k + 0] = t.x; x.q[4 * k + 1] = t.y; x.q[4 * k + 2] = t.z; x.q[4 * k + 3] = t.w;
        }
        x.dx = s.d[tk * s.nblk + i];
        const int16_t *bs = s.bs + (size_t)tk * (s.K / 16) + 16 * i + 8 * h + p;
#pragma unroll
        for (int k = 0; k < 4; ++k) x.bs32[k] = 32 * (int)bs[2 * k];
    }
    struct W {
        uint4 A, B, H;
        uint2 sc;
        uint32_t d;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const int i = unit >> 2, h = (unit >> 1) & 1, p = unit & 1;
        const uint8_t *sb = a.w + (size_t)row * a.row_bytes + (size_t)i * kBytesQ6_K;
        w.A = ldg16_a2(sb + 64 * h + 16 * p);  // 210-byte super-blocks: sb is only even
        w.B = ldg16_a2(sb + 64 * h + 32 + 16 * p);
        w.H = ldg16_a2(sb + 128 + 32 * h + 16 * p);
        w.sc = ldg8_a2(sb + 192 + 8 * h);
        w.d = *reinterpret_cast<const uint16_t *>(sb + 208);
    }
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        const int p = unit & 1;
        const float d = f16_bits_to_f32(w.d);
        // sc[8h + 2k + p], k = 0..3: bytes p, 2+p of sc.x and p, 2+p of sc.y
        int sc[4];
        sc[0] = (int)(int8_t)((w.sc.x >> (8 * p)) & 0xffu);
        sc[1] = (int)(int8_t)((w.sc.x >> (8 * (2 + p))) & 0xffu);
        sc[2] = (int)(int8_t)((w.sc.y >> (8 * p)) & 0xffu);
        sc[3] = (int)(int8_t)((w.sc.y >> (8 * (2 + p))) & 0xffu);
        const uint32_t A[4] = {w.A.x, w.A.y, w.A.z, w.A.w};
        const uint32_t B[4] = {w.B.x, w.B.y, w.B.z, w.B.w};
        const uint32_t H[4] = {w.H.x, w.H.y, w.H.z, w.H.w};
        uint32_t c[4][4];  // unsigned 6-bit codes, [quarter k][dword]
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            c[0][v] = (A[v] & 0x0f0f0f0fu) | ((H[v] << 4) & 0x30303030u);
            c[1][v] = (B[v] & 0x0f0f0f0fu) | ((H[v] << 2) & 0x30303030u);
            c[2][v] = ((A[v] >> 4) & 0x0f0f0f0fu) | (H[v] & 0x30303030u);
            c[3][v] = ((B[v] >> 4) & 0x0f0f0f0fu) | ((H[v] >> 2) & 0x30303030u);
        }
        {
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                int dk = 0;
#pragma unroll
                for (int v = 0; v < 4; ++v) dk = sdot4(c[k][v], xa.q[4 * k + v], dk);
                isum += sc[k] * (dk - xa.bs32[k]);
            }
            acc = fmaf(xa.dx * d, (float)isum, acc);
        }
    }
};

// ------------------------------------------------------------------ Q8_0

struct FmtQ80 {
    static constexpr int kUnitsPerBlock = 1;  // one 32-element block
    struct Act {
        uint32_t q[8];
        float dx;
    };
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const uint8_t *blk = a.xq + (size_t)tk * a.xq_stride + (size_t)unit * kBytesQ8_0;
        const uint4 t0 = ldg16_a2(blk + 2), t1 = ldg16_a2(blk + 18);  // 34-byte blocks
        x.q[0] = t0.x; x.q[1] = t0.y; x.q[2] = t0.z; x.q[3] = t0.w;
        x.q[4] = t1.x; x.q[5] = t1.y; x.q[6] = t1.z; x.q[7] = t1.w;
        x.dx = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
    }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) {
        const uint4 *p = reinterpret_cast<const uint4 *>(s.q + (size_t)tk * s.K + 32 * unit);
        const uint4 t0 = p[0], t1 = p[1];
        x.q[0] = t0.x; x.q[1] = t0.y; x.q[2] = t0.z; x.q[3] = t0.w;
        x.q[4] = t1.x; x.q[5] = t1.y; x.q[6] = t1.z; x.q[7] = t1.w;
        x.dx = s.d[tk * s.nblk + unit];
    }
    struct W {
        uint4 q0, q1;
        uint32_t d;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const uint8_t *blk = a.w + (size_t)row * a.row_bytes + (size_t)unit * kBytesQ8_0;
        w.d = *reinterpret_cast<const uint16_t *>(blk);
        w.q0 = ldg16_a2(blk + 2);  // 34-byte blocks: blk is only even
        w.q1 = ldg16_a2(blk + 18);
    }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        {
            int s = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) s = sdot4(q[k], xa.q[k], s);
            acc = fmaf(d * xa.dx, (float)s, acc);
        }
    }
};

// ------------------------------------------------------- Q4_0 / Q5_0 / Q5_K

// Q8_0 activation slice plus its code sum: the 4- and 5-bit formats store
// unsigned codes c with value c - 8 (Q4_0) or c - 16 (Q5_0), so a block's
// integer sum is sum(c * q8) - off * sum(q8), both with sdot4 on codes that
// fit a signed byte.
struct ActQ80S {
    uint32_t q[8];
    float dx;
    int sx;  // sum of the 32 int8 codes
};

template <class A>
__device__ static void load_act_q80s(const A &a, int unit, int tk, ActQ80S &x) {
    FmtQ80::Act t;
    FmtQ80::load_act(a, unit, tk, t);
    int sx = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        x.q[k] = t.q[k];
        sx = sdot4(0x01010101u, t.q[k], sx);
    }
    x.dx = t.dx;
    x.sx = sx;
}

__device__ static void load_act_lds_q80s(const ActLds &s, int unit, int tk, ActQ80S &x) {
    FmtQ80::Act t;
    FmtQ80::load_act_lds(s, unit, tk, t);
    int sx = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        x.q[k] = t.q[k];
        sx = sdot4(0x01010101u, t.q[k], sx);
    }
    x.dx = t.dx;
    x.sx = sx;
}

// Q4_0 rows against Q8_0 activations.  Unit = one 18-byte block: dword k of
// qs holds elements 4k..4k+3 (low nibbles) and 16+4k..16+4k+3 (high).
struct FmtQ40 {
    static constexpr int kUnitsPerBlock = 1;
    using Act = ActQ80S;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { load_act_q80s(a, unit, tk, x); }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) { load_act_lds_q80s(s, unit, tk, x); }
    struct W {
        uint4 q;
        uint32_t d;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const uint8_t *blk = a.w + (size_t)row * a.row_bytes + (size_t)unit * kBytesQ4_0;
        w.d = ldg_unaligned<uint16_t>(blk);
        w.q = ldg16_a2(blk + 2);  // 18-byte blocks
    }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        int s = -8 * xa.sx;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s = sdot4(q[k] & 0x0f0f0f0fu, xa.q[k], s);
            s = sdot4((q[k] >> 4) & 0x0f0f0f0fu, xa.q[4 + k], s);
        }
        acc = fmaf(d * xa.dx, (float)s, acc);
    }
};

// Four bits t (0..15) to bit 4 of four bytes: the multiplier's shifted copies
// of t do not overlap, so the product is their OR.
__device__ __forceinline__ uint32_t spread4_bit4(uint32_t t) { return (t * 0x02040810u) & 0x10101010u; }

// Q5_0 rows against Q8_0 activations.  Unit = one 22-byte block; the fifth
// bit of element e is bit e of qh.
struct FmtQ50 {
    static constexpr int kUnitsPerBlock = 1;
    using Act = ActQ80S;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { load_act_q80s(a, unit, tk, x); }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) { load_act_lds_q80s(s, unit, tk, x); }
    struct W {
        uint4 q;
        uint32_t qh;
        uint32_t d;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const uint8_t *blk = a.w + (size_t)row * a.row_bytes + (size_t)unit * kBytesQ5_0;
        const uint2 h = ldg8_a2(blk);  // 22-byte blocks: d, qh, 2 bytes of qs
        w.d = h.x & 0xffffu;
        w.qh = __builtin_amdgcn_alignbyte(h.y, h.x, 2);
        w.q = ldg16_a2(blk + 6);
    }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        int s = -16 * xa.sx;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = (q[k] & 0x0f0f0f0fu) | spread4_bit4((w.qh >> (4 * k)) & 0xfu);
            const uint32_t hi = ((q[k] >> 4) & 0x0f0f0f0fu) | spread4_bit4((w.qh >> (16 + 4 * k)) & 0xfu);
            s = sdot4(lo, xa.q[k], s);
            s = sdot4(hi, xa.q[4 + k], s);
        }
        acc = fmaf(d * xa.dx, (float)s, acc);
    }
};

// Q5_K rows against Q8_K activations.  Unit = (super-block i, 64-chunk j) as
// Q4_K; the 32 qh bytes hold the fifth bits of chunk j at bits 2j (first 32
// elements) and 2j+1 (next 32).
struct FmtQ5K {
    static constexpr int kUnitsPerBlock = 4;
    using Act = FmtQ4K::Act;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { FmtQ4K::load_act(a, unit, tk, x); }
    __device__ static void load_act_lds(const ActLds &s, int unit, int tk, Act &x) {
        FmtQ4K::load_act_lds(s, unit, tk, x);
    }
    struct W {
        uint4 h, q0, q1, h0, h1;
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const int i = unit >> 2, j = unit & 3;
        const uint8_t *sb = a.w + (size_t)row * a.row_bytes + (size_t)i * kBytesQ5_K;
        w.h = ldg16(sb);
        w.h0 = ldg16(sb + 16);
        w.h1 = ldg16(sb + 32);
        w.q0 = ldg16(sb + 48 + 32 * j);
        w.q1 = ldg16(sb + 64 + 32 * j);
    }
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        const int j = unit & 3;
        const float d = f16_bits_to_f32(w.h.x & 0xffffu);
        const float dmin = f16_bits_to_f32(w.h.x >> 16);
        // six-bit scale/min pairs of sub-blocks 2j, 2j+1, as Q4_K
        const int sh = 16 * (j & 1);
        uint32_t scp, mp;
        if (j < 2) {
            scp = (w.h.y >> sh) & 0x3f3fu;
            mp = (w.h.z >> sh) & 0x3f3fu;
        } else {
            scp = ((w.h.w >> sh) & 0x0f0fu) | (((w.h.y >> sh) >> 2) & 0x3030u);
            mp = (((w.h.w >> sh) >> 4) & 0x0f0fu) | (((w.h.z >> sh) >> 2) & 0x3030u);
        }
        const int sc0 = (int)(scp & 0xffu), sc1 = (int)(scp >> 8);
        const uint32_t mpair = (mp & 0xffu) | ((mp & 0xff00u) << 8);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const uint32_t hw[8] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t lo = (qw[k] & 0x0f0f0f0fu) | (((hw[k] >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t hi = ((qw[k] >> 4) & 0x0f0f0f0fu) | (((hw[k] >> (2 * j + 1)) & 0x01010101u) << 4);
            dlo = sdot4(lo, xa.q[k], dlo);
            dhi = sdot4(hi, xa.q[8 + k], dhi);
        }
        const int isum = sc0 * dlo + sc1 * dhi;
        const int imin = sdot2(mpair, xa.spair, 0);
        acc = fmaf(xa.dx * d, (float)isum, acc);
        acc = fmaf(-(xa.dx * dmin), (float)imin, acc);
    }
};

// ------------------------------------------------------------ f32 activations

// Sum of 16 consecutive activation floats in a fixed order: four pairs of
// pairs, accumulated from 0 (the 16-element sums the f32 K-quant dots take
// for their min / offset terms).
__device__ __forceinline__ float sum16(const float *x) {
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) s += (x[4 * v] + x[4 * v + 1]) + (x[4 * v + 2] + x[4 * v + 3]);
    return s;
}

// Q4_K weights against f32 activations (logits path, dot_q4_k).
// Unit = (super-block i, 64-chunk j); the activation slice is 64 floats.
struct FmtQ4KF32 {
    static constexpr int kUnitsPerBlock = 4;
    struct Act {
        float x[64];
        float sx0, sx1;   // sums of x over sub-blocks 2j and 2j+1
    };
    template <class A>  // GemvArgs or FusedArgs: a.xf, a.K
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const int i = unit >> 2, j = unit & 3;
        const float4 *p = reinterpret_cast<const float4 *>(a.xf + (size_t)tk * a.K + 256 * i + 64 * j);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float4 t = p[v];
            x.x[4 * v] = t.x; x.x[4 * v + 1] = t.y; x.x[4 * v + 2] = t.z; x.x[4 * v + 3] = t.w;
        }
        x.sx0 = sum16(x.x) + sum16(x.x + 16);
        x.sx1 = sum16(x.x + 32) + sum16(x.x + 48);
    }
    using W = FmtQ4K::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ4K::load_w(a, row, unit, w); }
    // Every token's dot with the unit's weights, each weight converted once.
    // The 4-bit codes go to f32 as fp8 (E4M3) bytes: a byte q < 16 is the
    // subnormal or first-binade value q * 2^-9 exactly (one conversion per
    // pair of codes), and the sub-block scales carry the 2^9 back (d * 512 *
    // sc is exact: 11 + 6 significant bits).  Every product and partial sum
    // is the one of (float)q * x scaled by 2^-9 exactly, so the roundings are
    // those of the plain loop unless a partial sum falls below 2^-117.
    template <int M>
    __device__ static void dotm(const W &w, int unit, const Act (&xa)[M], float *acc) {
        const int j = unit & 3;
        const float d = f16_bits_to_f32(w.h.x & 0xffffu) * 512.0f;
        const float dmin = f16_bits_to_f32(w.h.x >> 16);
        const int sh = 16 * (j & 1);
        uint32_t scp, mp;
        if (j < 2) {
            scp = (w.h.y >> sh) & 0x3f3fu;
            mp = (w.h.z >> sh) & 0x3f3fu;
        } else {
            scp = ((w.h.w >> sh) & 0x0f0fu) | (((w.h.y >> sh) >> 2) & 0x3030u);
            mp = (((w.h.w >> sh) >> 4) & 0x0f0fu) | (((w.h.z >> sh) >> 2) & 0x3030u);
        }
        const float d1 = d * (float)(scp & 0xffu), d2 = d * (float)(scp >> 8);
        const float m1 = dmin * (float)(mp & 0xffu), m2 = dmin * (float)(mp >> 8);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        float qlo[M], qhi[M];
#pragma unroll
        for (int t = 0; t < M; ++t) qlo[t] = qhi[t] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int lo = (int)(qw[k] & 0x0f0f0f0fu), hi = (int)((qw[k] >> 4) & 0x0f0f0f0fu);
            const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
#pragma unroll
            for (int t = 0; t < M; ++t) {
                qlo[t] = fmaf(l01[0], xa[t].x[4 * k + 0], qlo[t]);
                qlo[t] = fmaf(l01[1], xa[t].x[4 * k + 1], qlo[t]);
                qlo[t] = fmaf(l23[0], xa[t].x[4 * k + 2], qlo[t]);
                qlo[t] = fmaf(l23[1], xa[t].x[4 * k + 3], qlo[t]);
                qhi[t] = fmaf(h01[0], xa[t].x[32 + 4 * k + 0], qhi[t]);
                qhi[t] = fmaf(h01[1], xa[t].x[32 + 4 * k + 1], qhi[t]);
                qhi[t] = fmaf(h23[0], xa[t].x[32 + 4 * k + 2], qhi[t]);
                qhi[t] = fmaf(h23[1], xa[t].x[32 + 4 * k + 3], qhi[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < M; ++t) {
            float r = d1 * qlo[t] - m1 * xa[t].sx0;
            r += d2 * qhi[t] - m2 * xa[t].sx1;
            acc[t] += r;
        }
    }
    static constexpr bool kTokensShareW = true;  // dotm: M tokens per weight conversion
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        dotm<1>(w, unit, reinterpret_cast<const Act(&)[1]>(xa), &acc);
    }
};

// Q6_K weights against f32 activations (logits path, dot_q6_k).
// Unit = (super-block i, half h, l-half p): 4 sub-blocks of 16 elements.
struct FmtQ6KF32 {
    static constexpr int kUnitsPerBlock = 4;
    struct Act {
        float x[64];      // [k][16]
        float sx[4];      // sums of x per sub-block 8h+2k+p
    };
    template <class A>  // GemvArgs or FusedArgs: a.xf, a.K
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const int i = unit >> 2, h = (unit >> 1) & 1, p = unit & 1;
        const float *base = a.xf + (size_t)tk * a.K + 256 * i + 128 * h + 16 * p;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 *q = reinterpret_cast<const float4 *>(base + 32 * k);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float4 t = q[v];
                x.x[16 * k + 4 * v] = t.x; x.x[16 * k + 4 * v + 1] = t.y;
                x.x[16 * k + 4 * v + 2] = t.z; x.x[16 * k + 4 * v + 3] = t.w;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) x.sx[k] = sum16(x.x + 16 * k);
    }
    using W = FmtQ6K::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ6K::load_w(a, row, unit, w); }
    // Every token's dot with the unit's weights, each code converted once.
    template <int M>
    __device__ static void dotm(const W &w, int unit, const Act (&xa)[M], float *acc) {
        const int p = unit & 1;
        const float d = f16_bits_to_f32(w.d);
        float ds[4];
        ds[0] = d * (float)(int8_t)((w.sc.x >> (8 * p)) & 0xffu);
        ds[1] = d * (float)(int8_t)((w.sc.x >> (8 * (2 + p))) & 0xffu);
        ds[2] = d * (float)(int8_t)((w.sc.y >> (8 * p)) & 0xffu);
        ds[3] = d * (float)(int8_t)((w.sc.y >> (8 * (2 + p))) & 0xffu);
        const uint32_t A[4] = {w.A.x, w.A.y, w.A.z, w.A.w};
        const uint32_t B[4] = {w.B.x, w.B.y, w.B.z, w.B.w};
        const uint32_t H[4] = {w.H.x, w.H.y, w.H.z, w.H.w};
        uint32_t c[4][4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            c[0][v] = (A[v] & 0x0f0f0f0fu) | ((H[v] << 4) & 0x30303030u);
            c[1][v] = (B[v] & 0x0f0f0f0fu) | ((H[v] << 2) & 0x30303030u);
            c[2][v] = ((A[v] >> 4) & 0x0f0f0f0fu) | (H[v] & 0x30303030u);
            c[3][v] = ((B[v] >> 4) & 0x0f0f0f0fu) | ((H[v] >> 2) & 0x30303030u);
        }
        float r[M];
#pragma unroll
        for (int t = 0; t < M; ++t) r[t] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float s[M];
#pragma unroll
            for (int t = 0; t < M; ++t) s[t] = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t cv = c[k][v];
                const float f0 = (float)(cv & 0xffu), f1 = (float)((cv >> 8) & 0xffu);
                const float f2 = (float)((cv >> 16) & 0xffu), f3 = (float)(cv >> 24);
#pragma unroll
                for (int t = 0; t < M; ++t) {
                    s[t] = fmaf(f0, xa[t].x[16 * k + 4 * v + 0], s[t]);
                    s[t] = fmaf(f1, xa[t].x[16 * k + 4 * v + 1], s[t]);
                    s[t] = fmaf(f2, xa[t].x[16 * k + 4 * v + 2], s[t]);
                    s[t] = fmaf(f3, xa[t].x[16 * k + 4 * v + 3], s[t]);
                }
            }
            // sum (q-32)*x = sum q*x - 32*sum x
#pragma unroll
            for (int t = 0; t < M; ++t) r[t] = fmaf(ds[k], fmaf(-32.0f, xa[t].sx[k], s[t]), r[t]);
        }
#pragma unroll
        for (int t = 0; t < M; ++t) acc[t] += r[t];
    }
    static constexpr bool kTokensShareW = true;  // dotm: M tokens per weight conversion
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        dotm<1>(w, unit, reinterpret_cast<const Act(&)[1]>(xa), &acc);
    }
};

// Q8_0 weights against f32 activations (dot_q8_0; used when the activation
// cannot be quantized).  Unit = one block.
struct FmtQ80F32 {
    static constexpr int kUnitsPerBlock = 1;
    struct Act {
        float x[32];
    };
    template <class A>  // GemvArgs or FusedArgs: a.xf, a.K
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) {
        const float4 *p = reinterpret_cast<const float4 *>(a.xf + (size_t)tk * a.K + 32 * unit);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 t = p[v];
            x.x[4 * v] = t.x; x.x[4 * v + 1] = t.y; x.x[4 * v + 2] = t.z; x.x[4 * v + 3] = t.w;
        }
    }
    using W = FmtQ80::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ80::load_w(a, row, unit, w); }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                s = fmaf((float)(int8_t)(q[k] & 0xffu), xa.x[4 * k + 0], s);
                s = fmaf((float)(int8_t)((q[k] >> 8) & 0xffu), xa.x[4 * k + 1], s);
                s = fmaf((float)(int8_t)((q[k] >> 16) & 0xffu), xa.x[4 * k + 2], s);
                s = fmaf((float)(int8_t)(q[k] >> 24), xa.x[4 * k + 3], s);
            }
            acc = fmaf(d, s, acc);
        }
    }
};

// 32-float activation slice of one 32-element unit (the f32 paths below).
struct ActF32x32 {
    float x[32];
};

template <class A>
__device__ static void load_act_f32x32(const A &a, int unit, int tk, ActF32x32 &x) {
    const float4 *p = reinterpret_cast<const float4 *>(a.xf + (size_t)tk * a.K + 32 * unit);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        const float4 t = p[v];
        x.x[4 * v] = t.x; x.x[4 * v + 1] = t.y; x.x[4 * v + 2] = t.z; x.x[4 * v + 3] = t.w;
    }
}

// Q4_0 / Q5_0 rows against f32 activations (dot_q4_0, dot_q5_0).  Unit = one block.
struct FmtQ40F32 {
    static constexpr int kUnitsPerBlock = 1;
    using Act = ActF32x32;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { load_act_f32x32(a, unit, tk, x); }
    using W = FmtQ40::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ40::load_w(a, row, unit, w); }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t c = (q[k] >> (8 * e)) & 0xffu;
                s = fmaf((float)(int)(c & 0x0fu) - 8.0f, xa.x[4 * k + e], s);
                s = fmaf((float)(int)(c >> 4) - 8.0f, xa.x[16 + 4 * k + e], s);
            }
        }
        acc = fmaf(d, s, acc);
    }
};

struct FmtQ50F32 {
    static constexpr int kUnitsPerBlock = 1;
    using Act = ActF32x32;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { load_act_f32x32(a, unit, tk, x); }
    using W = FmtQ50::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ50::load_w(a, row, unit, w); }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        const float d = f16_bits_to_f32(w.d);
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int l = 4 * k + e;
                const uint32_t c = (q[k] >> (8 * e)) & 0xffu;
                const int c0 = (int)(c & 0x0fu) | (int)(((w.qh >> l) & 1u) << 4);
                const int c1 = (int)(c >> 4) | (int)(((w.qh >> (l + 16)) & 1u) << 4);
                s = fmaf((float)(c0 - 16), xa.x[l], s);
                s = fmaf((float)(c1 - 16), xa.x[16 + l], s);
            }
        }
        acc = fmaf(d, s, acc);
    }
};

// F16 rows against f32 activations (dot_f16).  Unit = 32 elements (64 bytes).
struct FmtF16F32 {
    static constexpr int kUnitsPerBlock = 1;
    using Act = ActF32x32;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { load_act_f32x32(a, unit, tk, x); }
    struct W {
        uint4 v[4];
    };
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) {
        const uint8_t *p = a.w + (size_t)row * a.row_bytes + (size_t)unit * 64;
#pragma unroll
        for (int k = 0; k < 4; ++k) w.v[k] = ldg16(p + 16 * k);
    }
    __device__ static void dot1(const W &w, int, const Act &xa, float &acc) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t u[4] = {w.v[k].x, w.v[k].y, w.v[k].z, w.v[k].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = fmaf(f16_bits_to_f32(u[e] & 0xffffu), xa.x[8 * k + 2 * e], s);
                s = fmaf(f16_bits_to_f32(u[e] >> 16), xa.x[8 * k + 2 * e + 1], s);
            }
        }
        acc += s;
    }
};

// Q5_K rows against f32 activations (dot_q5_k).  Unit = (super-block i,
// 64-chunk j) with the 64-float slice and its two 32-element sums, as Q4_K.
struct FmtQ5KF32 {
    static constexpr int kUnitsPerBlock = 4;
    using Act = FmtQ4KF32::Act;
    template <class A>
    __device__ static void load_act(const A &a, int unit, int tk, Act &x) { FmtQ4KF32::load_act(a, unit, tk, x); }
    using W = FmtQ5K::W;
    template <class A>
    __device__ static void load_w(const A &a, int row, int unit, W &w) { FmtQ5K::load_w(a, row, unit, w); }
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
        const int j = unit & 3;
        const float d = f16_bits_to_f32(w.h.x & 0xffffu);
        const float dmin = f16_bits_to_f32(w.h.x >> 16);
        const int sh = 16 * (j & 1);
        uint32_t scp, mp;
        if (j < 2) {
            scp = (w.h.y >> sh) & 0x3f3fu;
            mp = (w.h.z >> sh) & 0x3f3fu;
        } else {
            scp = ((w.h.w >> sh) & 0x0f0fu) | (((w.h.y >> sh) >> 2) & 0x3030u);
            mp = (((w.h.w >> sh) >> 4) & 0x0f0fu) | (((w.h.z >> sh) >> 2) & 0x3030u);
        }
        const float d1 = d * (float)(scp & 0xffu), d2 = d * (float)(scp >> 8);
        const float m1 = dmin * (float)(mp & 0xffu), m2 = dmin * (float)(mp >> 8);
        const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const uint32_t hw[8] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w};
        float qlo = 0.0f, qhi = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t lo = (qw[k] & 0x0f0f0f0fu) | (((hw[k] >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t hi = ((qw[k] >> 4) & 0x0f0f0f0fu) | (((hw[k] >> (2 * j + 1)) & 0x01010101u) << 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qlo = fmaf((float)((lo >> (8 * e)) & 0xffu), xa.x[4 * k + e], qlo);
                qhi = fmaf((float)((hi >> (8 * e)) & 0xffu), xa.x[32 + 4 * k + e], qhi);
            }
        }
        float r = d1 * qlo - m1 * xa.sx0;
        r += d2 * qhi - m2 * xa.sx1;
        acc += r;
    }
};

}  // namespace exq
