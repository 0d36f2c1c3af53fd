// Decode GEMV kernels of the quantized-weight path: y[t][o] = bias[o] + W[o]·x[t]
// for m <= 8 tokens, with W held as device-resident GGUF rows.
//
//   Q8_0 x Q8_0  -- dot_q8_0_q8_0  src/gguf_dot_q8.c:436-480
//   Q4_K x Q8_K  -- dot_q4_k_q8_k  src/gguf_dot_q8.c:603-762
//   Q6_K x Q8_K  -- dot_q6_k_q8_k  src/gguf_dot_q8.c:897-1002
//   Q4_K/Q6_K/Q8_0 x f32 -- dot_q4_k / dot_q6_k / dot_q8_0, src/gguf_quant.c:539-794
//     (the logits product of src/native.c:445-514 for K-quant output weights)
//
// Work decomposition.  A row's K range is cut into U "units" (64 elements of
// one super-block for the K-quants, one 32-element block for Q8_0).  A
// wavefront is split into S = 64/G slots of G lanes; lane g of a slot owns
// units g, g+G, g+2G, ... of every row it visits, and one wavefront covers
// S*R rows (R rows per slot).  A lane loads the activation slice of its unit
// once and reuses it for the R rows, so HBM sees only the weight stream; the
// activation slices stay in L1/L2.  Integer block sums are exact (sdot4 on
// the int8 codes); their fp32 combination differs from the reference only in
// summation order.  At the end the R*M partial sums are reduced over each
// G-lane slot.
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
    const float *xs;         // [m][K/16] 16-element sums of x (f32 path)
    const float *bias;       // [n_out] or null
    float *out;              // [m][ldo]
    int ldo;
};

// ------------------------------------------------------------------ Q4_K

struct FmtQ4K {
    static constexpr int kUnitsPerBlock = 4;  // (super-block i, 64-chunk j)
    struct Act {
        uint32_t q[16];   // codes of elements 64j..64j+63 of super-block i
        float dx;         // Q8_K block scale
        uint32_t spair;   // int16 pair: sums of sub-blocks 2j and 2j+1
    };
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
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
    struct W {
        uint4 h, q0, q1;
    };
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) {
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
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
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
    struct W {
        uint4 A, B, H;
        uint2 sc;
        uint32_t d;
    };
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) {
        const int i = unit >> 2, h = (unit >> 1) & 1, p = unit & 1;
        const uint8_t *sb = a.w + (size_t)row * a.row_bytes + (size_t)i * kBytesQ6_K;
        w.A = ldg16(sb + 64 * h + 16 * p);
        w.B = ldg16(sb + 64 * h + 32 + 16 * p);
        w.H = ldg16(sb + 128 + 32 * h + 16 * p);
        w.sc = ldg8(sb + 192 + 8 * h);
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
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
        const uint8_t *blk = a.xq + (size_t)tk * a.xq_stride + (size_t)unit * kBytesQ8_0;
        const uint4 t0 = ldg16(blk + 2), t1 = ldg16(blk + 18);
        x.q[0] = t0.x; x.q[1] = t0.y; x.q[2] = t0.z; x.q[3] = t0.w;
        x.q[4] = t1.x; x.q[5] = t1.y; x.q[6] = t1.z; x.q[7] = t1.w;
        x.dx = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
    }
    struct W {
        uint4 q0, q1;
        uint32_t d;
    };
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) {
        const uint8_t *blk = a.w + (size_t)row * a.row_bytes + (size_t)unit * kBytesQ8_0;
        w.d = *reinterpret_cast<const uint16_t *>(blk);
        w.q0 = ldg16(blk + 2);
        w.q1 = ldg16(blk + 18);
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

// ------------------------------------------------------------ f32 activations

// Q4_K weights against f32 activations (logits path, dot_q4_k).
// Unit = (super-block i, 64-chunk j); the activation slice is 64 floats.
struct FmtQ4KF32 {
    static constexpr int kUnitsPerBlock = 4;
    struct Act {
        float x[64];
        float sx0, sx1;   // sums of x over sub-blocks 2j and 2j+1
    };
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
        const int i = unit >> 2, j = unit & 3;
        const float4 *p = reinterpret_cast<const float4 *>(a.xf + (size_t)tk * a.K + 256 * i + 64 * j);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float4 t = p[v];
            x.x[4 * v] = t.x; x.x[4 * v + 1] = t.y; x.x[4 * v + 2] = t.z; x.x[4 * v + 3] = t.w;
        }
        const float *s = a.xs + (size_t)tk * (a.K / 16) + 16 * i + 4 * j;
        x.sx0 = s[0] + s[1];
        x.sx1 = s[2] + s[3];
    }
    using W = FmtQ4K::W;
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) { FmtQ4K::load_w(a, row, unit, w); }
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
        {
            float qlo = 0.0f, qhi = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t lo = qw[k] & 0x0f0f0f0fu;
                const uint32_t hi = (qw[k] >> 4) & 0x0f0f0f0fu;
                qlo = fmaf((float)(lo & 0xffu), xa.x[4 * k + 0], qlo);
                qlo = fmaf((float)((lo >> 8) & 0xffu), xa.x[4 * k + 1], qlo);
                qlo = fmaf((float)((lo >> 16) & 0xffu), xa.x[4 * k + 2], qlo);
                qlo = fmaf((float)(lo >> 24), xa.x[4 * k + 3], qlo);
                qhi = fmaf((float)(hi & 0xffu), xa.x[32 + 4 * k + 0], qhi);
                qhi = fmaf((float)((hi >> 8) & 0xffu), xa.x[32 + 4 * k + 1], qhi);
                qhi = fmaf((float)((hi >> 16) & 0xffu), xa.x[32 + 4 * k + 2], qhi);
                qhi = fmaf((float)(hi >> 24), xa.x[32 + 4 * k + 3], qhi);
            }
            float r = d1 * qlo - m1 * xa.sx0;
            r += d2 * qhi - m2 * xa.sx1;
            acc += r;
        }
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
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
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
        const float *s = a.xs + (size_t)tk * (a.K / 16) + 16 * i + 8 * h + p;
#pragma unroll
        for (int k = 0; k < 4; ++k) x.sx[k] = s[2 * k];
    }
    using W = FmtQ6K::W;
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) { FmtQ6K::load_w(a, row, unit, w); }
    __device__ static void dot1(const W &w, int unit, const Act &xa, float &acc) {
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
        {
            float r = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float s = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t cv = c[k][v];
                    s = fmaf((float)(cv & 0xffu), xa.x[16 * k + 4 * v + 0], s);
                    s = fmaf((float)((cv >> 8) & 0xffu), xa.x[16 * k + 4 * v + 1], s);
                    s = fmaf((float)((cv >> 16) & 0xffu), xa.x[16 * k + 4 * v + 2], s);
                    s = fmaf((float)(cv >> 24), xa.x[16 * k + 4 * v + 3], s);
                }
                // sum (q-32)*x = sum q*x - 32*sum x
                r = fmaf(ds[k], fmaf(-32.0f, xa.sx[k], s), r);
            }
            acc += r;
        }
    }
};

// Q8_0 weights against f32 activations (dot_q8_0; used when the activation
// cannot be quantized).  Unit = one block.
struct FmtQ80F32 {
    static constexpr int kUnitsPerBlock = 1;
    struct Act {
        float x[32];
    };
    __device__ static void load_act(const GemvArgs &a, int unit, int tk, Act &x) {
        const float4 *p = reinterpret_cast<const float4 *>(a.xf + (size_t)tk * a.K + 32 * unit);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 t = p[v];
            x.x[4 * v] = t.x; x.x[4 * v + 1] = t.y; x.x[4 * v + 2] = t.z; x.x[4 * v + 3] = t.w;
        }
    }
    using W = FmtQ80::W;
    __device__ static void load_w(const GemvArgs &a, int row, int unit, W &w) { FmtQ80::load_w(a, row, unit, w); }
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

// ------------------------------------------------------------------ skeleton

template <class Fmt, int M, int R>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int G = a.G;
    const int S = 64 / G;
    const int slot = lane / G;
    const int gl = lane & (G - 1);
    const int row0 = wave * S * R;
    if (row0 >= a.n_out) return;  // wavefront-uniform
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < M; ++t) acc[r][t] = 0.0f;

    for (int it = 0; it < a.T; ++it) {
        const int unit = gl + G * it;
        if (unit < a.U) {
            // weights stay in registers; the tokens stream through one
            // activation slice at a time
            typename Fmt::W w[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + slot + S * r, a.n_out - 1);
                Fmt::load_w(a, row, unit, w[r]);
            }
#pragma unroll
            for (int t = 0; t < M; ++t) {
                typename Fmt::Act x;
                Fmt::load_act(a, unit, t, x);
#pragma unroll
                for (int r = 0; r < R; ++r) Fmt::dot1(w[r], unit, x, acc[r][t]);
            }
        }
    }

    // R*M partials padded with zeros to a power of two for the halving reduction
    constexpr int NV = R * M;
    constexpr int V = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : NV <= 8 ? 8 : NV <= 16 ? 16 : 32;
    static_assert(NV <= 32, "too many partials per lane");
    float vals[V];
#pragma unroll
    for (int k = 0; k < V; ++k) vals[k] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < M; ++t) vals[r * M + t] = acc[r][t];
    group_reduce<V>(vals, G, lane);
    const int live = group_reduce_live(V, G);
    const int base = group_reduce_index(V, G, gl);
    // lanes left with identical copies of one value: only the lowest writes
    const int spread = V < G ? G / V : 1;
    if ((gl & (spread - 1)) != 0) return;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        if (k >= live) break;
        const int idx = base + k;
        if (idx >= NV) break;  // padding
        const int r = idx / M, t = idx % M;
        const int row = row0 + slot + S * r;
        if (row < a.n_out) {
            const float b = a.bias != nullptr ? a.bias[row] : 0.0f;
            a.out[(size_t)t * a.ldo + row] = b + vals[k];
        }
    }
}

// ------------------------------------------------------------ launch logic

static int pick_group(int U) {
    int best = 64;
    double best_util = -1.0;
    for (int G = 64; G >= 8; G >>= 1) {
        const int T = (U + G - 1) / G;
        const double util = (double)U / (double)(G * T);
        if (util > best_util + 1e-9) {
            best_util = util;
            best = G;
        }
    }
    return best;
}

template <class Fmt, int M, int R>
static hipError_t launch_fmt(GemvArgs a, hipStream_t st) {
    a.U = a.nblk * Fmt::kUnitsPerBlock;
    a.G = pick_group(a.U);
    a.T = (a.U + a.G - 1) / a.G;
    const int S = 64 / a.G;
    const int rows_per_wave = S * R;
    const int waves = (a.n_out + rows_per_wave - 1) / rows_per_wave;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    hipLaunchKernelGGL((gemv_kernel<Fmt, M, R>), dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <class Fmt>
static hipError_t launch_m(GemvArgs a, hipStream_t st) {
    switch (a.m) {
        case 1: return launch_fmt<Fmt, 1, 4>(a, st);
        case 2: return launch_fmt<Fmt, 2, 2>(a, st);
        case 3: return launch_fmt<Fmt, 3, 2>(a, st);
        case 4: return launch_fmt<Fmt, 4, 2>(a, st);
        case 5: return launch_fmt<Fmt, 5, 1>(a, st);
        case 6: return launch_fmt<Fmt, 6, 1>(a, st);
        case 7: return launch_fmt<Fmt, 7, 1>(a, st);
        case 8: return launch_fmt<Fmt, 8, 1>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace exq

using namespace exq;

// Quantized-activation GEMV over m <= 8 tokens; xq holds the tokens' Q8_0 /
// Q8_K block bytes, token t at xq + t*xq_stride.
hipError_t launch_gemv_q8(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m,
                          const uint8_t *xq, size_t xq_stride, const float *bias, float *out, int ldo,
                          hipStream_t st) {
    GemvArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.n_out = n_out;
    a.K = K;
    a.m = m;
    a.xq = xq;
    a.xq_stride = xq_stride;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    switch (type) {
        case kTypeQ8_0: a.nblk = K / kQK8_0; return launch_m<FmtQ80>(a, st);
        case kTypeQ4_K: a.nblk = K / kQKK; return launch_m<FmtQ4K>(a, st);
        case kTypeQ6_K: a.nblk = K / kQKK; return launch_m<FmtQ6K>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// f32-activation GEMV over m <= 8 rows of x (logits path).  xs holds the
// 16-element sums of x ([m][K/16]); unused for Q8_0.
hipError_t launch_gemv_f32(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m,
                           const float *xf, const float *xs, const float *bias, float *out, int ldo,
                           hipStream_t st) {
    GemvArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.n_out = n_out;
    a.K = K;
    a.m = m;
    a.xf = xf;
    a.xs = xs;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    switch (type) {
        case kTypeQ8_0: a.nblk = K / kQK8_0; return launch_m<FmtQ80F32>(a, st);
        case kTypeQ4_K: a.nblk = K / kQKK; return launch_m<FmtQ4KF32>(a, st);
        case kTypeQ6_K: a.nblk = K / kQKK; return launch_m<FmtQ6KF32>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// 16-element sums of f32 activations: xs[t][g] = sum_{e<16} x[t][16g+e].
__global__ __launch_bounds__(256) void xsum16_kernel(const float *__restrict__ x, int m, int K,
                                                     float *__restrict__ xs) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)m * (K / 16);
    if (g >= total) return;
    const float4 *p = reinterpret_cast<const float4 *>(x + g * 16);
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float4 t = p[v];
        s += (t.x + t.y) + (t.z + t.w);
    }
    xs[g] = s;
}

hipError_t launch_xsum16(const float *x, int m, int K, float *xs, hipStream_t st) {
    const long long total = (long long)m * (K / 16);
    hipLaunchKernelGGL(xsum16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, m, K, xs);
    return hipGetLastError();
}

// Greedy argmax over scores with the reference's rules (src/native.c:2355-2396):
// the largest score wins, the lowest index on ties, NaN never wins, and
// index 0 when nothing beats -inf.  Key = (order-preserving score bits, ~index).
__device__ __forceinline__ unsigned long long argmax_key(float s, unsigned idx) {
    if (!(s > -INFINITY)) return 0ull;  // NaN and -inf never win
    uint32_t u = __float_as_uint(s);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(~idx);
}

constexpr int kArgmaxParts = 1024;

// Pass 1: block b reduces a grid-strided share of s[] to partial[b].
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ s, int n,
                                                     unsigned long long *__restrict__ partial) {
    __shared__ unsigned long long red[4];
    unsigned long long best = 0ull;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned long long k = argmax_key(s[i], (unsigned)i);
        best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int k = 1; k < 4; ++k) b = red[k] > b ? red[k] : b;
        partial[blockIdx.x] = b;
    }
}

// Pass 2: one wavefront per row t reduces its nparts partials to best[t].
__global__ __launch_bounds__(64) void argmax_finish_kernel(const unsigned long long *__restrict__ partial,
                                                           int nparts, uint32_t *__restrict__ best) {
    const unsigned long long *p = partial + (size_t)blockIdx.x * kArgmaxParts;
    unsigned long long b = 0ull;
    for (int i = threadIdx.x; i < nparts; i += 64) b = p[i] > b ? p[i] : b;
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(b, off, 64);
        b = o > b ? o : b;
    }
    if (threadIdx.x == 0) best[blockIdx.x] = b != 0ull ? ~(uint32_t)(b & 0xffffffffull) : 0u;
}

// Greedy argmax of m score rows (row t at s + t*lds, n entries) into best[t];
// partial must hold m * 1024 keys.
hipError_t launch_argmax_rows(const float *s, int m, int n, size_t lds, unsigned long long *partial,
                              uint32_t *best, hipStream_t st) {
    int grid = (n + 255) / 256;
    if (grid > kArgmaxParts) grid = kArgmaxParts;
    for (int t = 0; t < m; ++t) {
        hipLaunchKernelGGL(argmax_kernel, dim3(grid), dim3(256), 0, st, s + (size_t)t * lds, n,
                           partial + (size_t)t * kArgmaxParts);
    }
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(m), dim3(64), 0, st, partial, grid, best);
    return hipGetLastError();
}
