// Decode GEMV kernels of the quantized-weight path: y[t][o] = bias[o] + W[o]·x[t]
// for m <= 8 tokens, with W held as device-resident GGUF rows.
//
//   Q8_0 x Q8_0  -- dot_q8_0_q8_0  src/gguf_dot_q8.c:436-480
//   Q4_K x Q8_K  -- dot_q4_k_q8_k  src/gguf_dot_q8.c:603-762
//   Q6_K x Q8_K  -- dot_q6_k_q8_k  src/gguf_dot_q8.c:897-1002
//   Q4_K/Q6_K/Q8_0 x f32 -- dot_q4_k / dot_q6_k / dot_q8_0, src/gguf_quant.c:539-794
//     (the logits product of src/native.c:445-514 for K-quant output weights)
//   Q4_0 / Q5_0 x Q8_0, Q5_K x Q8_K, and Q4_0 / Q5_0 / Q5_K / F16 x f32: the
//     dispatcher's other formats (src/gguf_dot_q8.c:482-601, 764-895;
//     src/gguf_quant.c:672-702, 796-892)
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
#include <stdlib.h>

#include "formats.h"

namespace exq {

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
        // loads are unconditional (clamped unit) so their count is static;
        // lanes past the last unit discard their products
        const int u = min(unit, a.U - 1);
        const bool use = unit < a.U;
        typename Fmt::W w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + slot + S * r, a.n_out - 1);
            Fmt::load_w(a, row, u, w[r]);
        }
#pragma unroll
        for (int t = 0; t < M; ++t) {
            typename Fmt::Act x;
            Fmt::load_act(a, u, t, x);
            if (use) {
#pragma unroll
                for (int r = 0; r < R; ++r) Fmt::dot1(w[r], u, x, acc[r][t]);
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
    static const int r1 = tuning_knob("EXQ_GEMV_R", 4);  // rows per slot at one token
    switch (a.m) {
        case 1:
            if (r1 == 1) return launch_fmt<Fmt, 1, 1>(a, st);
            if (r1 == 2) return launch_fmt<Fmt, 1, 2>(a, st);
            if (r1 == 8) return launch_fmt<Fmt, 1, 8>(a, st);
            return launch_fmt<Fmt, 1, 4>(a, st);
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
        case kTypeQ4_0: a.nblk = K / kQK8_0; return launch_m<FmtQ40>(a, st);
        case kTypeQ5_0: a.nblk = K / kQK8_0; return launch_m<FmtQ50>(a, st);
        case kTypeQ4_K: a.nblk = K / kQKK; return launch_m<FmtQ4K>(a, st);
        case kTypeQ5_K: a.nblk = K / kQKK; return launch_m<FmtQ5K>(a, st);
        case kTypeQ6_K: a.nblk = K / kQKK; return launch_m<FmtQ6K>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// f32-activation GEMV over m <= 8 rows of x (logits path, F16 rows, the
// per-row f32 dots).  F16 rows need K % 32 == 0.
hipError_t launch_gemv_f32(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m,
                           const float *xf, const float *bias, float *out, int ldo, hipStream_t st) {
    GemvArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.n_out = n_out;
    a.K = K;
    a.m = m;
    a.xf = xf;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    switch (type) {
        case kTypeQ8_0: a.nblk = K / kQK8_0; return launch_m<FmtQ80F32>(a, st);
        case kTypeQ4_0: a.nblk = K / kQK8_0; return launch_m<FmtQ40F32>(a, st);
        case kTypeQ5_0: a.nblk = K / kQK8_0; return launch_m<FmtQ50F32>(a, st);
        case kTypeF16: a.nblk = K / 32; return launch_m<FmtF16F32>(a, st);
        case kTypeQ4_K: a.nblk = K / kQKK; return launch_m<FmtQ4KF32>(a, st);
        case kTypeQ5_K: a.nblk = K / kQKK; return launch_m<FmtQ5KF32>(a, st);
        case kTypeQ6_K: a.nblk = K / kQKK; return launch_m<FmtQ6KF32>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// Greedy argmax over scores with the reference's rules (src/native.c:2355-2396):
// the largest score wins, the lowest index on ties, NaN never wins, and
// index 0 when nothing beats -inf.  Key = (order-preserving score bits, ~index).
__device__ __forceinline__ unsigned long long argmax_key(float s, unsigned idx) {
    if (!(s > -INFINITY)) return 0ull;  // NaN and -inf never win
    // -0.0 and +0.0 compare equal in the reference's `score > best`, so they
    // share one key (the lower index then wins)
    uint32_t u = s == 0.0f ? 0u : __float_as_uint(s);
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

// Pass 2: one 256-thread workgroup per row t reduces its nparts partials
// (at partial + t*stride, 1 <= nparts) to best[t].  Each thread issues its
// first four loads together (clamped indices, so none is conditional): the
// keys were just written by another kernel and every read misses in L2, so
// one round trip rather than one per key bounds the pass.
__global__ __launch_bounds__(256) void argmax_finish_kernel(const unsigned long long *__restrict__ partial,
                                                            int nparts, int stride, uint32_t *__restrict__ best) {
    const unsigned long long *p = partial + (size_t)blockIdx.x * stride;
    __shared__ unsigned long long red[4];
    const int tid = threadIdx.x;
    unsigned long long v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = p[min(tid + 256 * j, nparts - 1)];
    unsigned long long b = v[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) b = v[j] > b ? v[j] : b;
    for (int i = tid + 1024; i < nparts; i += 256) b = p[i] > b ? p[i] : b;
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(b, off, 64);
        b = o > b ? o : b;
    }
    if ((tid & 63) == 0) red[tid >> 6] = b;
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 4; ++k) b = red[k] > b ? red[k] : b;
        best[blockIdx.x] = b != 0ull ? ~(uint32_t)(b & 0xffffffffull) : 0u;
    }
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
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(m), dim3(256), 0, st, partial, grid, kArgmaxParts, best);
    return hipGetLastError();
}

// best[t] from the nparts keys of row t at partial + t*stride (keys written
// by the logits launch's argmax epilogue).
hipError_t launch_argmax_finish(const unsigned long long *partial, int m, int nparts, int stride, uint32_t *best,
                                hipStream_t st) {
    if (nparts < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(m), dim3(256), 0, st, partial, nparts, stride, best);
    return hipGetLastError();
}
