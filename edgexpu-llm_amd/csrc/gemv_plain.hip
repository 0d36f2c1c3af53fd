// Plain-float rows times f32 activations, for m <= 8 tokens per launch:
//
//   F32 rows            -- dot_f32_row, src/gguf_quant.c:506-536, and the
//                          one-token edgexpu_cpu_linear, src/cpu_kernel.c:462-523
//   F16 rows of a length that is no multiple of 32
//                       -- dot_f16, src/gguf_quant.c:796-808 (lengths that
//                          are multiples of 32 take the tiled F16 kernel)
//
// y[t][o] = bias[o] + W[o]·x[t].  For F32 the reference sums in eight fp32
// lanes and adds the lane total and the tail in double, for F16 it sums every
// product in double, element by element; here every product w*x is
// formed exactly in double (24-bit by 24-bit significands) and summed in
// double, so the one rounding to float at the end is the only fp32 rounding:
// the result is the correctly summed dot to within K·2^-53 of S = Σ|w x|.
// The bias is added as the reference adds it: in double before that rounding
// for the one-token F32 linear (acc starts at (double)bias), in float after
// it everywhere else (out = b + dot).
//
// Work decomposition: a wavefront owns R consecutive rows; lane l takes the
// 8-element chunks l, l+64, l+128, ... of every row (32 B of F32 or 16 B of
// F16 per chunk, so one wave instruction reads 2 KiB / 1 KiB of one row
// contiguously) and the K % 8 tail elements l, l+64, ... after the last
// chunk.  The activation chunk of a token is loaded once per chunk and used
// for the R rows.  The R*M double partials are summed over the 64 lanes by a
// butterfly.  HBM sees the weight rows once; the activations stay in cache.
#include "common.h"

namespace exq {

struct PlainArgs {
    const uint8_t *w;
    size_t row_bytes;
    const float *x;
    int ldx;
    const float *bias;
    float *out;
    int ldo;
    int n_out;
    int K;
    int bias_f64;  // add the bias in double before the final rounding
};

// 8 consecutive elements of a row as floats (exact conversions).
template <int ELEM>
__device__ __forceinline__ void load_row8(const uint8_t *p, float v[8]) {
    if constexpr (ELEM == 4) {
        const uint4 a = ldg16(p), b = ldg16(p + 16);
        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
        v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
        v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
        v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
    } else {
        const uint4 a = ldg16(p);
        const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = f16_bits_to_f32(u[e] & 0xffffu);
            v[2 * e + 1] = f16_bits_to_f32(u[e] >> 16);
        }
    }
}

template <int ELEM>
__device__ __forceinline__ float load_row1(const uint8_t *p) {
    if constexpr (ELEM == 4) return __uint_as_float(ldg4(p));
    else return f16_bits_to_f32(ldg_unaligned<uint16_t>(p));
}

template <int ELEM, int M, int R>
__global__ __launch_bounds__(256) void gemv_plain_kernel(PlainArgs a) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= a.n_out) return;  // wavefront-uniform
    const uint8_t *wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r] = a.w + (size_t)min(row0 + r, a.n_out - 1) * a.row_bytes;
    double acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < M; ++t) acc[r][t] = 0.0;

    const int nc = a.K >> 3;
    for (int c = lane; c < nc; c += 64) {
        float wv[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) load_row8<ELEM>(wr[r] + (size_t)c * 8 * ELEM, wv[r]);
#pragma unroll
        for (int t = 0; t < M; ++t) {
            float xv[8];
            load_row8<4>(reinterpret_cast<const uint8_t *>(a.x + (size_t)t * a.ldx + (size_t)c * 8), xv);
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r][t] = fma((double)wv[r][e], (double)xv[e], acc[r][t]);
        }
    }
    for (int k = 8 * nc + lane; k < a.K; k += 64) {
#pragma unroll
        for (int t = 0; t < M; ++t) {
            const double xv = (double)a.x[(size_t)t * a.ldx + k];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][t] = fma((double)load_row1<ELEM>(wr[r] + (size_t)k * ELEM), xv, acc[r][t]);
        }
    }

#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < M; ++t) acc[r][t] += __shfl_xor(acc[r][t], off, 64);
    if (lane != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= a.n_out) break;
        const float b = a.bias != nullptr ? a.bias[row] : 0.0f;
#pragma unroll
        for (int t = 0; t < M; ++t)
            a.out[(size_t)t * a.ldo + row] = a.bias_f64 ? (float)((double)b + acc[r][t]) : b + (float)acc[r][t];
    }
}

template <int ELEM, int M, int R>
static hipError_t launch_plain_mr(const PlainArgs &a, hipStream_t st) {
    const int waves = (a.n_out + R - 1) / R;
    hipLaunchKernelGGL((gemv_plain_kernel<ELEM, M, R>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
    return hipGetLastError();
}

// R rows per wave: more rows in flight for one token, fewer registers for many.
template <int ELEM>
static hipError_t launch_plain_m(const PlainArgs &a, int m, hipStream_t st) {
    switch (m) {
        case 1: return launch_plain_mr<ELEM, 1, 4>(a, st);
        case 2: return launch_plain_mr<ELEM, 2, 2>(a, st);
        case 3: return launch_plain_mr<ELEM, 3, 2>(a, st);
        case 4: return launch_plain_mr<ELEM, 4, 2>(a, st);
        case 5: return launch_plain_mr<ELEM, 5, 1>(a, st);
        case 6: return launch_plain_mr<ELEM, 6, 1>(a, st);
        case 7: return launch_plain_mr<ELEM, 7, 1>(a, st);
        case 8: return launch_plain_mr<ELEM, 8, 1>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace exq

using namespace exq;

// F32 / F16 rows (row_bytes apart) times m <= 8 f32 activation rows (ldx
// floats apart); out[t * ldo + o].  Any K >= 1; no alignment needed.
hipError_t launch_gemv_plain(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const float *x,
                             int ldx, const float *bias, bool bias_f64, float *out, int ldo, hipStream_t st) {
    PlainArgs a{};
    a.w = w;
    a.row_bytes = row_bytes;
    a.x = x;
    a.ldx = ldx;
    a.bias = bias;
    a.out = out;
    a.ldo = ldo;
    a.n_out = n_out;
    a.K = K;
    a.bias_f64 = bias_f64 ? 1 : 0;
    if (type == kTypeF32) return launch_plain_m<4>(a, m, st);
    if (type == kTypeF16) return launch_plain_m<2>(a, m, st);
    return hipErrorInvalidValue;
}
