// Fused decode GEMV entry points: type dispatch over the kernel and
// schedules of gemv_fused_kernel.h (edgexpu_cpu_linear_quant_batch,
// src/cpu_kernel.c:545-644, and the f32-activation logits product,
// src/native.c:445-462).  The dispatcher's other quantized formats (Q4_0,
// Q5_0, Q5_K) are instantiated in gemv_fused_more.hip.
#include "gemv_fused_kernel.h"

namespace exq {
// gemv_fused_more.hip: plain projections of Q4_0 / Q5_0 / Q5_K rows
hipError_t launch_gemv_fused_more(int type, const FusedArgs &a, bool stage, hipStream_t st);
// gemv_stream.hip: one to four tokens of Q4_K / Q6_K rows at the decode row lengths
bool gemv_stream_f32_take(int type, int K, int m, const uint8_t *w, int n_out);
hipError_t launch_gemv_stream_f32(int type, int K, int m, const uint8_t *w, int n_out, const float *bias,
                                  float *out, const float *xf, unsigned long long *amax, int *nparts, hipStream_t st);
bool gemv_stream_take(int type, int K, int m, long long rows, int nmat, const uint8_t *const *w, int code,
                      bool staged);
hipError_t launch_gemv_stream(int type, int nmat, const uint8_t *const *w, const int *n_out,
                              const float *const *bias, const float *const *resid, float *const *out, int K, int m,
                              const float *x, const uint8_t *xq, const float *x2, const float *nw, float eps, int pro,
                              bool pair, hipStream_t st);
}  // namespace exq

using namespace exq;

// Rows split over three waves (12-wave workgroups) are instantiated for one
// staged token of Q4_K / Q6_K rows (knob EXQ_FUSED_KS3=0: never).
static bool fused_with3(int type, int m, bool staged) {
    static const int ks3 = tuning_knob("EXQ_FUSED_KS3", 1);
    return ks3 != 0 && m == 1 && staged && (type == kTypeQ4_K || type == kTypeQ6_K);
}

// True when the fused kernel covers (type, K, m): every unit in one pass and
// the quantized activation fits the LDS budget.
bool gemv_fused_supported(int type, int K, int m) {
    if (m < 1 || m > 4) return false;
    if (!q8_0_family(type) && !k_family(type)) return false;
    const bool q80 = q8_0_family(type);
    const int U = q80 ? K / kQK8_0 : (K / kQKK) * 4;
    int G = 64, KS = 1;
    if (!pick_fused_shape(U, G, KS)) return false;
    const FusedLds L(m, K, q80 ? K / kQK8_0 : K / kQKK, !q80, 8, 64 / G, 4);
    return L.total() <= 64 * 1024;
}

// True when the fused kernel covers the f32-activation product (one token):
// K-quant logits rows of type Q4_K / Q6_K, Q8_0 when its quantization fails.
bool gemv_fused_f32_supported(int type, int K) {
    if (type != kTypeQ8_0 && type != kTypeQ4_K && type != kTypeQ6_K) return false;
    const int U = type == kTypeQ8_0 ? K / kQK8_0 : (K / kQKK) * 4;
    int G = 64, KS = 1;
    if (!pick_fused_shape(U, G, KS)) return false;
    const FusedLds L(1, K, 0, false, 8, 64 / G, 2, false);
    return L.total() <= 64 * 1024;
}

// One token of f32 activations xf against one matrix: the logits product (src/native.c:445-462).  Rows per
// slot R = 1 or 2 (the activation slice takes the registers of larger R).
namespace {
// The f32 logits launch with the argmax epilogue: the same shapes and
// schedules as launch_gemv_fused_f32, one key per workgroup of the grid.
template <class F, int R, int NW, int LOOP, bool STAGE = false>
hipError_t launch_argmax_fmt(FusedArgs a, hipStream_t st, int *nparts) {
    const hipError_t e = launch_fused_fmt<F, 1, R, NW, STAGE, LOOP, 16>(a, st);
    *nparts = fused_last_grid();
    return e;
}
}  // namespace

hipError_t launch_gemv_fused_f32_argmax(int type, const uint8_t *w, int n_out, const float *bias, float *out,
                                        size_t row_bytes, int K, const float *xf, hipStream_t st,
                                        unsigned long long *amax, int *nparts) {
    FusedArgs a{};
    a.amax_cap = kFusedArgmaxParts;
    a.nmat = 1;
    a.w[0] = w;
    a.n_out[0] = n_out;
    a.bias[0] = bias;
    a.out[0] = out;
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = 1;
    a.xf = xf;
    a.amax = amax;
    a.nblk = type == kTypeQ8_0 ? K / kQK8_0 : K / kQKK;
    a.U = type == kTypeQ8_0 ? a.nblk : a.nblk * 4;
    if (!pick_fused_shape(a.U, a.G, a.KS)) return hipErrorInvalidValue;
    static const int f32_ks3 = tuning_knob("EXQ_FUSED_F32_KS3", 1);
    if (f32_ks3 != 0 && type != kTypeQ8_0 && a.U > 32 && a.U <= 48) {
        a.G = 16;
        a.KS = 3;
        return type == kTypeQ4_K ? launch_argmax_fmt<FmtQ4KF32, 2, 12, 0>(a, st, nparts)
                                 : launch_argmax_fmt<FmtQ6KF32, 2, 12, 0>(a, st, nparts);
    }
    const int rows_per_tile = (64 / a.G) * 2;
    const int tiles = (n_out + rows_per_tile - 1) / rows_per_tile;
    const bool balanced = a.KS == 1 && tiles > 2 * device_cus() * 8 && tuning_knob("EXQ_FUSED_DYN", 1) != 0;
    switch (type) {
        case kTypeQ8_0:
            return balanced ? launch_argmax_fmt<FmtQ80F32, 2, 8, 2>(a, st, nparts)
                            : launch_argmax_fmt<FmtQ80F32, 2, 8, 0>(a, st, nparts);
        case kTypeQ4_K:
            return balanced ? launch_argmax_fmt<FmtQ4KF32, 2, 8, 2>(a, st, nparts)
                            : launch_argmax_fmt<FmtQ4KF32, 2, 8, 0>(a, st, nparts);
        default:
            return balanced ? launch_argmax_fmt<FmtQ6KF32, 2, 8, 2>(a, st, nparts)
                            : launch_argmax_fmt<FmtQ6KF32, 2, 8, 0>(a, st, nparts);
    }
}

// One token of f32 activations x, quantized to Q8_0 inside each workgroup,
// against Q8_0 rows, with the argmax epilogue: the Q8_0 logits product
// (src/native.c:2317-2319) and its greedy pick's per-workgroup keys in one
// launch (at least kFusedArgmaxParts keys at amax, *nparts the count).
hipError_t launch_gemv_fused_q8_0_argmax(const uint8_t *w, int n_out, const float *bias, float *out,
                                         size_t row_bytes, int K, const float *x, hipStream_t st,
                                         unsigned long long *amax, int *nparts) {
    if (!gemv_fused_supported(kTypeQ8_0, K, 1)) return hipErrorInvalidValue;
    FusedArgs a{};
    a.amax_cap = kFusedArgmaxParts;
    a.nmat = 1;
    a.w[0] = w;
    a.n_out[0] = n_out;
    a.bias[0] = bias;
    a.out[0] = out;
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = 1;
    a.x = x;
    a.amax = amax;
    a.nblk = K / kQK8_0;
    a.U = a.nblk;
    if (!pick_fused_shape(a.U, a.G, a.KS) || 8 % a.KS != 0) return hipErrorInvalidValue;
    // more than two workgroups' worth of tiles per CU: the balanced per-wave
    // schedule (logits [49152 x 576]: 11.5 us, against 13.8 us for the two
    // register buffers of the scores-only launch with this epilogue)
    const int r1 = a.KS == 1 && n_out <= 4096 ? 2 : 4;
    const int rows_per_tile = (64 / a.G) * r1;
    const int tiles = (n_out + rows_per_tile - 1) / rows_per_tile;
    if (a.KS == 1 && tiles > 2 * device_cus() * 8) return launch_argmax_fmt<FmtQ80, 2, 8, 2, true>(a, st, nparts);
    return r1 == 2 ? launch_argmax_fmt<FmtQ80, 2, 8, 0, true>(a, st, nparts)
                   : launch_argmax_fmt<FmtQ80, 4, 8, 0, true>(a, st, nparts);
}

// With amax non-null (at least kFusedArgmaxParts keys) the launch also
// writes one greedy-argmax key per workgroup there and *nparts the count.
hipError_t launch_gemv_fused_f32(int type, const uint8_t *w, int n_out, const float *bias, float *out,
                                 size_t row_bytes, int K, const float *xf, hipStream_t st, unsigned long long *amax,
                                 int *nparts) {
    if (!gemv_fused_f32_supported(type, K)) return hipErrorInvalidValue;
    if (gemv_stream_f32_take(type, K, 1, w, n_out))
        return launch_gemv_stream_f32(type, K, 1, w, n_out, bias, out, xf, amax, nparts, st);
    if (amax != nullptr) return launch_gemv_fused_f32_argmax(type, w, n_out, bias, out, row_bytes, K, xf, st, amax, nparts);
    FusedArgs a{};
    a.nmat = 1;
    a.w[0] = w;
    a.n_out[0] = n_out;
    a.bias[0] = bias;
    a.out[0] = out;
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = 1;
    a.xf = xf;
    a.nblk = type == kTypeQ8_0 ? K / kQK8_0 : K / kQKK;
    a.U = type == kTypeQ8_0 ? a.nblk : a.nblk * 4;
    if (!pick_fused_shape(a.U, a.G, a.KS)) return hipErrorInvalidValue;
    static const int r_env = tuning_knob("EXQ_FUSED_F32_R", 2);
    // one row per lane group spills the Q6_K decode's registers; Q6_K keeps two
    const int r1 = r_env == 1 && type != kTypeQ6_K ? 1 : 2;
    const int rows_per_tile = (64 / a.G) * r1;
    const int tiles = (n_out + rows_per_tile - 1) / rows_per_tile;
    const bool balanced = a.KS == 1 && tiles > 2 * device_cus() * 8 && tuning_knob("EXQ_FUSED_DYN", 1) != 0;
#define EXQ_F32_LAUNCH(F)                                                                              \
    return balanced ? (r1 == 1 ? launch_fused_fmt<F, 1, 1, 8, false, 2>(a, st) : launch_fused_fmt<F, 1, 2, 8, false, 2>(a, st)) \
                    : (r1 == 1 ? launch_fused_fmt<F, 1, 1, 8, false, 0>(a, st) : launch_fused_fmt<F, 1, 2, 8, false, 0>(a, st))
    // K-quant rows of 33-48 units (K = 2112..3072): 16-lane slots over three
    // waves use 83 % of the lanes where one 64-lane slot uses 62.5 %
    static const int f32_ks3 = tuning_knob("EXQ_FUSED_F32_KS3", 1);
    if (f32_ks3 != 0 && type != kTypeQ8_0 && a.U > 32 && a.U <= 48) {
        a.G = 16;
        a.KS = 3;
        return type == kTypeQ4_K ? launch_fused_fmt<FmtQ4KF32, 1, 2, 12, false, 0>(a, st)
                                 : launch_fused_fmt<FmtQ6KF32, 1, 2, 12, false, 0>(a, st);
    }
    switch (type) {
        case kTypeQ8_0: EXQ_F32_LAUNCH(FmtQ80F32);
        case kTypeQ4_K: EXQ_F32_LAUNCH(FmtQ4KF32);
        default:
            return balanced ? launch_fused_fmt<FmtQ6KF32, 1, 2, 8, false, 2>(a, st)
                            : launch_fused_fmt<FmtQ6KF32, 1, 2, 8, false, 0>(a, st);
    }
#undef EXQ_F32_LAUNCH
}

// Two tokens of f32 activations (xf, token stride K) against one K-quant matrix, outputs at out and out + n_out: the weights are
// read once for both.  Each score equals the one-token launch's bit for bit
// (the same lane partials, summed by the same reduction tree whichever value
// slot holds them).
hipError_t launch_gemv_fused_f32_pair(int type, const uint8_t *w, int n_out, const float *bias, float *out,
                                      size_t row_bytes, int K, const float *xf, hipStream_t st) {
    if ((type != kTypeQ4_K && type != kTypeQ6_K) || !gemv_fused_f32_supported(type, K)) return hipErrorInvalidValue;
    if (gemv_stream_f32_take(type, K, 2, w, n_out))
        return launch_gemv_stream_f32(type, K, 2, w, n_out, bias, out, xf, nullptr, nullptr, st);
    FusedArgs a{};
    a.nmat = 1;
    a.w[0] = w;
    a.n_out[0] = n_out;
    a.bias[0] = bias;
    a.out[0] = out;
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = 2;
    a.xf = xf;
    a.nblk = K / kQKK;
    a.U = a.nblk * 4;
    if (!pick_fused_shape(a.U, a.G, a.KS)) return hipErrorInvalidValue;
    static const int f32_ks3 = tuning_knob("EXQ_FUSED_F32_KS3", 1);
    if (f32_ks3 != 0 && a.U > 32 && a.U <= 48) {
        // the one-token launch's split (16-lane slots over three waves), in
        // 6-wave workgroups: two row groups, at most two waves per SIMD, so
        // both tokens' activation slices fit the registers
        a.G = 16;
        a.KS = 3;
        return type == kTypeQ4_K ? launch_fused_fmt<FmtQ4KF32, 2, 1, 6, false, 0>(a, st)
                                 : launch_fused_fmt<FmtQ6KF32, 2, 1, 6, false, 0>(a, st);
    }
    return type == kTypeQ4_K ? launch_fused_fmt<FmtQ4KF32, 2, 1, 8, false, 0>(a, st)
                             : launch_fused_fmt<FmtQ6KF32, 2, 1, 8, false, 0>(a, st);
}

// nmat matrices of the same type and K, all applied to the same m tokens:
// f32 x quantized inside the kernel (x != null), or codes already quantized
// in the reference block layout (xq, token stride xq_stride).
namespace {
// pro: prologue (0, 1, 2) | 4 for a residual epilogue | 8 for gate/up
// pairs.  The instantiated one-token combinations are the layer's: RMSNorm
// (q/k/v, gate/up), residual (o), SiLU-mul with or without residual (down),
// gate/up pairs with or without RMSNorm.
template <class Fmt>
hipError_t dispatch_fused(const FusedArgs &a, bool stage, int pro, hipStream_t st) {
    switch (pro) {
        case 0: return launch_fused_nw<Fmt>(a, stage, st);
        case 1: return launch_fused_pro<Fmt, 1>(a, st);
        case 2: return launch_fused_pro<Fmt, 2>(a, st);
        case 4: return launch_fused_pro<Fmt, 4>(a, st);
        case 6: return launch_fused_pro<Fmt, 6>(a, st);
        case 8: return launch_fused_pro<Fmt, 8>(a, st);
        case 9: return launch_fused_pro<Fmt, 9>(a, st);
        default: return hipErrorInvalidValue;
    }
}
}  // namespace

// nmat matrices of the same type and K, all applied to the same m tokens:
// f32 x quantized inside the kernel (x != null), or codes already quantized
// in the reference block layout (xq, token stride xq_stride).  With a
// prologue (pro 1: x is RMSNorm-ed with nw and eps; pro 2: x is silu(x) * x2)
// or a residual (resid non-null: added to each output after its bias) x is
// staged and m must be 1 (gemv_fused_pro_supported); RMSNorm with a residual
// is not a layer's combination and is not instantiated.
hipError_t launch_gemv_fused_layer(int type, int nmat, const uint8_t *const *w, const int *n_out,
                                   const float *const *bias, const float *const *resid, float *const *out,
                                   size_t row_bytes, int K, int m, const float *x, const float *x2, const float *nw,
                                   float eps, int pro, const uint8_t *xq, size_t xq_stride, hipStream_t st) {
    if (nmat < 1 || nmat > kFusedMaxMats) return hipErrorInvalidValue;
    const bool pair = (pro & 8) != 0;
    pro &= 3;
    // pairs: w[0] / bias[0] gate, w[1] / bias[1] up, out[0] the product,
    // n_out[0] their common row count; the tiles run over gate's rows
    if (pair && (nmat != 2 || n_out[1] != n_out[0] || (resid != nullptr && (resid[0] || resid[1]))))
        return hipErrorInvalidValue;
    FusedArgs a{};
    a.nmat = pair ? 1 : nmat;
    for (int z = 0; z < nmat; ++z) {
        a.w[z] = w[z];
        a.n_out[z] = n_out[z];
        a.bias[z] = bias != nullptr ? bias[z] : nullptr;
        a.resid[z] = resid != nullptr ? resid[z] : nullptr;
        a.out[z] = out[z];
    }
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = m;
    a.x = x;
    a.xq = xq;
    a.xq_stride = xq_stride;
    a.x2 = x2;
    a.nw = nw;
    a.eps = eps;
    if ((x == nullptr) == (xq == nullptr)) return hipErrorInvalidValue;
    bool any_resid = false;
    for (int z = 0; z < nmat; ++z) any_resid = any_resid || a.resid[z] != nullptr;
    const int code = pro | (any_resid ? 4 : 0) | (pair ? 8 : 0);
    if (code != 0 && (x == nullptr || m != 1 || code == 5 || (pair && pro == 2) || (pro == 1 && nw == nullptr) ||
                      (pro == 2 && x2 == nullptr)))
        return hipErrorInvalidValue;
    // Q4_K rows at the decode lengths: the streaming kernel (one token: every
    // variant -- plain, prologues, residual, pairs, staged or Q8_K input;
    // two to four tokens: plain projections of staged tokens), and staged
    // tokens of Q6_K rows of 9728; its rows equal this kernel's bit for bit
    long long rows = 0;
    for (int z = 0; z < nmat; ++z) rows += n_out[z];
    if (gemv_stream_take(type, K, m, rows, nmat, w, code, x != nullptr))
        return launch_gemv_stream(type, nmat, w, n_out, bias, resid, out, K, m, x, xq, x2, nw, eps, pro, pair, st);
    a.nblk = q8_0_family(type) ? K / kQK8_0 : K / kQKK;
    a.U = q8_0_family(type) ? a.nblk : a.nblk * 4;
    // three waves per row: one-token K-quant launches (Q4_K, Q6_K)
    const bool with3 = fused_with3(type, m, x != nullptr);
    if (!pick_fused_shape(a.U, a.G, a.KS, with3)) return hipErrorInvalidValue;
    switch (type) {
        case kTypeQ8_0: return dispatch_fused<FmtQ80>(a, x != nullptr, code, st);
        case kTypeQ4_K: return dispatch_fused<FmtQ4K>(a, x != nullptr, code, st);
        case kTypeQ6_K: return dispatch_fused<FmtQ6K>(a, x != nullptr, code, st);
        case kTypeQ4_0:
        case kTypeQ5_0:
        case kTypeQ5_K: return code == 0 ? launch_gemv_fused_more(type, a, x != nullptr, st) : hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_fused(int type, int nmat, const uint8_t *const *w, const int *n_out,
                             const float *const *bias, float *const *out, size_t row_bytes, int K, int m,
                             const float *x, const uint8_t *xq, size_t xq_stride, hipStream_t st) {
    return launch_gemv_fused_layer(type, nmat, w, n_out, bias, nullptr, out, row_bytes, K, m, x, nullptr, nullptr,
                                   0.0f, 0, xq, xq_stride, st);
}

// True when the fused kernel runs (type, K) for one token with staging
// prologue pro (1 RMSNorm, 2 SiLU-mul): the RMSNorm needs the whole row in
// one staging round (8-wave workgroups: 8192 elements for the K-quants, 2048
// for Q8_0; the 16-wave row-split ones: 16384).
bool gemv_fused_pro_supported(int type, int K, int pro) {
    // prologues, residual epilogues and gate/up pairs: Q8_0, Q4_K, Q6_K rows
    if (type != kTypeQ8_0 && type != kTypeQ4_K && type != kTypeQ6_K) return false;
    if (!gemv_fused_supported(type, K, 1)) return false;
    const int U = type == kTypeQ8_0 ? K / kQK8_0 : (K / kQKK) * 4;
    int G = 64, KS = 1;
    if (!pick_fused_shape(U, G, KS, fused_with3(type, 1, true))) return false;
    if (pro != 1) return true;
    if (type == kTypeQ8_0) return K <= 8 * 64 * 4;
    return K <= (KS == 3 ? 12 : KS > 1 ? 16 : 8) * 64 * 16;
}
