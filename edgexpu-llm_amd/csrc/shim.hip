// libedgexpu_hip.so: the thin C-ABI between the C host side and the gfx950
// kernels.  Holds the per-process device state (one device, one stream, one
// growable workspace, device staging for host-pointer calls) and the sticky
// error, validates every argument before launching, and sequences the
// quantize -> GEMV / dequant kernels of the quantized-weight path.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "edgexpu_hip.h"

using namespace exq;

// kernels (quantize.hip, dequant.hip, gemv.hip, gemm.hip, gemm_kq.hip, gemm_g32.hip)
hipError_t launch_quantize_q8_0(const float *x, int m, int K, int ldx, uint8_t *packed, hipStream_t st);
hipError_t launch_quantize_q8_k(const float *x, int m, int K, int ldx, uint8_t *packed, hipStream_t st);
hipError_t launch_dequantize(const uint8_t *src, int type, unsigned long long n, float *dst, hipStream_t st);
hipError_t launch_dequantize_rows(const uint8_t *table, int type, long long n_rows, int n_embd, const int32_t *ids,
                                  int n_ids, float *out, int *bad, hipStream_t st);
hipError_t launch_gemv_q8(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                          size_t xq_stride, const float *bias, float *out, int ldo, hipStream_t st);
hipError_t launch_gemv_f32(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const float *xf,
                           const float *bias, float *out, int ldo, hipStream_t st);
hipError_t launch_gemv_plain(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const float *x,
                             int ldx, const float *bias, bool bias_f64, float *out, int ldo, hipStream_t st);
hipError_t launch_rmsnorm(const float *x, const float *w, float *out, int m, int n, float eps, hipStream_t st);
hipError_t launch_elementwise(const float *a, const float *b, float *out, long long n, int kind, hipStream_t st);
hipError_t launch_argmax_rows(const float *s, int m, int n, size_t lds, unsigned long long *partial, uint32_t *best,
                              hipStream_t st);
size_t gemm_q4k_pack_bytes(int m, int K);
size_t gemm_q4k_part_bytes(int m, int n_out, int K);
size_t gemm_q4k_counter_bytes();
hipError_t launch_q8k_pack_f32(const float *x, int m, int K, int ldx, uint8_t *pack, hipStream_t st);
hipError_t launch_q8k_pack_q8k(const uint8_t *xq, size_t xq_stride, int m, int K, uint8_t *pack, hipStream_t st);
hipError_t launch_gemm_q4k(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *pack,
                           float *part, unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st);
hipError_t launch_gemm_f16(const uint8_t *w, size_t row_bytes, int n_out, int K, int m, const uint8_t *xq,
                           size_t xq_stride, void *ws, const float *bias, float *out, int ldo, hipStream_t st);
size_t gemm_f16_workspace(int m, int n_out, int K);
bool gemm_q8_supported(int type, int n_out, int K, int m);
bool gemm_kq_supported(int type, int n_out, int K, int m);
size_t gemm_kq_repack_bytes(int n_out, int K);
size_t gemm_kq_part_bytes(int m, int n_out, int K);
hipError_t launch_kq_repack(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, uint8_t *rw,
                            hipStream_t st);
hipError_t launch_gemm_kq(int type, const uint8_t *rw, int n_out, int K, int m, const uint8_t *pack, float *part,
                          unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st);
bool gemm_g32_supported(int type, int n_out, int K, int m);
size_t gemm_g32_repack_bytes(int n_out, int K);
size_t gemm_g32_pack_bytes(int m, int K);
size_t gemm_g32_part_bytes(int m, int n_out, int K);
hipError_t launch_g32_repack(int type, const uint8_t *w, size_t row_bytes, int n_out, int K, uint8_t *rw,
                             hipStream_t st);
hipError_t launch_g32_pack(const float *x, const uint8_t *xq, size_t xq_stride, int m, int K, uint8_t *pack,
                           hipStream_t st);
hipError_t launch_gemm_g32(int type, const uint8_t *rw, int n_out, int K, int m, const uint8_t *pack, float *part,
                           unsigned *cnt, const float *bias, float *out, int ldo, hipStream_t st);
bool gemv_fused_supported(int type, int K, int m);
bool gemv_fused_f32_supported(int type, int K);
bool gemv_fused_pro_supported(int type, int K, int pro);
hipError_t launch_gemv_fused_layer(int type, int nmat, const uint8_t *const *w, const int *n_out,
                                   const float *const *bias, const float *const *resid, float *const *out,
                                   size_t row_bytes, int K, int m, const float *x, const float *x2, const float *nw,
                                   float eps, int pro, const uint8_t *xq, size_t xq_stride, hipStream_t st);
hipError_t launch_gemv_fused_f32(int type, const uint8_t *w, int n_out, const float *bias, float *out,
                                 size_t row_bytes, int K, const float *xf, hipStream_t st,
                                 unsigned long long *amax = nullptr, int *nparts = nullptr);
hipError_t launch_gemv_fused_f32_pair(int type, const uint8_t *w, int n_out, const float *bias, float *out,
                                      size_t row_bytes, int K, const float *xf, hipStream_t st);
hipError_t launch_gemv_fused_q8_0_argmax(const uint8_t *w, int n_out, const float *bias, float *out,
                                         size_t row_bytes, int K, const float *x, hipStream_t st,
                                         unsigned long long *amax, int *nparts);
hipError_t launch_sample_softmax(float *x, int n, float top_p, double u, uint32_t *out, void *ws, hipStream_t st);
size_t sample_workspace_bytes(int n);
hipError_t launch_div_scalar(float *io, long long n, float d, hipStream_t st);
hipError_t launch_argmax_finish(const unsigned long long *partial, int m, int nparts, int stride, uint32_t *best,
                                hipStream_t st);
hipError_t launch_gemv_fused(int type, int nmat, const uint8_t *const *w, const int *n_out, const float *const *bias,
                             float *const *out, size_t row_bytes, int K, int m, const float *x, const uint8_t *xq,
                             size_t xq_stride, hipStream_t st);

// gemv_stream.hip: the decode GEMV kernel choice for one-token Q4_K launches
namespace exq {
void set_gemv_stream_mode(int mode);
int gemv_stream_mode();
bool gemv_stream_take(int type, int K, int m, long long rows, int nmat, const uint8_t *const *w, int code,
                      bool staged);
}  // namespace exq

namespace {

constexpr int kGemvMaxTokens = 8;
constexpr int kFusedMaxTokens = 4;
// From 16 tokens the matrix-core GEMM reads each weight row once for all
// tokens; below that the GEMV reads it once per 8 tokens.  Measured at
// [14336 x 4096] Q4_K: GEMV 44 / 80 / 151 us at 8 / 16 / 32 tokens, GEMM
// 40 / 41 / 46 us at 16 / 32 / 64 ([4096 x 4096]: GEMV 18 / 31 / 55, GEMM
// 29 / 31 / 35).  Q5_K pays a weight repack per call: GEMV 31 / 55 us at 16 /
// 32 tokens against 47 / 48, so it switches at 32.
int gemm_min_tokens(uint32_t type) { return type == (uint32_t)kTypeQ5_K ? 32 : 16; }
// Rows up to this many elements quantize the activation inside the GEMV
// workgroups; longer rows quantize it once in its own launch (the in-kernel
// staging costs one load latency per 8192 elements per workgroup) ...
constexpr int kStageMaxK = 4096;
// ... except one token's Q8_K activation up to this many elements, which
// the 16-wave workgroups of the row-split GEMV quantize in one round.
constexpr int kStageMaxKWide = 16384;
constexpr int kArgmaxParts = 4096;  // per token: the two-pass argmax's 1024, or one key per wave of a logits launch

struct State {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;
    void *ws = nullptr;  // device workspace (quantized activations, sums, argmax partials)
    void *sws = nullptr;  // sampling workspace (segment sums, sort keys)
    size_t sws_cap = 0;
    size_t ws_cap = 0;
    void *dbuf = nullptr;  // device staging for host-pointer calls
    void *f16ws = nullptr;  // fp16 prefill GEMM workspace
    size_t f16ws_cap = 0;
    void *lws = nullptr;    // layer entry: prologue activation and pre-residual outputs
    size_t lws_cap = 0;
    int prefill_mode = 0;   // EDGEXPU_HIP_PREFILL_EXACT_INT8 / _F16
    void *gws = nullptr;    // exact prefill GEMM: activation pack
    size_t gws_cap = 0;
    size_t dbuf_cap = 0;
    int err = 0;
    char msg[512] = {0};
};

State g;

// Fixed device scratch of edgexpu_hip_logits_noalloc_dev: the quantized
// hidden vectors and the argmax partial keys of up to
// kGemvMaxTokens vectors of kScratchMaxEmbd elements (each GPU the library
// runs on holds its own copy until the process ends).  Host code never hands
// `scratch` itself to a kernel: its device address comes from
// hipGetSymbolAddress, once per device at init, into g_scratch_ptr.
constexpr int kScratchMaxEmbd = 16384;
constexpr size_t kScratchBytes =
    ((size_t)kGemvMaxTokens * (kScratchMaxEmbd / kQKK) * kBytesQ8_K + 255) / 256 * 256 +  // Q8_K (> Q8_0) codes
    (size_t)kGemvMaxTokens * kArgmaxParts * sizeof(unsigned long long);                  // argmax keys
static_assert(kScratchBytes <= 512 * 1024, "a modest fixed scratch");
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
void *g_scratch_ptr[kMaxDevices];

void set_error(int code, const char *fmt, ...) {
    if (g.err != 0) return;  // sticky: keep the first error
    g.err = code != 0 ? code : -1;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g.msg, sizeof(g.msg), fmt, ap);
    va_end(ap);
    fprintf(stderr, "edgexpu_hip: %s\n", g.msg);
}

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_error((int)e, "%s: %s", what, hipGetErrorString(e));
    return false;
}

bool ensure_init() {
    if (g.ready) return true;
    return edgexpu_hip_init(0) != 0;
}

// A NULL handle is HIP's default (null) stream, as everywhere in HIP: work then
// orders with the caller's other default-stream work.
hipStream_t pick_stream(void *s) { return (hipStream_t)s; }

// Every type of the reference's dispatcher (src/gguf_quant.c:69-108): the
// Q8_0 family and the K-quants through their integer dots, F16 and F32
// through the f32-activation dot.
bool plain_type(uint32_t t) { return t == (uint32_t)kTypeF16 || t == (uint32_t)kTypeF32; }
bool gpu_type(uint32_t t) { return q8_0_family((int)t) || k_family((int)t) || plain_type(t); }

size_t block_elems(uint32_t t) {
    return q8_0_family((int)t) ? (size_t)kQK8_0 : (k_family((int)t) ? (size_t)kQKK : (size_t)1);
}

size_t block_bytes(uint32_t t) {
    switch (t) {
        case kTypeQ8_0: return kBytesQ8_0;
        case kTypeQ4_0: return kBytesQ4_0;
        case kTypeQ5_0: return kBytesQ5_0;
        case kTypeQ4_K: return kBytesQ4_K;
        case kTypeQ5_K: return kBytesQ5_K;
        case kTypeQ6_K: return kBytesQ6_K;
        case kTypeF16: return 2;
        case kTypeF32: return 4;
        default: return 0;
    }
}

// The granule of n_in the products take: a block (F16 and F32 rows of any
// length: the tiled F16 kernel for multiples of 32, the plain kernel else).
size_t unit_elems(uint32_t t) { return block_elems(t); }

// The granule of n_embd a row gather takes: a block, or 4 plain values (the
// gathered rows are written with 16-byte stores).
size_t embed_unit(uint32_t t) { return plain_type(t) ? (size_t)4 : block_elems(t); }

// Bytes of one token's quantized activation: Q8_0 blocks for the Q8_0
// family, Q8_K blocks for the K-quants (src/cpu_kernel.c:577-631).
size_t act_bytes(uint32_t t, int K) {
    return q8_0_family((int)t) ? (size_t)(K / kQK8_0) * kBytesQ8_0 : (size_t)(K / kQKK) * kBytesQ8_K;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Tuning knobs: EXQ_FUSED=0 never quantizes inside the GEMV, 2 always does
// (where the kernel covers the shape), 1 (default) by row length;
// EXQ_GENERIC=1 sends every quantized-activation GEMV to the generic kernel.
bool stage_in_kernel(uint32_t type, int K, int m) {
    static const int mode = tuning_knob("EXQ_FUSED", 1);
    static const int generic = tuning_knob("EXQ_GENERIC", 0);
    if (mode == 0 || generic != 0 || !gemv_fused_supported((int)type, K, m)) return false;
    return mode == 2 || K <= kStageMaxK || (k_family((int)type) && m == 1 && K <= kStageMaxKWide);
}

bool split_gemv(uint32_t type, int K, int m) {
    static const int generic = tuning_knob("EXQ_GENERIC", 0);
    return generic == 0 && m <= kFusedMaxTokens && gemv_fused_supported((int)type, K, m);
}

// Device workspace grown on demand (freed only at shutdown).
void *workspace(size_t bytes) {
    if (bytes <= g.ws_cap) return g.ws;
    if (g.ws != nullptr) {
        // kernels on any stream may still read the old buffer
        if (!hip_ok(hipDeviceSynchronize(), "workspace sync")) return nullptr;
        (void)hipFree(g.ws);
        g.ws = nullptr;
        g.ws_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.ws, cap), "hipMalloc workspace")) return nullptr;
    g.ws_cap = cap;
    return g.ws;
}

void *devbuf(size_t bytes) {
    if (bytes <= g.dbuf_cap) return g.dbuf;
    if (g.dbuf != nullptr) {
        if (!hip_ok(hipDeviceSynchronize(), "staging sync")) return nullptr;
        (void)hipFree(g.dbuf);
        g.dbuf = nullptr;
        g.dbuf_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.dbuf, cap), "hipMalloc staging")) return nullptr;
    g.dbuf_cap = cap;
    return g.dbuf;
}

// Workspace of the fp16 prefill GEMM (fp16 activations, split-K partials),
// grown on demand.
// The layer entry's own workspace (separate from workspace(), which the
// projection paths it calls may grow).
void *layer_ws(size_t bytes) {
    if (bytes <= g.lws_cap) return g.lws;
    if (g.lws != nullptr) {
        if (!hip_ok(hipDeviceSynchronize(), "layer workspace sync")) return nullptr;
        (void)hipFree(g.lws);
        g.lws = nullptr;
        g.lws_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.lws, cap), "hipMalloc layer workspace")) return nullptr;
    g.lws_cap = cap;
    return g.lws;
}

void *sample_ws(size_t bytes) {
    if (bytes <= g.sws_cap) return g.sws;
    if (g.sws != nullptr) {
        if (!hip_ok(hipDeviceSynchronize(), "sample workspace sync")) return nullptr;
        (void)hipFree(g.sws);
        g.sws = nullptr;
        g.sws_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.sws, cap), "hipMalloc sample workspace")) return nullptr;
    g.sws_cap = cap;
    return g.sws;
}

void *f16ws(size_t bytes) {
    if (bytes <= g.f16ws_cap) return g.f16ws;
    if (g.f16ws != nullptr) {
        if (!hip_ok(hipDeviceSynchronize(), "f16 workspace sync")) return nullptr;
        (void)hipFree(g.f16ws);
        g.f16ws = nullptr;
        g.f16ws_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.f16ws, cap), "hipMalloc f16 workspace")) return nullptr;
    g.f16ws_cap = cap;
    return g.f16ws;
}

// Workspace of the exact prefill GEMM (the activation pack), grown on demand.
void *gemm_ws(size_t bytes) {
    if (bytes <= g.gws_cap) return g.gws;
    if (g.gws != nullptr) {
        if (!hip_ok(hipDeviceSynchronize(), "gemm workspace sync")) return nullptr;
        (void)hipFree(g.gws);
        g.gws = nullptr;
        g.gws_cap = 0;
    }
    size_t cap = align_up(bytes, (size_t)1 << 20);
    if (!hip_ok(hipMalloc(&g.gws, cap), "hipMalloc gemm workspace")) return nullptr;
    // the K-split arrival counters at its start are zero between launches
    // (each tile's last workgroup resets its own); cleared here once, outside
    // any stream work a caller may capture
    if (!hip_ok(hipMemset(g.gws, 0, gemm_q4k_counter_bytes()), "clear gemm counters")) return nullptr;
    g.gws_cap = cap;
    return g.gws;
}

// Formats with an exact matrix-core prefill GEMM: Q4_K straight from its
// blocks (gemm.hip), Q5_K and Q6_K over a per-call repack (gemm_kq.hip), and
// Q8_0 / Q4_0 / Q5_0 over a per-call repack against Q8_0 activations
// (gemm_g32.hip).  The GEMMs also need their weight pointers aligned: Q4_K
// rows are read as 16-byte vectors (and by the fp16 mode's GEMM likewise),
// the repacks read 2-byte scale words.  Blocks at other addresses (a GGUF
// data section may place a tensor at any offset its writer chose) take the
// GEMV path, which reads bytes at any alignment.
bool exact_gemm_type(uint32_t type, int nmat, const void *const *w, const int *n_out, int n_in, int m) {
    const uintptr_t need = type == (uint32_t)kTypeQ4_K ? 15u : 1u;
    for (int z = 0; z < nmat; ++z) {
        if (!(gemm_q8_supported((int)type, n_out[z], n_in, m) || gemm_kq_supported((int)type, n_out[z], n_in, m) ||
              gemm_g32_supported((int)type, n_out[z], n_in, m)))
            return false;
        if (((uintptr_t)w[z] & need) != 0) return false;
    }
    return true;
}

// Exact prefill GEMM of nmat matrices over one input: f32 activations
// (x != nullptr) or quantized blocks already in memory (xq: Q8_K for the
// K-quants, Q8_0 for the 32-element formats).  The activations are packed
// once into the GEMM's operand layout, then one launch per matrix (all but
// Q4_K: a repack of the matrix into the workspace, then the GEMM; the
// launches are stream-ordered, so one repack buffer serves every matrix).
bool run_gemm_exact(uint32_t type, int nmat, const void *const *w, const int *n_out, int n_in, int m, const float *x,
                    const uint8_t *xq, size_t xq_stride, const float *const *bias, float *const *out, const int *ldo,
                    hipStream_t st) {
    const bool g32 = q8_0_family((int)type);
    const bool kq = !g32 && type != (uint32_t)kTypeQ4_K;
    // workspace: arrival counters | activation pack | K-split partial tiles | repacked weights
    size_t part_bytes = 0, rw_bytes = 0;
    for (int z = 0; z < nmat; ++z) {
        const size_t pb = g32  ? gemm_g32_part_bytes(m, n_out[z], n_in)
                          : kq ? gemm_kq_part_bytes(m, n_out[z], n_in)
                               : gemm_q4k_part_bytes(m, n_out[z], n_in);
        part_bytes = pb > part_bytes ? pb : part_bytes;
        const size_t rb = g32 ? gemm_g32_repack_bytes(n_out[z], n_in) : kq ? gemm_kq_repack_bytes(n_out[z], n_in) : 0;
        rw_bytes = rb > rw_bytes ? rb : rw_bytes;
    }
    const size_t cnt_bytes = gemm_q4k_counter_bytes();
    const size_t pack_bytes =
        align_up(g32 ? gemm_g32_pack_bytes(m, n_in) : gemm_q4k_pack_bytes(m, n_in), (size_t)256);
    part_bytes = align_up(part_bytes, (size_t)256);
    uint8_t *ws = (uint8_t *)gemm_ws(cnt_bytes + pack_bytes + part_bytes + rw_bytes);
    if (ws == nullptr) return false;
    unsigned *cnt = (unsigned *)ws;
    uint8_t *pack = ws + cnt_bytes;
    float *part = part_bytes != 0 ? (float *)(pack + pack_bytes) : nullptr;
    uint8_t *rw = pack + pack_bytes + part_bytes;
    const hipError_t e = g32            ? launch_g32_pack(x, xq, xq_stride, m, n_in, pack, st)
                         : x != nullptr ? launch_q8k_pack_f32(x, m, n_in, n_in, pack, st)
                                        : launch_q8k_pack_q8k(xq, xq_stride, m, n_in, pack, st);
    if (!hip_ok(e, "pack activations")) return false;
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    for (int z = 0; z < nmat; ++z) {
        const float *bz = bias != nullptr ? bias[z] : nullptr;
        if (g32) {
            if (!hip_ok(launch_g32_repack((int)type, (const uint8_t *)w[z], rb, n_out[z], n_in, rw, st), "g32 repack") ||
                !hip_ok(launch_gemm_g32((int)type, rw, n_out[z], n_in, m, pack, part, cnt, bz, out[z], ldo[z], st),
                        "gemm_g32"))
                return false;
        } else if (kq) {
            if (!hip_ok(launch_kq_repack((int)type, (const uint8_t *)w[z], rb, n_out[z], n_in, rw, st), "kq repack") ||
                !hip_ok(launch_gemm_kq((int)type, rw, n_out[z], n_in, m, pack, part, cnt, bz, out[z], ldo[z], st),
                        "gemm_kq"))
                return false;
        } else if (!hip_ok(launch_gemm_q4k((const uint8_t *)w[z], rb, n_out[z], n_in, m, pack, part, cnt, bz, out[z],
                                           ldo[z], st),
                           "gemm_q4k")) {
            return false;
        }
    }
    return true;
}

bool use_exact_gemm(uint32_t type, int nmat, const void *const *w, const int *n_out, int n_in, int m) {
    return m >= gemm_min_tokens(type) && g.prefill_mode == EDGEXPU_HIP_PREFILL_EXACT_INT8 &&
           exact_gemm_type(type, nmat, w, n_out, n_in, m);
}

// Workspace carve-up for m tokens of K elements.
struct ActWs {
    uint8_t *xq;               // m * act_bytes   quantized activations
    unsigned long long *keys;  // m * 4096        argmax partials
};

// Byte sizes of the two parts, each a multiple of 256.
void act_ws_sizes(uint32_t type, int m, int K, size_t &qb, size_t &kb) {
    qb = align_up((size_t)m * act_bytes(type, K), 256);
    kb = align_up((size_t)m * kArgmaxParts * sizeof(unsigned long long), 256);
}

// The two parts carved out of base (256-byte aligned).
void act_ws_carve(uint32_t type, int m, int K, uint8_t *base, ActWs &a) {
    size_t qb, kb;
    act_ws_sizes(type, m, K, qb, kb);
    a.xq = base;
    a.keys = (unsigned long long *)(base + qb);
}

bool act_ws(uint32_t type, int m, int K, ActWs &a) {
    size_t qb, kb;
    act_ws_sizes(type, m, K, qb, kb);
    uint8_t *base = (uint8_t *)workspace(qb + kb);
    if (base == nullptr) return false;
    act_ws_carve(type, m, K, base, a);
    return true;
}

bool check_linear_args(const void *out, const void *x, const void *w, uint32_t type, int m, int n_out, int n_in,
                       const char *who) {
    if (out == nullptr || x == nullptr || w == nullptr || m <= 0 || n_out <= 0 || n_in <= 0) {
        set_error(-2, "%s: null buffer or non-positive size (m=%d n_out=%d n_in=%d)", who, m, n_out, n_in);
        return false;
    }
    if (!gpu_type(type)) {
        set_error(-3, "%s: GGUF type %u is not supported (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)", who, type);
        return false;
    }
    if ((size_t)n_in % unit_elems(type) != 0) {
        set_error(-2, "%s: n_in=%d is not a multiple of %zu for type %u", who, n_in, unit_elems(type), type);
        return false;
    }
    return true;
}

// Device blocks of the formats whose blocks are an even but not a 4-byte
// multiple long (Q8_0 34, Q4_0 18, Q5_0 22, Q6_K 210 bytes) are read as
// aligned 32-bit words joined by byte shifts that assume an even block
// address, so their device pointers must be even.  File-backed weights always
// are: GGUF places tensors at multiples of the file's alignment (8 or more)
// after a data section that starts at a multiple of 32 (src/gguf.c:595), and
// device allocations start at 256.  Weights given as host memory are copied
// to the device first and are not affected.
bool check_weight_align(const void *w, uint32_t type, const char *who) {
    if (((uintptr_t)w & 1u) != 0 && (q8_0_family((int)type) || type == (uint32_t)kTypeQ6_K)) {
        set_error(-2, "%s: type-%u blocks must start at an even device address (got %p)", who, type, w);
        return false;
    }
    return true;
}

// f32-activation products (F16 and F32 rows in the batch driver; every type
// in the per-row f32 dot and the logits of the non-Q8_0 formats): at most
// kGemvMaxTokens tokens per launch of the generic kernels, or the fused
// kernel one token at a time for the K-quant formats it covers.  bias_f64: F32 rows add the
// bias in double before the final rounding (the one-token linear of
// src/cpu_kernel.c:566-569, 462-523).
bool run_f32_product(uint32_t type, const void *w, int n_out, int n_in, int m, const float *x, const float *bias,
                     float *out, int ldo, hipStream_t st, bool bias_f64 = false) {
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    if (type == (uint32_t)kTypeF32 || (type == (uint32_t)kTypeF16 && n_in % 32 != 0)) {
        for (int t0 = 0; t0 < m; t0 += kGemvMaxTokens) {
            const int mt = m - t0 < kGemvMaxTokens ? m - t0 : kGemvMaxTokens;
            if (!hip_ok(launch_gemv_plain((int)type, (const uint8_t *)w, rb, n_out, n_in, mt, x + (size_t)t0 * n_in,
                                          n_in, bias, bias_f64, out + (size_t)t0 * ldo, ldo, st),
                        "gemv_plain"))
                return false;
        }
        return true;
    }
    if (k_family((int)type) && ldo == n_out && gemv_fused_f32_supported((int)type, n_in)) {
        // tokens in pairs where the format has the two-token launch (the
        // weights read once per pair), else one at a time
        const bool pairs = type == (uint32_t)kTypeQ4_K || type == (uint32_t)kTypeQ6_K;
        for (int t = 0; t < m;) {
            const int mt = pairs && m - t >= 2 ? 2 : 1;
            const float *xt = x + (size_t)t * n_in;
            const hipError_t e =
                mt == 2 ? launch_gemv_fused_f32_pair((int)type, (const uint8_t *)w, n_out, bias, out + (size_t)t * ldo,
                                                     rb, n_in, xt, st)
                        : launch_gemv_fused_f32((int)type, (const uint8_t *)w, n_out, bias, out + (size_t)t * ldo, rb,
                                                n_in, xt, st);
            if (!hip_ok(e, "gemv_f32 fused")) return false;
            t += mt;
        }
        return true;
    }
    for (int t0 = 0; t0 < m; t0 += kGemvMaxTokens) {
        const int mt = m - t0 < kGemvMaxTokens ? m - t0 : kGemvMaxTokens;
        if (!hip_ok(launch_gemv_f32((int)type, (const uint8_t *)w, rb, n_out, n_in, mt, x + (size_t)t0 * n_in, bias,
                                    out + (size_t)t0 * ldo, ldo, st),
                    "gemv_f32"))
            return false;
    }
    return true;
}

// GEMV (m <= 8 per launch) or MFMA GEMM over already-quantized activations.
bool run_q8_product(uint32_t type, const void *w, int n_out, int n_in, int m, const uint8_t *xq, const float *bias,
                    float *out, int ldo, hipStream_t st) {
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    const size_t ab = act_bytes(type, n_in);
    if (m >= gemm_min_tokens(type) && exact_gemm_type(type, 1, &w, &n_out, n_in, m)) {
        if (g.prefill_mode == EDGEXPU_HIP_PREFILL_F16 && gemm_q8_supported((int)type, n_out, n_in, m)) {
            void *ws = f16ws(gemm_f16_workspace(m, n_out, n_in));
            if (ws == nullptr) return false;
            return hip_ok(launch_gemm_f16((const uint8_t *)w, rb, n_out, n_in, m, xq, ab, ws, bias, out, ldo, st),
                          "gemm_f16");
        }
        return run_gemm_exact(type, 1, &w, &n_out, n_in, m, nullptr, xq, ab, &bias, &out, &ldo, st);
    }
    if (ldo == n_out && split_gemv(type, n_in, m)) {
        const uint8_t *wp = (const uint8_t *)w;
        return hip_ok(launch_gemv_fused((int)type, 1, &wp, &n_out, &bias, &out, rb, n_in, m, nullptr, xq, ab, st),
                      "gemv_split");
    }
    for (int t0 = 0; t0 < m; t0 += kGemvMaxTokens) {
        const int mt = m - t0 < kGemvMaxTokens ? m - t0 : kGemvMaxTokens;
        if (!hip_ok(launch_gemv_q8((int)type, (const uint8_t *)w, rb, n_out, n_in, mt, xq + (size_t)t0 * ab, ab,
                                   bias, out + (size_t)t0 * ldo, ldo, st),
                    "gemv_q8"))
            return false;
    }
    return true;
}

// nmat products over one input x (f32, [m][n_in]): either one launch that
// quantizes x inside its workgroups, or one quantize launch followed by one
// launch over all nmat matrices (m <= 4) or per-matrix products.
bool run_linear_group(uint32_t type, int nmat, const void *const *w, const int *n_out, const float *const *bias,
                      float *const *out, const float *x, int m, int n_in, hipStream_t st) {
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    if (plain_type(type)) {
        // src/cpu_kernel.c:632-641: rows with neither activation quantizer
        // take the f32-activation row dot, out = bias + dot per token; F32
        // at one token is edgexpu_cpu_linear (src/cpu_kernel.c:566-569),
        // whose sum starts at the bias in double
        const bool f64 = type == (uint32_t)kTypeF32 && m == 1;
        for (int z = 0; z < nmat; ++z)
            if (!run_f32_product(type, w[z], n_out[z], n_in, m, x, bias != nullptr ? bias[z] : nullptr,
                                 out[z], n_out[z], st, f64))
                return false;
        return true;
    }
    // two to four tokens of the rows the streaming GEMV takes are quantized
    // inside its workgroups too; other long rows quantize once in their own
    // launch
    long long rows = 0;
    for (int z = 0; z < nmat; ++z) rows += n_out[z];
    const bool stream_staged =
        m > 1 && m <= kFusedMaxTokens &&
        gemv_stream_take((int)type, n_in, m, rows, nmat, (const uint8_t *const *)w, 0, true);
    if (stream_staged || stage_in_kernel(type, n_in, m)) {
        return hip_ok(launch_gemv_fused((int)type, nmat, (const uint8_t *const *)w, n_out, bias, out, rb, n_in, m, x,
                                        nullptr, 0, st),
                      "gemv_fused");
    }
    if (use_exact_gemm(type, nmat, w, n_out, n_in, m))  // the GEMM quantizes x into its own operand layout
        return run_gemm_exact(type, nmat, w, n_out, n_in, m, x, nullptr, 0, bias, out, n_out, st);
    ActWs a;
    if (!act_ws(type, m, n_in, a)) return false;
    const hipError_t e = q8_0_family((int)type) ? launch_quantize_q8_0(x, m, n_in, n_in, a.xq, st)
                                                : launch_quantize_q8_k(x, m, n_in, n_in, a.xq, st);
    if (!hip_ok(e, "quantize activations")) return false;
    if (split_gemv(type, n_in, m) && m < gemm_min_tokens(type)) {
        return hip_ok(launch_gemv_fused((int)type, nmat, (const uint8_t *const *)w, n_out, bias, out, rb, n_in, m,
                                        nullptr, a.xq, act_bytes(type, n_in), st),
                      "gemv_split");
    }
    for (int z = 0; z < nmat; ++z) {
        if (!run_q8_product(type, w[z], n_out[z], n_in, m, a.xq, bias != nullptr ? bias[z] : nullptr, out[z],
                            n_out[z], st))
            return false;
    }
    return true;
}

}  // namespace

struct edgexpu_hip_weight {
    void *data;
    float *bias;
    uint32_t type;
    int n_out;
    int n_in;
    bool owned;
};

extern "C" {

int edgexpu_hip_init(int device) {
    if (g.ready) {
        if (device == g.device) return 1;
        set_error(-4, "edgexpu_hip_init: already initialised on device %d", g.device);
        return 0;
    }
    int n = 0;
    if (!hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount")) return 0;
    if (device < 0 || device >= n) {
        set_error(-4, "edgexpu_hip_init: device %d out of range (%d devices)", device, n);
        return 0;
    }
    if (!hip_ok(hipSetDevice(device), "hipSetDevice")) return 0;
    if (device < kMaxDevices && g_scratch_ptr[device] == nullptr) {
        void *p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch address")) return 0;
        g_scratch_ptr[device] = p;
    }
    if (!hip_ok(hipStreamCreate(&g.stream), "hipStreamCreate")) return 0;
    g.device = device;
    g.ready = true;
    return 1;
}

void edgexpu_hip_shutdown(void) {
    if (!g.ready) return;
    (void)hipDeviceSynchronize();
    if (g.ws) (void)hipFree(g.ws);
    if (g.dbuf) (void)hipFree(g.dbuf);
    if (g.f16ws) (void)hipFree(g.f16ws);
    if (g.sws) (void)hipFree(g.sws);
    if (g.lws) (void)hipFree(g.lws);
    if (g.gws) (void)hipFree(g.gws);
    (void)hipStreamDestroy(g.stream);
    const int err = g.err;
    char msg[sizeof(g.msg)];
    memcpy(msg, g.msg, sizeof(msg));
    g = State();
    g.err = err;
    memcpy(g.msg, msg, sizeof(msg));
}

int edgexpu_hip_last_error(char *buf, size_t size) {
    if (buf != nullptr && size > 0) snprintf(buf, size, "%s", g.err ? g.msg : "");
    return g.err;
}

void edgexpu_hip_clear_error(void) {
    g.err = 0;
    g.msg[0] = 0;
}

int edgexpu_hip_supports_type(uint32_t type) { return gpu_type(type) ? 1 : 0; }

int edgexpu_hip_set_prefill_mode(int mode) {
    if (mode != EDGEXPU_HIP_PREFILL_EXACT_INT8 && mode != EDGEXPU_HIP_PREFILL_F16) {
        set_error(-2, "set_prefill_mode: unknown mode %d", mode);
        return 0;
    }
    g.prefill_mode = mode;
    return 1;
}

int edgexpu_hip_prefill_mode(void) { return g.prefill_mode; }

int edgexpu_hip_set_gemv_mode(int mode) {
    if (mode != EDGEXPU_HIP_GEMV_AUTO && mode != EDGEXPU_HIP_GEMV_FUSED && mode != EDGEXPU_HIP_GEMV_STREAM) {
        set_error(-2, "set_gemv_mode: unknown mode %d", mode);
        return 0;
    }
    set_gemv_stream_mode(mode);
    return 1;
}

int edgexpu_hip_gemv_mode(void) { return gemv_stream_mode(); }

int edgexpu_hip_synchronize(void) {
    if (!ensure_init()) return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "hipStreamSynchronize") ? 1 : 0;
}

void *edgexpu_hip_stream(void) {
    if (!ensure_init()) return nullptr;
    return (void *)g.stream;
}

size_t edgexpu_hip_row_bytes(uint32_t type, int n_in) {
    if (!gpu_type(type) || n_in <= 0 || (size_t)n_in % block_elems(type) != 0) return 0;
    return (size_t)n_in / block_elems(type) * block_bytes(type);
}

// ------------------------------------------------------------------ weights

edgexpu_hip_weight *edgexpu_hip_weight_upload(const uint8_t *blocks, uint32_t type, int n_out, int n_in,
                                              const float *bias) {
    if (!ensure_init()) return nullptr;
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    if (blocks == nullptr || n_out <= 0 || rb == 0) {
        set_error(-2, "edgexpu_hip_weight_upload: bad arguments (type=%u n_out=%d n_in=%d)", type, n_out, n_in);
        return nullptr;
    }
    edgexpu_hip_weight *w = (edgexpu_hip_weight *)calloc(1, sizeof(edgexpu_hip_weight));
    if (w == nullptr) {
        set_error(-5, "edgexpu_hip_weight_upload: out of host memory");
        return nullptr;
    }
    const size_t nbytes = rb * (size_t)n_out;
    if (!hip_ok(hipMalloc(&w->data, align_up(nbytes, 256)), "hipMalloc weight")) {
        free(w);
        return nullptr;
    }
    if (!hip_ok(hipMemcpy(w->data, blocks, nbytes, hipMemcpyHostToDevice), "upload weight")) {
        (void)hipFree(w->data);
        free(w);
        return nullptr;
    }
    if (bias != nullptr) {
        if (!hip_ok(hipMalloc((void **)&w->bias, (size_t)n_out * sizeof(float)), "hipMalloc bias") ||
            !hip_ok(hipMemcpy(w->bias, bias, (size_t)n_out * sizeof(float), hipMemcpyHostToDevice), "upload bias")) {
            if (w->bias) (void)hipFree(w->bias);
            (void)hipFree(w->data);
            free(w);
            return nullptr;
        }
    }
    w->type = type;
    w->n_out = n_out;
    w->n_in = n_in;
    w->owned = true;
    return w;
}

void *edgexpu_hip_upload_bytes(const void *host, size_t n) {
    if (!ensure_init()) return nullptr;
    if (host == nullptr || n == 0) {
        set_error(-2, "edgexpu_hip_upload_bytes: bad arguments (host=%p n=%zu)", host, n);
        return nullptr;
    }
    void *dev = nullptr;
    if (!hip_ok(hipMalloc(&dev, align_up(n, 256)), "hipMalloc upload")) return nullptr;
    if (!hip_ok(hipMemcpy(dev, host, n, hipMemcpyHostToDevice), "upload bytes")) {
        (void)hipFree(dev);
        return nullptr;
    }
    return dev;
}

int edgexpu_hip_download_bytes(void *host, const void *dev, size_t n) {
    if (!ensure_init()) return 0;
    if (host == nullptr || dev == nullptr) {
        set_error(-2, "edgexpu_hip_download_bytes: bad arguments");
        return 0;
    }
    return hip_ok(hipMemcpy(host, dev, n, hipMemcpyDeviceToHost), "download bytes") ? 1 : 0;
}

void edgexpu_hip_free_bytes(void *dev) {
    if (dev != nullptr) (void)hipFree(dev);
}

edgexpu_hip_weight *edgexpu_hip_weight_wrap(const void *dev_blocks, uint32_t type, int n_out, int n_in,
                                            const float *dev_bias) {
    if (dev_blocks == nullptr || n_out <= 0 || edgexpu_hip_row_bytes(type, n_in) == 0) {
        set_error(-2, "edgexpu_hip_weight_wrap: bad arguments (type=%u n_out=%d n_in=%d)", type, n_out, n_in);
        return nullptr;
    }
    edgexpu_hip_weight *w = (edgexpu_hip_weight *)calloc(1, sizeof(edgexpu_hip_weight));
    if (w == nullptr) {
        set_error(-5, "edgexpu_hip_weight_wrap: out of host memory");
        return nullptr;
    }
    w->data = (void *)dev_blocks;
    w->bias = (float *)dev_bias;
    w->type = type;
    w->n_out = n_out;
    w->n_in = n_in;
    w->owned = false;
    return w;
}

void edgexpu_hip_weight_free(edgexpu_hip_weight *w) {
    if (w == nullptr) return;
    if (w->owned) {
        if (g.ready) (void)hipDeviceSynchronize();
        (void)hipFree(w->data);
        if (w->bias) (void)hipFree(w->bias);
    }
    free(w);
}

const void *edgexpu_hip_weight_data(const edgexpu_hip_weight *w) { return w ? w->data : nullptr; }
uint32_t edgexpu_hip_weight_type(const edgexpu_hip_weight *w) { return w ? w->type : 0u; }
int edgexpu_hip_weight_n_out(const edgexpu_hip_weight *w) { return w ? w->n_out : 0; }
int edgexpu_hip_weight_n_in(const edgexpu_hip_weight *w) { return w ? w->n_in : 0; }

// ------------------------------------------------------------ device entries

int edgexpu_hip_linear_quant_batch_dev(float *out, const float *x, const void *w, uint32_t type, const float *bias,
                                       int m, int n_out, int n_in, void *stream) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(out, x, w, type, m, n_out, n_in, "linear_quant_batch") ||
        !check_weight_align(w, type, "linear_quant_batch"))
        return 0;
    if (!aligned16(x)) {
        set_error(-2, "linear_quant_batch: x must be 16-byte aligned");
        return 0;
    }
    const void *wp = w;
    return run_linear_group(type, 1, &wp, &n_out, &bias, &out, x, m, n_in, pick_stream(stream)) ? 1 : 0;
}

int edgexpu_hip_linear_quant_group_dev(int nmat, float *const *out, const float *x, const void *const *w,
                                       uint32_t type, const float *const *bias, const int *n_out, int m, int n_in,
                                       void *stream) {
    if (!ensure_init()) return 0;
    if (nmat < 1 || nmat > 4 || out == nullptr || w == nullptr || n_out == nullptr) {
        set_error(-2, "linear_quant_group: nmat must be 1..4 with out, w and n_out arrays");
        return 0;
    }
    for (int z = 0; z < nmat; ++z) {
        if (!check_linear_args(out[z], x, w[z], type, m, n_out[z], n_in, "linear_quant_group") ||
            !check_weight_align(w[z], type, "linear_quant_group"))
            return 0;
    }
    if (!aligned16(x)) {
        set_error(-2, "linear_quant_group: x must be 16-byte aligned");
        return 0;
    }
    return run_linear_group(type, nmat, w, n_out, bias, out, x, m, n_in, pick_stream(stream)) ? 1 : 0;
}

int edgexpu_hip_layer_linear_dev(int nmat, float *const *out, const float *x, const float *x2,
                                 const float *norm_weight, float eps, const void *const *w, uint32_t type,
                                 const float *const *bias, const float *const *residual, const int *n_out, int m,
                                 int n_in, void *stream) {
    if (!ensure_init()) return 0;
    if (nmat < 1 || nmat > 4 || out == nullptr || w == nullptr || n_out == nullptr) {
        set_error(-2, "layer_linear: nmat must be 1..4 with out, w and n_out arrays");
        return 0;
    }
    if (x2 != nullptr && norm_weight != nullptr) {
        set_error(-2, "layer_linear: give norm_weight (RMSNorm) or x2 (SiLU-mul), not both");
        return 0;
    }
    for (int z = 0; z < nmat; ++z) {
        if (!check_linear_args(out[z], x, w[z], type, m, n_out[z], n_in, "layer_linear") ||
            !check_weight_align(w[z], type, "layer_linear"))
            return 0;
    }
    if (!aligned16(x) || (x2 != nullptr && !aligned16(x2)) || (norm_weight != nullptr && !aligned16(norm_weight))) {
        set_error(-2, "layer_linear: x, x2 and norm_weight must be 16-byte aligned");
        return 0;
    }
    const int pro = norm_weight != nullptr ? 1 : (x2 != nullptr ? 2 : 0);
    hipStream_t st = pick_stream(stream);
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    bool any_resid = false;
    size_t res_floats = 0;
    for (int z = 0; z < nmat; ++z)
        if (residual != nullptr && residual[z] != nullptr) {
            any_resid = true;
            res_floats += align_up((size_t)m * n_out[z], 64);
        }
    // one launch: the prologue in the GEMV's staging, the residual in its
    // store (one token; without either, any token count the kernel covers)
    const bool plain = pro == 0 && !any_resid;
    const bool one_token = m == 1 && !(pro == 1 && any_resid) && gemv_fused_pro_supported((int)type, n_in, pro);
    if (stage_in_kernel(type, n_in, m) && (plain || one_token))
        return hip_ok(launch_gemv_fused_layer((int)type, nmat, (const uint8_t *const *)w, n_out, bias, residual, out,
                                              rb, n_in, m, x, x2, norm_weight, eps, pro, nullptr, 0, st),
                      "layer_linear fused")
                   ? 1
                   : 0;
    // otherwise the same arithmetic in steps: prologue kernel, projection,
    // residual add (the projection writes to the workspace first, so out may
    // be the residual)
    const size_t act_floats = pro != 0 ? align_up((size_t)m * n_in, 64) : 0;
    float *base = (float *)layer_ws((act_floats + res_floats) * sizeof(float) + 256);
    if (base == nullptr) return 0;
    const float *act = x;
    if (pro == 1) {
        if (!hip_ok(launch_rmsnorm(x, norm_weight, base, m, n_in, eps, st), "layer_linear rmsnorm")) return 0;
        act = base;
    } else if (pro == 2) {
        if (!hip_ok(launch_elementwise(x, x2, base, (long long)m * n_in, 3, st), "layer_linear silu_mul")) return 0;
        act = base;
    }
    float *outs[4];
    float *tmp = base + act_floats;
    for (int z = 0; z < nmat; ++z) {
        if (residual != nullptr && residual[z] != nullptr) {
            outs[z] = tmp;
            tmp += align_up((size_t)m * n_out[z], 64);
        } else {
            outs[z] = out[z];
        }
    }
    if (!run_linear_group(type, nmat, w, n_out, bias, outs, act, m, n_in, st)) return 0;
    if (any_resid)
        for (int z = 0; z < nmat; ++z)
            if (residual[z] != nullptr &&
                !hip_ok(launch_elementwise(residual[z], outs[z], out[z], (long long)m * n_out[z], 2, st),
                        "layer_linear residual"))
                return 0;
    return 1;
}

int edgexpu_hip_gate_up_silu_dev(float *act, const float *x, const float *norm_weight, float eps, const void *w_gate,
                                 const void *w_up, uint32_t type, const float *b_gate, const float *b_up, int m,
                                 int n_ff, int n_in, void *stream) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(act, x, w_gate, type, m, n_ff, n_in, "gate_up_silu") ||
        !check_linear_args(act, x, w_up, type, m, n_ff, n_in, "gate_up_silu") ||
        !check_weight_align(w_gate, type, "gate_up_silu") || !check_weight_align(w_up, type, "gate_up_silu"))
        return 0;
    if (!aligned16(x) || (norm_weight != nullptr && !aligned16(norm_weight))) {
        set_error(-2, "gate_up_silu: x and norm_weight must be 16-byte aligned");
        return 0;
    }
    hipStream_t st = pick_stream(stream);
    const int pro = norm_weight != nullptr ? 1 : 0;
    const size_t rb = edgexpu_hip_row_bytes(type, n_in);
    const void *wg[2] = {w_gate, w_up};
    const float *bg[2] = {b_gate, b_up};
    const int nn[2] = {n_ff, n_ff};
    // one launch: gate row j and up row j in the same wave, silu(gate) * up
    // from the store
    if (m == 1 && stage_in_kernel(type, n_in, 1) && gemv_fused_pro_supported((int)type, n_in, pro)) {
        float *outs[2] = {act, act};
        return hip_ok(launch_gemv_fused_layer((int)type, 2, (const uint8_t *const *)wg, nn, bg, nullptr, outs, rb,
                                              n_in, 1, x, nullptr, norm_weight, eps, pro | 8, nullptr, 0, st),
                      "gate_up_silu fused")
                   ? 1
                   : 0;
    }
    // otherwise: the RMSNorm, gate and up into one sizing of the layer
    // workspace (nothing below grows it), then silu * up
    const size_t nf = align_up((size_t)m * n_ff, 64), ni = pro != 0 ? align_up((size_t)m * n_in, 64) : 0;
    float *base = (float *)layer_ws((2 * nf + ni) * sizeof(float) + 256);
    if (base == nullptr) return 0;
    const float *a_in = x;
    if (pro != 0) {
        if (!hip_ok(launch_rmsnorm(x, norm_weight, base + 2 * nf, m, n_in, eps, st), "gate_up_silu rmsnorm")) return 0;
        a_in = base + 2 * nf;
    }
    float *outs[2] = {base, base + nf};
    if (!run_linear_group(type, 2, wg, nn, bg, outs, a_in, m, n_in, st)) return 0;
    return hip_ok(launch_elementwise(outs[0], outs[1], act, (long long)m * n_ff, 3, st), "gate_up_silu silu_mul") ? 1
                                                                                                                   : 0;
}

int edgexpu_hip_gemv_q8_dev(float *out, const uint8_t *xq, const void *w, uint32_t type, const float *bias, int m,
                            int n_out, int n_in, void *stream) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(out, xq, w, type, m, n_out, n_in, "gemv_q8") || !check_weight_align(w, type, "gemv_q8"))
        return 0;
    if (plain_type(type)) {
        set_error(-3, "gemv_q8: F16 and F32 rows have no quantized-activation dot (src/gguf_dot_q8.c:414-434)");
        return 0;
    }
    // the block scale heads every Q8_K (f32) / Q8_0 (f16) block
    const bool q80 = q8_0_family((int)type);
    if (((uintptr_t)xq & (q80 ? 1u : 3u)) != 0) {
        set_error(-2, "gemv_q8: xq must be %d-byte aligned", q80 ? 2 : 4);
        return 0;
    }
    return run_q8_product(type, w, n_out, n_in, m, xq, bias, out, n_out, pick_stream(stream)) ? 1 : 0;
}

}  // extern "C"

namespace {

bool check_logits_args(float *scores, const float *hidden, const void *w, uint32_t type, int m, int vocab,
                       int n_embd, int chunk_rows, const char *who) {
    if (!check_linear_args(scores, hidden, w, type, m, vocab, n_embd, who) || !check_weight_align(w, type, who))
        return false;
    if (m > kGemvMaxTokens) {
        set_error(-2, "%s: at most %d hidden vectors per call (m=%d)", who, kGemvMaxTokens, m);
        return false;
    }
    if (!aligned16(hidden)) {
        set_error(-2, "%s: hidden must be 16-byte aligned", who);
        return false;
    }
    if (chunk_rows < 0) {
        set_error(-2, "%s: chunk_rows must be >= 0 (got %d)", who, chunk_rows);
        return false;
    }
    return true;
}

// The logits product and greedy argmax over scratch `a` (quantized hidden
// vectors, 16-element sums, argmax partial keys), every part of which the
// kernels write before they read it.
bool logits_run(float *scores, uint32_t *best_dev, const float *hidden, const void *w, uint32_t type,
                const float *bias, int m, int vocab, int n_embd, hipStream_t st, const ActWs &a) {
    const size_t rb = edgexpu_hip_row_bytes(type, n_embd);
    // The reference walks the rows in chunks of chunk_rows (its host-memory
    // budget, src/native.c:2262-2274); every row's score is independent of
    // the chunking, so one launch covers all chunks in row order.
    if (q8_0_family((int)type)) {
        // src/native.c:2317-2319: the Q8_0 family scores rows against the
        // Q8_0-quantized hidden vector.  Fused launches of up to 4 hidden
        // vectors quantize them inside each workgroup (the same quantizer; a
        // row's score does not depend on how many vectors share the launch,
        // as in the reference's per-token loop); one vector of Q8_0 rows
        // also keeps the argmax epilogue's keys, reduced by one small launch.
        if (stage_in_kernel(type, n_embd, m < kFusedMaxTokens ? m : kFusedMaxTokens)) {
            const uint8_t *wp = (const uint8_t *)w;
            if (m == 1 && best_dev != nullptr && type == (uint32_t)kTypeQ8_0) {
                int nparts = 0;
                if (!hip_ok(launch_gemv_fused_q8_0_argmax(wp, vocab, bias, scores, rb, n_embd, hidden, st, a.keys,
                                                          &nparts),
                            "logits gemv + argmax"))
                    return false;
                return hip_ok(launch_argmax_finish(a.keys, 1, nparts, kArgmaxParts, best_dev, st), "argmax");
            }
            for (int t = 0; t < m; t += kFusedMaxTokens) {
                const int mt = m - t < kFusedMaxTokens ? m - t : kFusedMaxTokens;
                float *out = scores + (size_t)t * vocab;
                if (!hip_ok(launch_gemv_fused((int)type, 1, &wp, &vocab, &bias, &out, rb, n_embd, mt,
                                              hidden + (size_t)t * n_embd, nullptr, 0, st),
                            "logits gemv"))
                    return false;
            }
        } else {
            if (!hip_ok(launch_quantize_q8_0(hidden, m, n_embd, n_embd, a.xq, st), "quantize_q8_0")) return false;
            if (!hip_ok(launch_gemv_q8((int)type, (const uint8_t *)w, rb, vocab, n_embd, m, a.xq,
                                       act_bytes(type, n_embd), bias, scores, vocab, st),
                        "logits gemv"))
                return false;
        }
    } else {
        // the other formats use the f32-activation dots (src/native.c:445-462);
        // K-quant rows: one hidden vector in a launch (the streaming kernel for
        // Q4_K rows of 4096 and Q6_K rows of 2560 at 16-byte addresses, the
        // fused one otherwise, same words) that also keeps each workgroup's
        // greedy-argmax key (one small launch then reduces those keys instead
        // of re-reading the scores); several in launches of two (the weights
        // read once per pair), then the argmax over the scores.  A row's score
        // does not depend on m, as in the reference's per-token loop.
        if (m == 1 && best_dev != nullptr && k_family((int)type) && gemv_fused_f32_supported((int)type, n_embd)) {
            int nparts = 0;
            for (int t = 0; t < m; ++t) {
                const hipError_t e = launch_gemv_fused_f32(
                    (int)type, (const uint8_t *)w, vocab, bias, scores + (size_t)t * vocab, rb, n_embd,
                    hidden + (size_t)t * n_embd, st, a.keys + (size_t)t * kArgmaxParts, &nparts);
                if (!hip_ok(e, "logits gemv + argmax")) return false;
            }
            return hip_ok(launch_argmax_finish(a.keys, m, nparts, kArgmaxParts, best_dev, st), "argmax");
        }
        if (!run_f32_product(type, w, vocab, n_embd, m, hidden, bias, scores, vocab, st))
            return false;
    }
    if (best_dev != nullptr &&
        !hip_ok(launch_argmax_rows(scores, m, vocab, (size_t)vocab, a.keys, best_dev, st), "argmax"))
        return false;
    return true;
}

}  // namespace

extern "C" {

int edgexpu_hip_logits_dev(float *scores, uint32_t *best_dev, const float *hidden, const void *w, uint32_t type,
                           const float *bias, int m, int vocab, int n_embd, int chunk_rows, void *stream) {
    if (!ensure_init()) return 0;
    if (!check_logits_args(scores, hidden, w, type, m, vocab, n_embd, chunk_rows, "logits")) return 0;
    ActWs a;
    if (!act_ws(type, m, n_embd, a)) return 0;
    return logits_run(scores, best_dev, hidden, w, type, bias, m, vocab, n_embd, pick_stream(stream), a) ? 1 : 0;
}

int edgexpu_hip_logits_noalloc_dev(float *scores, uint32_t *best_dev, const float *hidden, const void *w,
                                   uint32_t type, const float *bias, int m, int vocab, int n_embd, int chunk_rows,
                                   void *stream) {
    // no allocation of any kind here: the library must be set up already
    if (!g.ready || g.device >= kMaxDevices || g_scratch_ptr[g.device] == nullptr) {
        set_error(-4, "logits_noalloc: call edgexpu_hip_init first (this entry point allocates nothing)");
        return 0;
    }
    if (!check_logits_args(scores, hidden, w, type, m, vocab, n_embd, chunk_rows, "logits_noalloc")) return 0;
    size_t qb, kb;
    act_ws_sizes(type, m, n_embd, qb, kb);
    if (n_embd > kScratchMaxEmbd || qb + kb > kScratchBytes) {
        set_error(-2, "logits_noalloc: m=%d x n_embd=%d exceeds the fixed scratch (n_embd <= %d, m <= %d)", m,
                  n_embd, kScratchMaxEmbd, kGemvMaxTokens);
        return 0;
    }
    ActWs a;
    act_ws_carve(type, m, n_embd, (uint8_t *)g_scratch_ptr[g.device], a);
    return logits_run(scores, best_dev, hidden, w, type, bias, m, vocab, n_embd, pick_stream(stream), a) ? 1 : 0;
}

int edgexpu_hip_dequantize_dev(const void *src, uint32_t type, uint64_t n_elements, float *dst, void *stream) {
    if (!ensure_init()) return 0;
    if (src == nullptr || dst == nullptr || n_elements == 0) {
        set_error(-2, "dequantize: null buffer or zero elements");
        return 0;
    }
    if (!gpu_type(type)) {
        set_error(-3, "dequantize: GGUF type %u is not supported (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)", type);
        return 0;
    }
    if (n_elements % block_elems(type) != 0) {
        set_error(-2, "dequantize: %llu elements is not a multiple of the type-%u block",
                  (unsigned long long)n_elements, type);
        return 0;
    }
    if (!aligned16(dst)) {
        set_error(-2, "dequantize: dst must be 16-byte aligned");
        return 0;
    }
    if (!check_weight_align(src, type, "dequantize")) return 0;
    return hip_ok(launch_dequantize((const uint8_t *)src, (int)type, n_elements, dst, pick_stream(stream)),
                  "dequantize")
               ? 1
               : 0;
}

int edgexpu_hip_embed_rows_dev(float *out, const void *table, uint32_t type, long long n_rows, int n_embd,
                               const int32_t *ids, int n_ids, int *bad, void *stream) {
    if (!ensure_init()) return 0;
    if (out == nullptr || table == nullptr || ids == nullptr || n_rows <= 0 || n_embd <= 0 || n_ids <= 0 ||
        n_ids > 65535) {
        set_error(-2, "embed_rows: null buffer or bad size (n_rows=%lld n_embd=%d n_ids=%d, at most 65535 ids)",
                  n_rows, n_embd, n_ids);
        return 0;
    }
    if (!gpu_type(type)) {
        set_error(-3, "embed_rows: GGUF type %u is not supported (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)", type);
        return 0;
    }
    if ((size_t)n_embd % embed_unit(type) != 0 || !aligned16(out)) {
        set_error(-2, "embed_rows: n_embd=%d must be a multiple of %zu for type %u and out 16-byte aligned", n_embd,
                  embed_unit(type), type);
        return 0;
    }
    if (!check_weight_align(table, type, "embed_rows")) return 0;
    return hip_ok(launch_dequantize_rows((const uint8_t *)table, (int)type, n_rows, n_embd, ids, n_ids, out, bad,
                                         pick_stream(stream)),
                  "embed_rows")
               ? 1
               : 0;
}

// The reference's generator step (src/cpu_kernel.c:781-786) and its uniform
// (src/cpu_kernel.c:820,834): (state & 0xFFFFFFF) / 2^28.
static double sample_uniform(uint64_t *rng) {
    if (*rng == 0) *rng = 0x00ED6E50ULL;
    *rng ^= *rng << 13;
    *rng ^= *rng >> 7;
    *rng ^= *rng << 17;
    return (double)(*rng & 0xFFFFFFFu) / (double)0x10000000u;
}

int edgexpu_hip_sample_softmax_dev(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out, void *stream) {
    if (!ensure_init()) return 0;
    if (logits == nullptr || rng == nullptr || out == nullptr || n <= 0 || n > (1 << 24)) {
        set_error(-2, "sample_softmax: null argument or n=%d outside 1..2^24", n);
        return 0;
    }
    void *ws = sample_ws(sample_workspace_bytes(n));
    if (ws == nullptr) return 0;
    const double u = sample_uniform(rng);
    return hip_ok(launch_sample_softmax(logits, n, top_p, u, out, ws, pick_stream(stream)), "sample_softmax") ? 1 : 0;
}

int edgexpu_hip_div_scalar_dev(float *io, long long n, float d, void *stream) {
    if (!ensure_init()) return 0;
    if (io == nullptr || n <= 0) {
        set_error(-2, "div_scalar: null buffer or n=%lld", n);
        return 0;
    }
    return hip_ok(launch_div_scalar(io, n, d, pick_stream(stream)), "div_scalar") ? 1 : 0;
}

int edgexpu_hip_softmax_dev(float *io, int n, void *stream) {
    if (!ensure_init()) return 0;
    if (io == nullptr || n <= 0 || n > (1 << 24)) {
        set_error(-2, "softmax: null argument or n=%d outside 1..2^24", n);
        return 0;
    }
    void *ws = sample_ws(sample_workspace_bytes(n));
    if (ws == nullptr) return 0;
    return hip_ok(launch_sample_softmax(io, n, 1.0f, 0.0, nullptr, ws, pick_stream(stream)), "softmax") ? 1 : 0;
}

static int quantize_dev(const float *x, int m, int n, uint8_t *dst, void *stream, bool k_quant) {
    if (!ensure_init()) return 0;
    const int qk = k_quant ? kQKK : kQK8_0;
    if (x == nullptr || dst == nullptr || m <= 0 || n <= 0 || n % qk != 0) {
        set_error(-2, "quantize_q8_%s: bad arguments (m=%d n=%d)", k_quant ? "k" : "0", m, n);
        return 0;
    }
    if (!aligned16(x) || (k_quant && ((uintptr_t)dst & 3u) != 0) || (!k_quant && ((uintptr_t)dst & 1u) != 0)) {
        set_error(-2, "quantize: x must be 16-byte and dst %d-byte aligned", k_quant ? 4 : 2);
        return 0;
    }
    hipStream_t st = pick_stream(stream);
    const hipError_t e = k_quant ? launch_quantize_q8_k(x, m, n, n, dst, st) : launch_quantize_q8_0(x, m, n, n, dst, st);
    return hip_ok(e, "quantize") ? 1 : 0;
}

int edgexpu_hip_quantize_q8_0_dev(const float *x, int m, int n, uint8_t *dst, void *stream) {
    return quantize_dev(x, m, n, dst, stream, false);
}

int edgexpu_hip_quantize_q8_k_dev(const float *x, int m, int n, uint8_t *dst, void *stream) {
    return quantize_dev(x, m, n, dst, stream, true);
}

// ------------------------------------------------------ layer elementwise ops

int edgexpu_hip_rmsnorm_dev(float *out, const float *x, const float *weight, int m, int n, float eps, void *stream) {
    if (!ensure_init()) return 0;
    if (out == nullptr || x == nullptr || weight == nullptr || m <= 0 || n <= 0) {
        set_error(-2, "rmsnorm: null buffer or bad size (m=%d n=%d)", m, n);
        return 0;
    }
    return hip_ok(launch_rmsnorm(x, weight, out, m, n, eps, pick_stream(stream)), "rmsnorm") ? 1 : 0;
}

namespace {
int elementwise_dev(float *out, const float *a, const float *b, long long n, int kind, void *stream, const char *what) {
    if (!ensure_init()) return 0;
    if (out == nullptr || a == nullptr || (kind != 0 && b == nullptr) || n <= 0) {
        set_error(-2, "%s: null buffer or bad size (n=%lld)", what, n);
        return 0;
    }
    return hip_ok(launch_elementwise(a, b, out, n, kind, pick_stream(stream)), what) ? 1 : 0;
}
}  // namespace

int edgexpu_hip_silu_dev(float *out, const float *x, long long n, void *stream) {
    return elementwise_dev(out, x, nullptr, n, 0, stream, "silu");
}
int edgexpu_hip_mul_dev(float *out, const float *a, const float *b, long long n, void *stream) {
    return elementwise_dev(out, a, b, n, 1, stream, "mul");
}
int edgexpu_hip_add_dev(float *out, const float *a, const float *b, long long n, void *stream) {
    return elementwise_dev(out, a, b, n, 2, stream, "add");
}
int edgexpu_hip_silu_mul_dev(float *out, const float *gate, const float *up, long long n, void *stream) {
    return elementwise_dev(out, gate, up, n, 3, stream, "silu_mul");
}

// ------------------------------------------------------------ host entries

int edgexpu_hip_linear_quant_batch(float *out, const float *x, const edgexpu_hip_weight *w, int m) {
    if (!ensure_init()) return 0;
    if (w == nullptr || out == nullptr || x == nullptr || m <= 0) {
        set_error(-2, "linear_quant_batch: null argument or m <= 0");
        return 0;
    }
    const size_t xb = align_up((size_t)m * w->n_in * sizeof(float), 256);
    const size_t ob = (size_t)m * w->n_out * sizeof(float);
    uint8_t *d = (uint8_t *)devbuf(xb + ob);
    if (d == nullptr) return 0;
    if (!hip_ok(hipMemcpyAsync(d, x, (size_t)m * w->n_in * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D x"))
        return 0;
    if (!edgexpu_hip_linear_quant_batch_dev((float *)(d + xb), (const float *)d, w->data, w->type, w->bias, m,
                                            w->n_out, w->n_in, g.stream))
        return 0;
    if (!hip_ok(hipMemcpyAsync(out, d + xb, ob, hipMemcpyDeviceToHost, g.stream), "D2H out")) return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

int edgexpu_hip_linear_quant_batch_host(float *out, const float *x, const uint8_t *weight, uint32_t type,
                                        const float *bias, int m, int n_out, int n_in) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(out, x, weight, type, m, n_out, n_in, "linear_quant_batch")) return 0;
    edgexpu_hip_weight *w = edgexpu_hip_weight_upload(weight, type, n_out, n_in, bias);
    if (w == nullptr) return 0;
    const int ok = edgexpu_hip_linear_quant_batch(out, x, w, m);
    edgexpu_hip_weight_free(w);
    return ok;
}

int edgexpu_hip_logits(float *scores, uint32_t *best, const float *hidden, const edgexpu_hip_weight *w,
                       int chunk_rows) {
    if (!ensure_init()) return 0;
    if (w == nullptr || hidden == nullptr) {
        set_error(-2, "logits: null argument");
        return 0;
    }
    const size_t hb = align_up((size_t)w->n_in * sizeof(float), 256);
    const size_t sb = align_up((size_t)w->n_out * sizeof(float), 256);
    uint8_t *d = (uint8_t *)devbuf(hb + sb + 256);
    if (d == nullptr) return 0;
    float *dh = (float *)d;
    float *ds = (float *)(d + hb);
    uint32_t *dbest = (uint32_t *)(d + hb + sb);
    if (!hip_ok(hipMemcpyAsync(dh, hidden, (size_t)w->n_in * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D"))
        return 0;
    if (!edgexpu_hip_logits_dev(ds, dbest, dh, w->data, w->type, w->bias, 1, w->n_out, w->n_in, chunk_rows,
                                g.stream))
        return 0;
    if (scores != nullptr &&
        !hip_ok(hipMemcpyAsync(scores, ds, (size_t)w->n_out * sizeof(float), hipMemcpyDeviceToHost, g.stream), "D2H"))
        return 0;
    uint32_t b = 0;
    if (!hip_ok(hipMemcpyAsync(&b, dbest, sizeof(b), hipMemcpyDeviceToHost, g.stream), "D2H best")) return 0;
    if (!hip_ok(hipStreamSynchronize(g.stream), "sync")) return 0;
    if (best != nullptr) *best = b;
    return 1;
}

int edgexpu_hip_dequantize(const uint8_t *src, uint32_t type, uint64_t n_elements, float *dst) {
    if (!ensure_init()) return 0;
    if (src == nullptr || dst == nullptr || n_elements == 0 || !gpu_type(type) ||
        n_elements % block_elems(type) != 0) {
        set_error(-2, "dequantize: bad arguments (type=%u n=%llu)", type, (unsigned long long)n_elements);
        return 0;
    }
    const size_t sbytes = (size_t)(n_elements / block_elems(type)) * block_bytes(type);
    const size_t so = align_up(sbytes, 256);
    uint8_t *d = (uint8_t *)devbuf(so + (size_t)n_elements * sizeof(float));
    if (d == nullptr) return 0;
    if (!hip_ok(hipMemcpyAsync(d, src, sbytes, hipMemcpyHostToDevice, g.stream), "H2D src")) return 0;
    if (!edgexpu_hip_dequantize_dev(d, type, n_elements, (float *)(d + so), g.stream)) return 0;
    if (!hip_ok(hipMemcpyAsync(dst, d + so, (size_t)n_elements * sizeof(float), hipMemcpyDeviceToHost, g.stream),
                "D2H dst"))
        return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

static int quantize_host(const float *x, int n, uint8_t *dst, bool k_quant) {
    if (!ensure_init()) return 0;
    const int qk = k_quant ? kQKK : kQK8_0;
    if (x == nullptr || dst == nullptr || n <= 0 || n % qk != 0) {
        set_error(-2, "quantize: bad arguments (n=%d)", n);
        return 0;
    }
    const size_t qb = (size_t)(n / qk) * (k_quant ? kBytesQ8_K : kBytesQ8_0);
    const size_t xo = align_up((size_t)n * sizeof(float), 256);
    uint8_t *d = (uint8_t *)devbuf(xo + qb);
    if (d == nullptr) return 0;
    if (!hip_ok(hipMemcpyAsync(d, x, (size_t)n * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D x")) return 0;
    if (!quantize_dev((const float *)d, 1, n, d + xo, g.stream, k_quant)) return 0;
    if (!hip_ok(hipMemcpyAsync(dst, d + xo, qb, hipMemcpyDeviceToHost, g.stream), "D2H q")) return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

int edgexpu_hip_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out) {
    if (!ensure_init()) return 0;
    if (logits == nullptr || rng == nullptr || out == nullptr || n <= 0 || n > (1 << 24)) {
        set_error(-2, "sample_softmax: null argument or n=%d outside 1..2^24", n);
        return 0;
    }
    const size_t xb = align_up((size_t)n * sizeof(float), 256);
    uint8_t *d = (uint8_t *)devbuf(xb + 256);
    if (d == nullptr) return 0;
    uint32_t *dout = (uint32_t *)(d + xb);
    if (!hip_ok(hipMemcpyAsync(d, logits, (size_t)n * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D logits"))
        return 0;
    if (!edgexpu_hip_sample_softmax_dev((float *)d, n, top_p, rng, dout, g.stream)) return 0;
    if (!hip_ok(hipMemcpyAsync(logits, d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, g.stream), "D2H p") ||
        !hip_ok(hipMemcpyAsync(out, dout, sizeof(uint32_t), hipMemcpyDeviceToHost, g.stream), "D2H token"))
        return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

int edgexpu_hip_softmax(float *io, int n) {
    if (!ensure_init()) return 0;
    if (io == nullptr || n <= 0 || n > (1 << 24)) {
        set_error(-2, "softmax: null argument or n=%d outside 1..2^24", n);
        return 0;
    }
    float *d = (float *)devbuf(align_up((size_t)n * sizeof(float), 256));
    if (d == nullptr) return 0;
    if (!hip_ok(hipMemcpyAsync(d, io, (size_t)n * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D x") ||
        !edgexpu_hip_softmax_dev(d, n, g.stream) ||
        !hip_ok(hipMemcpyAsync(io, d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, g.stream), "D2H p"))
        return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

int edgexpu_hip_quantize_q8_0(const float *x, int n, uint8_t *dst) { return quantize_host(x, n, dst, false); }
int edgexpu_hip_quantize_q8_k(const float *x, int n, uint8_t *dst) { return quantize_host(x, n, dst, true); }

int edgexpu_hip_dot_f32_rows(float *out, const uint8_t *w, uint32_t type, const float *x, int rows, int n) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(out, x, w, type, 1, rows, n, "dot_f32_rows")) return 0;
    const size_t rb = edgexpu_hip_row_bytes(type, n);
    const size_t wo = align_up(rb * (size_t)rows, 256);
    const size_t xo = align_up((size_t)n * sizeof(float), 256);
    uint8_t *d = (uint8_t *)devbuf(wo + xo + align_up((size_t)rows * sizeof(float), 256));
    if (d == nullptr) return 0;
    float *dx = (float *)(d + wo);
    float *dout = (float *)(d + wo + xo);
    if (!hip_ok(hipMemcpyAsync(d, w, rb * (size_t)rows, hipMemcpyHostToDevice, g.stream), "H2D w")) return 0;
    if (!hip_ok(hipMemcpyAsync(dx, x, (size_t)n * sizeof(float), hipMemcpyHostToDevice, g.stream), "H2D x")) return 0;
    // the f32-activation dot for every type (edgexpu_gguf_dot_quant never
    // quantizes x, src/gguf_quant.c:894-918)
    if (!run_f32_product(type, d, rows, n, 1, dx, nullptr, dout, rows, g.stream)) return 0;
    if (!hip_ok(hipMemcpyAsync(out, dout, (size_t)rows * sizeof(float), hipMemcpyDeviceToHost, g.stream), "D2H"))
        return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

int edgexpu_hip_dot_q8_rows(float *out, const uint8_t *w, uint32_t type, const uint8_t *xq, int rows, int n) {
    if (!ensure_init()) return 0;
    if (!check_linear_args(out, xq, w, type, 1, rows, n, "dot_q8_rows")) return 0;
    const size_t rb = edgexpu_hip_row_bytes(type, n);
    const size_t xb = act_bytes(type, n);
    const size_t wo = align_up(rb * (size_t)rows, 256);
    const size_t xo = align_up(xb, 256);
    uint8_t *d = (uint8_t *)devbuf(wo + xo + align_up((size_t)rows * sizeof(float), 256));
    if (d == nullptr) return 0;
    float *dout = (float *)(d + wo + xo);
    if (!hip_ok(hipMemcpyAsync(d, w, rb * (size_t)rows, hipMemcpyHostToDevice, g.stream), "H2D w")) return 0;
    if (!hip_ok(hipMemcpyAsync(d + wo, xq, xb, hipMemcpyHostToDevice, g.stream), "H2D xq")) return 0;
    if (!edgexpu_hip_gemv_q8_dev(dout, d + wo, d, type, nullptr, 1, rows, n, g.stream)) return 0;
    if (!hip_ok(hipMemcpyAsync(out, dout, (size_t)rows * sizeof(float), hipMemcpyDeviceToHost, g.stream), "D2H"))
        return 0;
    return hip_ok(hipStreamSynchronize(g.stream), "sync") ? 1 : 0;
}

}  // extern "C"
