/*
 * edgexpu_hip.h -- C-ABI of libedgexpu_hip.so, the MI355X (gfx950) kernel set
 * for the GGUF quantized-weight matrix path (Q8_0 / Q4_K / Q6_K, and the
 * dispatcher's other formats Q4_0 / Q5_0 / Q5_K / F16 / F32).
 *
 * Plain C types only (no HIP or torch types): device pointers are `void *` /
 * typed pointers into device memory, streams are `void *` holding a
 * hipStream_t; NULL is HIP's default (null) stream.  The host-pointer entry
 * points run on the library's own stream (edgexpu_hip_stream()) and return
 * only when their results are in host memory.
 *
 * Conventions shared by every entry point:
 *  - Return 1 on success, 0 on failure.  A failure records a sticky error
 *    (code + message) readable with edgexpu_hip_last_error(); the library
 *    never returns silently wrong data.  Bad arguments are rejected before
 *    any launch (the reference silently returns for them:
 *    src/cpu_kernel.c:562-564,571-574).
 *  - Single caller: like the reference path (process-global activation
 *    scratch, src/cpu_kernel.c:525-543) the library keeps one device, one
 *    stream and one workspace per process and is not reentrant.
 *  - Type ids are GGUF's (include/edgexpu/gguf_quant.h:17-24).  Every type
 *    of the reference's dispatcher runs on the GPU: F32 (0), F16 (1),
 *    Q4_0 (2), Q5_0 (6), Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14); any other
 *    id is rejected as unsupported.
 */
#ifndef EDGEXPU_HIP_H
#define EDGEXPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EDGEXPU_HIP_TYPE_Q8_0 8
#define EDGEXPU_HIP_TYPE_Q4_K 12
#define EDGEXPU_HIP_TYPE_Q6_K 14

/* ---- lifecycle and errors (no reference counterpart: the reference has no
 * device; these replace its implicit process-global CPU state) ---- */

/* Selects `device`, creates the library stream.  Optional: every entry point
 * initialises device 0 on first use. */
int edgexpu_hip_init(int device);
/* Releases the stream, workspace and staging buffers. */
void edgexpu_hip_shutdown(void);
/* Sticky error: returns the last error code (0 = none) and copies its
 * message into buf.  The error stays set until edgexpu_hip_clear_error(). */
int edgexpu_hip_last_error(char *buf, size_t size);
void edgexpu_hip_clear_error(void);
/* 1 when `type` runs on the GPU: every type of the reference's dispatcher
 * (src/gguf_quant.c:69-108; src/gguf_dot_q8.c:414-434): Q4_0, Q5_0, Q8_0
 * with Q8_0 activations, Q4_K, Q5_K, Q6_K with Q8_K activations, F16 and F32
 * with f32 activations (any n_in). */
int edgexpu_hip_supports_type(uint32_t type);
/* Prefill (m >= 16 tokens; Q5_K from 32) arithmetic.  No reference
 * counterpart: the reference has one CPU path.
 *  EDGEXPU_HIP_PREFILL_EXACT_INT8 (default, every quantized format): the
 *    matrix cores on integer operands with every block integer exact,
 *    outputs within the 1e-5 bound of the reference;
 *  EDGEXPU_HIP_PREFILL_F16 (Q4_K; the other formats stay exact): fp16 matrix
 *    cores on the Q8_K activation and the dequantized weight (each rounded
 *    once to fp16, after exact power-of-two row prescales that keep any
 *    magnitude in fp16 range), fp32 sums: outputs within the 1e-3 prefill
 *    bound.
 * Process-wide setting of this library (like its stream); decode (m < 16)
 * is unaffected.  Returns 1, or 0 (sticky error) for an unknown mode. */
#define EDGEXPU_HIP_PREFILL_EXACT_INT8 0
#define EDGEXPU_HIP_PREFILL_F16 1
int edgexpu_hip_set_prefill_mode(int mode);
int edgexpu_hip_prefill_mode(void);
/* Decode GEMV kernel for the launches both kernels cover: one token of Q4_K
 * rows of 2560, 4096 or 14336 elements or of Q6_K rows of 9728 (every
 * variant), plain projections of 2-4 tokens of those rows (activations
 * given as f32), and the f32-activation logits of one or two tokens against
 * Q4_K rows of 4096 or Q6_K rows of 2560.  No reference counterpart (the
 * reference has one CPU kernel).
 *  EDGEXPU_HIP_GEMV_AUTO (default): the streaming kernel (weight rows
 *    through LDS by DMA), except launches of fewer than 2048 rows of 9728
 *    Q6_K elements or of 14336 Q4_K elements at 1-3 tokens, which take the
 *    fused kernel;
 *  EDGEXPU_HIP_GEMV_FUSED / EDGEXPU_HIP_GEMV_STREAM: always that kernel
 *    (FUSED at four tokens of 14336 elements, whose codes exceed the fused
 *    kernel's LDS: a quantize launch and the generic GEMV).
 * The two give the same outputs bit for bit (same lane partials, same
 * reduction order), so the setting moves time, never results -- except four
 * tokens of 14336 elements, where the generic GEMV's summation order differs
 * (both within 1e-5 of each row's conditioning scale of the reference).
 * Process-wide setting of this library.  Returns 1, or 0 (sticky error) for
 * an unknown mode. */
#define EDGEXPU_HIP_GEMV_AUTO 0
#define EDGEXPU_HIP_GEMV_FUSED 1
#define EDGEXPU_HIP_GEMV_STREAM 2
int edgexpu_hip_set_gemv_mode(int mode);
int edgexpu_hip_gemv_mode(void);
/* Blocks until the library stream is idle. */
int edgexpu_hip_synchronize(void);
/* hipStream_t of the library stream. */
void *edgexpu_hip_stream(void);

/* ---- layout (src/gguf_quant.c:69-108,468-480; src/gguf_dot_q8.c:255-267) ---- */
size_t edgexpu_hip_row_bytes(uint32_t type, int n_in);

/* ---- device-resident GGUF weights ----
 * Replaces the per-token staging copy of src/native.c:350-380,593-655: a
 * tensor's blocks are uploaded once and addressed by handle, never by the
 * (aliasing) host staging pointer. */
typedef struct edgexpu_hip_weight edgexpu_hip_weight;

/* Copies n_out rows of GGUF blocks (and n_out f32 biases, may be NULL) to
 * the device.  Returns NULL on error. */
edgexpu_hip_weight *edgexpu_hip_weight_upload(const uint8_t *blocks, uint32_t type, int n_out, int n_in,
                                              const float *bias);
/* Wraps blocks already in device memory (not owned; the caller keeps them
 * alive).  dev_bias may be NULL. */
edgexpu_hip_weight *edgexpu_hip_weight_wrap(const void *dev_blocks, uint32_t type, int n_out, int n_in,
                                            const float *dev_bias);
void edgexpu_hip_weight_free(edgexpu_hip_weight *w);
/* One device allocation holding a copy of n bytes of host memory (pageable
 * memory or a mapped file; copied synchronously), for the model upload of
 * edgexpu_gguf_upload.h.  NULL on error.  Free with edgexpu_hip_free_bytes. */
void *edgexpu_hip_upload_bytes(const void *host, size_t n);
/* Copies n bytes of device memory to host memory (synchronous). */
int edgexpu_hip_download_bytes(void *host, const void *dev, size_t n);
void edgexpu_hip_free_bytes(void *dev);
const void *edgexpu_hip_weight_data(const edgexpu_hip_weight *w);
uint32_t edgexpu_hip_weight_type(const edgexpu_hip_weight *w);
int edgexpu_hip_weight_n_out(const edgexpu_hip_weight *w);
int edgexpu_hip_weight_n_in(const edgexpu_hip_weight *w);

/* ---- device-pointer entry points (all buffers in device memory; work is
 * queued on `stream` and not waited for).  Weight blocks may start at any
 * address except that Q8_0, Q4_0, Q5_0 and Q6_K blocks (34, 18, 22 and 210
 * bytes) must start at an even one: an odd one is refused with error -2.
 * GGUF tensors in a device copy of a file's data section always qualify.
 * Blocks at 16-byte addresses can take the streaming GEMV and logits (Q4_K,
 * Q6_K) and the matrix-core prefill (Q4_K; the others need even addresses);
 * blocks elsewhere take the fused GEMV, with the same results. ---- */

/* out[t*n_out + o] = bias[o] + dot(W[o], q8(x[t]))  for t < m.
 * Replaces edgexpu_cpu_linear_quant_batch (include/edgexpu/cpu_kernel.h:71-80,
 * src/cpu_kernel.c:545-644): activations are quantized once per token
 * (Q8_0 for the Q8_0 family, Q8_K for the K-quants) and every row is dotted
 * with the integer block kernels; F16 and F32 rows take the f32-activation
 * dot (F32 at m == 1 adds the bias in double, as edgexpu_cpu_linear,
 * src/cpu_kernel.c:462-523).  x is [m][n_in] f32, out [m][n_out] f32, x
 * 16-byte aligned; bias may be NULL. */
int edgexpu_hip_linear_quant_batch_dev(float *out, const float *x, const void *w, uint32_t type,
                                       const float *bias, int m, int n_out, int n_in, void *stream);

/* Several projections of the same input in one launch (q/k/v, or gate/up):
 * out[z][t*n_out[z] + o] = bias[z][o] + dot(W_z[o], q8(x[t])) for z < nmat
 * (1..4).  All matrices share type and n_in; bias may be NULL or hold NULL
 * entries.  Equivalent to nmat edgexpu_hip_linear_quant_batch_dev calls
 * (src/native.c:2530-2532 and :2576-2577 issue them back to back). */
int edgexpu_hip_linear_quant_group_dev(int nmat, float *const *out, const float *x, const void *const *w,
                                       uint32_t type, const float *const *bias, const int *n_out, int m, int n_in,
                                       void *stream);

/* The integer block-dot product alone, for activations already quantized
 * into the reference's block bytes (one token = n_in/32 Q8_0 blocks for Q8_0
 * weights, n_in/256 Q8_K blocks for Q4_K / Q6_K; token t at
 * xq + t * that size): out[t*n_out + o] = bias[o] + dot(W[o], xq[t]).
 * edgexpu_gguf_dot_quant_q8 / _q8k (src/gguf_dot_q8.c:1004-1044) over all
 * rows and tokens at once; lets several projections share one quantized
 * input. */
int edgexpu_hip_gemv_q8_dev(float *out, const uint8_t *xq, const void *w, uint32_t type, const float *bias, int m,
                            int n_out, int n_in, void *stream);

/* Logits product of src/native.c:2292-2401 for m hidden vectors:
 * scores[t*vocab + i] = dot(W[i], h[t]) (+ bias[i]) with the Q8_0-activation
 * dot for Q8_0 weights and the f32-activation dots for Q4_K / Q6_K
 * (src/native.c:445-514, src/gguf_quant.c:704-794).  chunk_rows (>= 0) is the
 * reference's row chunking (0 = its 48 MiB budget,
 * include/edgexpu/scheduler.h:34); no score depends on it, and the GPU covers
 * every chunk in one launch.
 * When best_dev is non-NULL, best_dev[t] receives the greedy argmax of row t
 * (lowest index on ties, NaN never wins, 0 when nothing beats -inf). */
int edgexpu_hip_logits_dev(float *scores, uint32_t *best_dev, const float *hidden, const void *w, uint32_t type,
                           const float *bias, int m, int vocab, int n_embd, int chunk_rows, void *stream);

/* edgexpu_hip_logits_dev with no allocation of any kind, for callers that
 * cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  No counterpart in the reference.
 * Same arguments, checks and results (bit for bit) as edgexpu_hip_logits_dev.
 * Its scratch (quantized hidden vectors, argmax partial keys) is one fixed
 * device array of 402 KiB per GPU, held until the
 * process ends: m <= 8 and n_embd <= 16384, larger calls are refused.
 * edgexpu_hip_init must have run on the device first.  Every call on a GPU
 * shares that GPU's array, which keeps the last call's contents (every part
 * is written before it is read, nothing needs clearing): calls that overlap
 * on one GPU (several streams or threads) race. */
int edgexpu_hip_logits_noalloc_dev(float *scores, uint32_t *best_dev, const float *hidden, const void *w,
                                   uint32_t type, const float *bias, int m, int vocab, int n_embd, int chunk_rows,
                                   void *stream);

/* Bulk dequantization (edgexpu_gguf_dequantize, include/edgexpu/gguf_quant.h:32-39,
 * src/gguf_quant.c:355-411), bit-identical to the reference's x86 build.
 * n_elements must be a multiple of the block size; dst 16-byte aligned. */
int edgexpu_hip_dequantize_dev(const void *src, uint32_t type, uint64_t n_elements, float *dst, void *stream);

/* Embedding lookup on device: rows ids[0..n_ids) of the [n_rows x n_embd]
 * matrix `table` (device-resident GGUF rows of `type`) dequantized into
 * out[n_ids][n_embd] (16-byte aligned), each bit-identical to
 * edgexpu_gguf_dequantize_row on that row (src/gguf_quant.c:428-466, called
 * per token by src/native.c:428-443).  ids is a device array (for example
 * the greedy argmax of the previous step); an id outside [0, n_rows) gives a
 * row of zeros and, when `bad` (device int) is non-null, stores 1 into it
 * (the reference reports "row out of range").  n_embd a multiple of the
 * type's block (of 4 for F16 and F32, whose rows are written with 16-byte
 * stores); 1 <= n_ids <= 65535. */
int edgexpu_hip_embed_rows_dev(float *out, const void *table, uint32_t type, long long n_rows, int n_embd,
                               const int32_t *ids, int n_ids, int *bad, void *stream);

/* Sampling on device (edgexpu_cpu_sample_softmax,
 * include/edgexpu/cpu_kernel.h:86-94, src/cpu_kernel.c:762-849, the
 * temperature path of src/native.c:2326-2350): softmax of logits[0..n) in
 * place (edgexpu_cpu_softmax, cpu_kernel.h:24, src/cpu_kernel.c:328-353),
 * then one draw into *out (a device uint32): from the whole distribution in
 * index order, or with 0 < top_p < 1 from the smallest prefix, in (p desc,
 * id asc) order, whose sum reaches top_p.  *rng is a host word advanced by the
 * reference's xorshift step (a zero state is seeded with 0x00ED6E50); the
 * uniform is (state & 0xFFFFFFF) / 2^28 as in the reference.  Probabilities
 * agree with the reference within a few float ulp (device expf; sums in
 * double in a fixed segment order); the token differs only where the pick
 * falls within that distance of a running sum.  logits 16-byte aligned,
 * 1 <= n <= 2^24.  The library's sampling workspace (8 bytes per entry plus
 * ~230 KiB) is allocated on the first call of a larger n and reused. */
int edgexpu_hip_sample_softmax_dev(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out, void *stream);
/* io[i] = io[i] / d on device, float division: the temperature scaling of
 * the scores before sampling (src/native.c:2339). */
int edgexpu_hip_div_scalar_dev(float *io, long long n, float d, void *stream);
/* Softmax of io[0..n) in place on device (edgexpu_cpu_softmax). */
int edgexpu_hip_softmax_dev(float *io, int n, void *stream);

/* Activation quantizers writing the reference's block bytes
 * (edgexpu_gguf_quantize_q8_0 / _q8_k, include/edgexpu/gguf_quant.h:80-87,
 * src/gguf_dot_q8.c:269-412): m rows of n f32 -> m*(n/32)*34 or
 * m*(n/256)*292 bytes, bit-identical to the reference's x86 build. */
int edgexpu_hip_quantize_q8_0_dev(const float *x, int m, int n, uint8_t *dst, void *stream);
int edgexpu_hip_quantize_q8_k_dev(const float *x, int m, int n, uint8_t *dst, void *stream);

/* The elementwise layer ops around the projections, on device-resident
 * activations (the ops a decode layer applies between its projections,
 * src/native.c:2529-2580), so that a layer's activations need not leave the
 * GPU.  Same arithmetic as the reference op for op:
 *   rmsnorm:  edgexpu_cpu_rmsnorm (include/edgexpu/cpu_kernel.h:19,
 *             src/cpu_kernel.c:220-242), over m rows of n elements with one
 *             weight vector of n; double sum of squares (as a tree: the float
 *             mean can differ from the reference's index-order sum only where
 *             its rounding falls within the double sum's error);
 *   silu:     edgexpu_cpu_silu (cpu_kernel.h:20, src/cpu_kernel.c:244-252),
 *             with the device expf (about one ulp; the host libm's 0.502):
 *             within four ulp of the reference's silu;
 *   mul, add: edgexpu_cpu_mul / edgexpu_cpu_add (src/cpu_kernel.c:200-218),
 *             exact;
 *   silu_mul: silu(gate) then * up in one pass, the reference's
 *             edgexpu_cpu_silu + edgexpu_cpu_mul (src/native.c:2577-2578).
 * out may equal an input.  Return 1 on success, 0 on bad arguments or a HIP
 * error (see edgexpu_hip_last_error). */
int edgexpu_hip_rmsnorm_dev(float *out, const float *x, const float *weight, int m, int n, float eps, void *stream);
int edgexpu_hip_silu_dev(float *out, const float *x, long long n, void *stream);
int edgexpu_hip_mul_dev(float *out, const float *a, const float *b, long long n, void *stream);
int edgexpu_hip_add_dev(float *out, const float *a, const float *b, long long n, void *stream);
int edgexpu_hip_silu_mul_dev(float *out, const float *gate, const float *up, long long n, void *stream);

/* A decode layer's projection with the ops around it, on device-resident
 * activations (src/native.c:2529-2580: rmsnorm -> q/k/v, o -> add,
 * rmsnorm -> gate/up, silu * up -> down -> add):
 *   act    = rmsnorm(x; norm_weight, eps)  when norm_weight != NULL
 *          = silu(x) * x2                  when x2 != NULL (not both)
 *          = x                             otherwise
 *   out[z] = residual[z] + (bias[z] + W[z] . q8(act))
 * for nmat <= 4 matrices of one type and n_in that share the input (q/k/v,
 * gate/up), with residual (or any residual[z]) and bias optional, as
 * edgexpu_cpu_rmsnorm / edgexpu_cpu_silu + edgexpu_cpu_mul, then
 * edgexpu_cpu_linear_quant_batch (include/edgexpu/cpu_kernel.h:60-80), then
 * edgexpu_cpu_add compute it: the same result as those entry points of this
 * library in sequence (the layer ops above, edgexpu_hip_linear_quant_group_dev).
 * One token with the prologue, or no prologue, runs as one launch (the
 * prologue in the GEMV's activation staging, the residual in its store);
 * other shapes run the same steps as separate launches.  out[z] may be
 * residual[z] (an in-place residual update); out must not overlap x or x2.
 * x, x2, norm_weight 16-byte aligned.  Returns 1 on success, 0 on bad
 * arguments or a HIP error. */
int edgexpu_hip_layer_linear_dev(int nmat, float *const *out, const float *x, const float *x2,
                                 const float *norm_weight, float eps, const void *const *w, uint32_t type,
                                 const float *const *bias, const float *const *residual, const int *n_out, int m,
                                 int n_in, void *stream);

/* A decode layer's gate and up projections with the SwiGLU product
 * (src/native.c:2575-2578):
 *   a   = rmsnorm(x; norm_weight, eps)  (norm_weight != NULL) or x
 *   act = silu(b_gate + W_gate . q8(a)) * (b_up + W_up . q8(a))   [m][n_ff]
 * as edgexpu_hip_layer_linear_dev over gate and up followed by
 * edgexpu_hip_silu_mul_dev compute it (bit for bit).  At one token it is one
 * launch: row j of gate and row j of up are reduced in the same wave and the
 * store writes their product, so SiLU runs once per element and the down
 * projection takes act with no prologue.  Biases optional; act must not
 * overlap x.  Returns 1 on success, 0 on bad arguments or a HIP error. */
int edgexpu_hip_gate_up_silu_dev(float *act, const float *x, const float *norm_weight, float eps, const void *w_gate,
                                 const void *w_up, uint32_t type, const float *b_gate, const float *b_up, int m,
                                 int n_ff, int n_in, void *stream);

/* ---- host-pointer entry points (synchronous: inputs copied in, outputs
 * copied out before return; the PCIe copies are part of the call) ---- */

/* edgexpu_cpu_linear_quant_batch with a device-resident weight handle: x is
 * host [m][n_in], out host [m][n_out]; the handle's bias is applied. */
int edgexpu_hip_linear_quant_batch(float *out, const float *x, const edgexpu_hip_weight *w, int m);

/* Same, with the weight rows passed as host GGUF bytes (uploaded for this call
 * only: correct for the reference's reused staging buffer, but PCIe-bound). */
int edgexpu_hip_linear_quant_batch_host(float *out, const float *x, const uint8_t *weight, uint32_t type,
                                        const float *bias, int m, int n_out, int n_in);

/* Logits with a device-resident output weight: hidden host [n_embd], scores
 * host [vocab] (may be NULL), *best receives the greedy argmax. */
int edgexpu_hip_logits(float *scores, uint32_t *best, const float *hidden, const edgexpu_hip_weight *w,
                       int chunk_rows);

/* Host-buffer sampling and softmax: logits / io host f32 (overwritten with
 * the probabilities), *out a host word. */
int edgexpu_hip_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out);
int edgexpu_hip_softmax(float *io, int n);

/* Host-buffer dequantization: src host bytes, dst host f32. */
int edgexpu_hip_dequantize(const uint8_t *src, uint32_t type, uint64_t n_elements, float *dst);

/* Host-buffer quantizers (reference block bytes). */
int edgexpu_hip_quantize_q8_0(const float *x, int n, uint8_t *dst);
int edgexpu_hip_quantize_q8_k(const float *x, int n, uint8_t *dst);

/* f32-activation row dots on the GPU for `rows` consecutive rows
 * (edgexpu_gguf_dot_quant, src/gguf_quant.c:894-918, batched over rows):
 * host in/out. */
int edgexpu_hip_dot_f32_rows(float *out, const uint8_t *w, uint32_t type, const float *x, int rows, int n);

/* Quantized-activation row dots on the GPU for `rows` consecutive rows against
 * one activation already in the reference's Q8_0 (34 B/32) or Q8_K
 * (292 B/256) block bytes (edgexpu_gguf_dot_quant_q8 / _q8k,
 * src/gguf_dot_q8.c:1004-1044, batched over rows): host in/out. */
int edgexpu_hip_dot_q8_rows(float *out, const uint8_t *w, uint32_t type, const uint8_t *xq, int rows, int n);

#ifdef __cplusplus
}
#endif

#endif
