/*
 * edgexpu_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A clean-room CPU restatement of tangjie133/edgexpu-llm's quantized-weight
 * matrix path (GGUF Q8_0 / Q4_K / Q6_K, and the dispatcher's other formats
 * Q4_0 / Q5_0 / Q5_K / F16 / F32), used as the parity checker for the
 * HIP kernels and as the "port" CPU baseline.  Nothing in the product links,
 * loads or calls this code; only tests/, the smoke entry and the bench's CPU
 * baseline leg do.
 *
 * Numerics follow the reference's x86 build (gcc -std=c11, so no FMA
 * contraction; AVX2 + FMA + F16C intrinsics): every function below
 * reproduces the reference's lane decomposition and fp32 combination order,
 * so its results are bit-identical to the reference's on the same inputs.
 * Each function cites the reference lines it restates.
 */
#ifndef EDGEXPU_ORACLE_H
#define EDGEXPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (include/edgexpu/gguf_quant.h:17-24). */
enum {
    ORA_F32 = 0, ORA_F16 = 1, ORA_Q4_0 = 2, ORA_Q5_0 = 6,
    ORA_Q8_0 = 8, ORA_Q4_K = 12, ORA_Q5_K = 13, ORA_Q6_K = 14
};

/* fp16 codecs: src/gguf_quant.c:34-37 (F16C widen) and
 * src/gguf_dot_q8.c:33-35 (F16C narrow, round-to-nearest-even). */
float ora_fp16_to_fp32(uint16_t h);
uint16_t ora_fp32_to_fp16(float f);

/* Layout constants: src/gguf_quant.c:69-108, 468-480; src/gguf_dot_q8.c:255-267. */
size_t ora_block_size(uint32_t type);
size_t ora_block_bytes(uint32_t type);
size_t ora_row_bytes(uint32_t type, int n);
size_t ora_q8_0_nbytes(int n);
size_t ora_q8_k_nbytes(int n);

/* Bulk dequantization: src/gguf_quant.c:139-353 (F16, Q4_0, Q5_0, Q8_0, Q4_K,
 * Q5_K, Q6_K), dispatched as in 355-411.
 * Returns 1 on success, 0 for a bad argument or unsupported type. */
int ora_dequantize(const uint8_t *src, uint32_t type, uint64_t n, float *dst);

/* Activation quantizers: src/gguf_dot_q8.c:276-324 (Q8_0, AVX2 variant)
 * and 360-412 (Q8_K). */
int ora_quantize_q8_0(const float *x, int n, uint8_t *dst);
int ora_quantize_q8_k(const float *x, int n, uint8_t *dst);

/* Per-block integers the fp32 combination consumes (for exact integer checks).
 *   q8_0: lanes[u] = sum_{e=4u..4u+3} w[e]*x[e], u < 8           (gguf_dot_q8.c:440-452)
 *   q4_k: lanes[u] (u<8) as in gguf_dot_q8.c:646-660, mins[k] (k<4) as :635-638
 *   q6_k: lanes[u] (u<8) as in gguf_dot_q8.c:917-959 (after the -32*bsum term) */
void ora_q8_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]);
void ora_q4_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8], int32_t mins[4]);
void ora_q6_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8]);
/*   q4_0 / q5_0: lanes[u] = sum_{e=4u..4u+3} (c[e]-8 | c[e]-16) * x[e]   (gguf_dot_q8.c:552-568, 482-502)
 *   q5_k: lanes[u] as q4_k with 5-bit codes; *mins = sum_k m[k]*(bs[2k]+bs[2k+1]) (gguf_dot_q8.c:772-838) */
void ora_q4_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]);
void ora_q5_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]);
void ora_q5_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8], int32_t *mins);

/* Row dots against quantized activations: src/gguf_dot_q8.c:436-1002 (AVX2
 * variants), dispatched as in 1004-1044. */
float ora_dot_q8(uint32_t type, const uint8_t *wrow, const uint8_t *xq, int n);
float ora_dot_q8k(uint32_t type, const uint8_t *wrow, const uint8_t *xq, int n);

/* Row dots against f32 activations: src/gguf_quant.c:506-892, dispatched as
 * in 894-918 (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K). */
float ora_dot_f32(uint32_t type, const uint8_t *wrow, const float *x, int n);

/* The matvec / prefill driver: src/cpu_kernel.c:462-656 (OpenMP row loop,
 * activations quantized once per token; F32 at one token through the
 * edgexpu_cpu_linear arithmetic; F16 and other rows through the f32 dot).  Returns 0 on bad arguments or an
 * unsupported type, 1 otherwise. */
int ora_linear_quant_batch(float *out, const float *x, const uint8_t *w, uint32_t type,
                           const float *bias, int m, int n_out, int n_in);

/* Logits product of src/native.c:2292-2401: scores[i] = dot(W[i], h) (+ bias[i]),
 * with the Q8_0 activation path for the Q8_0 family (Q4_0, Q5_0, Q8_0) and the
 * f32 path for the others; rows processed in chunks of chunk_rows (0 = the 48 MiB budget of
 * include/edgexpu/scheduler.h:34).  Returns the greedy argmax (lowest index
 * on ties).  scores may be NULL. */
uint32_t ora_logits(float *scores, const float *hidden, const uint8_t *w, uint32_t type,
                    const float *bias, int vocab, int n_embd, size_t chunk_rows);


/* The elementwise layer ops around the projections (src/cpu_kernel.c:
 * 200-252), used by the device-resident layer entry points:
 *   rmsnorm: double sum of x^2 in index order, mean = (float)(ss / n),
 *            scale = 1.0f / sqrtf(mean + eps), out = x * scale, out *= w;
 *   silu:    out = x / (1.0f + expf(-x));
 *   mul/add: out = a * b, out = a + b. */
void ora_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void ora_silu(float *out, const float *x, int n);
void ora_mul(float *out, const float *a, const float *b, int n);
void ora_add(float *out, const float *a, const float *b, int n);

/* Temperature sampling of src/native.c:2326-2350: softmax in place
 * (src/cpu_kernel.c:328-353), the xorshift64 step (:781-786) and the
 * full-distribution or top-p draw (:762-849). */
void ora_softmax(float *io, int n);
uint64_t ora_rng_step(uint64_t *rng);
int ora_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out);
/* Self-checks restated from src/gguf_quant.c:934-1061 (Q4_K, Q4_0, F16, Q5_K,
 * Q8_0 and Q5_0 parts).
 * Returns 1 when they pass. */
int ora_selftest(char *error, size_t error_size);

#ifdef __cplusplus
}
#endif

#endif
