/*
 * edgexpu_kernels.h -- the drop-in kernel set of libedgexpu_kernels.so (C11).
 *
 * Exports the reference's own entry points for the quantized-weight matrix
 * path, with the same names, signatures, argument meaning and error behaviour,
 * so a host built against include/edgexpu/cpu_kernel.h and
 * include/edgexpu/gguf_quant.h links against this library instead of
 * src/cpu_kernel.c + src/gguf_quant.c + src/gguf_dot_q8.c.  Every compute
 * entry runs on the GPU through libedgexpu_hip.so; nothing here computes on
 * the CPU.  Every type of the reference's dispatcher runs on the GPU: F32,
 * F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K and Q6_K, rows of any length the type's
 * block allows.  What the reference silently ignores (NULL buffers,
 * non-positive sizes, unknown types, lengths that are not whole blocks) is
 * ignored here too: void entries leave `out` untouched, the others return
 * 0 / 0.0f, and a sticky error readable with edgexpu_hip_last_error() names
 * the cause.
 *
 * The row entry points take the reference's edgexpu_gguf_tensor
 * (include/edgexpu/gguf.h:21-27).  Hosts that include that header include it
 * before this one; otherwise the same layout is declared here.
 */
#ifndef EDGEXPU_KERNELS_H
#define EDGEXPU_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#include "edgexpu_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids: include/edgexpu/gguf_quant.h:17-24 */
#ifndef EDGEXPU_GGUF_TYPE_F32
#define EDGEXPU_GGUF_TYPE_F32 0
#define EDGEXPU_GGUF_TYPE_F16 1
#define EDGEXPU_GGUF_TYPE_Q4_0 2
#define EDGEXPU_GGUF_TYPE_Q5_0 6
#define EDGEXPU_GGUF_TYPE_Q8_0 8
#define EDGEXPU_GGUF_TYPE_Q4_K 12
#define EDGEXPU_GGUF_TYPE_Q5_K 13
#define EDGEXPU_GGUF_TYPE_Q6_K 14
#endif

/* ---- layout constants (pure arithmetic) ---- */
size_t edgexpu_gguf_type_block_size(uint32_t type);   /* gguf_quant.h:26, src/gguf_quant.c:69-85 */
size_t edgexpu_gguf_type_block_bytes(uint32_t type);  /* gguf_quant.h:27, src/gguf_quant.c:87-108 */
size_t edgexpu_gguf_row_bytes(uint32_t type, int n);  /* gguf_quant.h:69, src/gguf_quant.c:468-480 */
size_t edgexpu_gguf_q8_0_nbytes(int n);               /* gguf_quant.h:80, src/gguf_dot_q8.c:255-260 */
size_t edgexpu_gguf_q8_k_nbytes(int n);               /* gguf_quant.h:85, src/gguf_dot_q8.c:262-267 */
int edgexpu_gguf_can_dot_q8(uint32_t type);           /* gguf_quant.h:82, src/gguf_dot_q8.c:414-423 */
int edgexpu_gguf_can_dot_q8k(uint32_t type);          /* gguf_quant.h:87, src/gguf_dot_q8.c:425-434 */

#ifndef EDGEXPU_GGUF_H
/* include/edgexpu/gguf.h:19-27: one entry of the GGUF tensor table, same
 * field order and types (name, n_dims, type, dims, data offset). */
#define EDGEXPU_GGUF_TENSOR_NAME 96
typedef struct edgexpu_gguf_tensor {
    char name[EDGEXPU_GGUF_TENSOR_NAME];
    uint32_t n_dims;
    uint32_t type;
    uint64_t dims[4];
    uint64_t offset;
} edgexpu_gguf_tensor;
#endif

/* include/edgexpu/gguf_quant.h:28-29 (src/gguf_quant.c:110-136): element
 * count (product of dims) and block bytes of a tensor; 0 for NULL, unknown
 * types or counts that are not whole blocks. */
uint64_t edgexpu_gguf_tensor_elements(const edgexpu_gguf_tensor *tensor);
size_t edgexpu_gguf_tensor_nbytes(const edgexpu_gguf_tensor *tensor);

/* ---- GPU entry points with the reference signatures ---- */

/* include/edgexpu/gguf_quant.h:32-39 (src/gguf_quant.c:355-411): returns 1 on
 * success, 0 with a message in `error` otherwise. */
int edgexpu_gguf_dequantize(const uint8_t *src, uint32_t type, uint64_t n_elements, float *dst, char *error,
                            size_t error_size);

/* include/edgexpu/gguf_quant.h:42-57 (src/gguf_quant.c:413-466): one row of
 * an [rows x n_embd] matrix (the embedding lookup of src/native.c:428-443),
 * bit-identical to the reference.  _q8_0_rows: Q8_0 rows, returns 0 for bad
 * arguments; _row: any type, with the reference's checks and messages (row
 * width, row range, byte split).  Device-resident tables use
 * edgexpu_hip_embed_rows_dev, which gathers many rows in one launch. */
int edgexpu_gguf_dequantize_q8_0_rows(const uint8_t *src, uint64_t row, int n_embd, float *dst);
int edgexpu_gguf_dequantize_row(const uint8_t *src, const edgexpu_gguf_tensor *tensor, uint64_t row, int n_embd,
                                float *dst, char *error, size_t error_size);

/* include/edgexpu/gguf_quant.h:58-63 (src/gguf_quant.c:920-932): the f32 dot
 * of row `row` of a Q8_0 matrix with x; 0.0f for bad arguments. */
float edgexpu_gguf_q8_0_dot_row(const uint8_t *src, uint64_t row, int n_embd, const float *x);

/* include/edgexpu/gguf_quant.h:103 (src/gguf_quant.c:934-1061): the
 * reference's known-answer checks (Q4_K, Q4_0, F16, Q5_K f32 dots; Q8_0 and
 * Q5_0 integer dots) run through this kernel set on the GPU; 1 when all pass,
 * else 0 with the failing check in `error`. */
int edgexpu_gguf_quant_selftest(char *error, size_t error_size);

/* include/edgexpu/gguf_quant.h:81,86 (src/gguf_dot_q8.c:269-412): reference
 * block bytes, bit-identical to the reference's x86 build. */
int edgexpu_gguf_quantize_q8_0(const float *x, int n, uint8_t *dst);
int edgexpu_gguf_quantize_q8_k(const float *x, int n, uint8_t *dst);

/* include/edgexpu/gguf_quant.h:72-77,90-102 (src/gguf_quant.c:894-918,
 * src/gguf_dot_q8.c:1004-1044): one row per call, on the GPU.  Correct, but
 * each call is a device round trip: two host-to-device copies, one launch,
 * one device-to-host copy and a stream synchronisation: 32-41 us per call
 * measured on MI355X for Q8_0 [576], Q6_K [2560], F32 and Q4_K [4096] rows,
 * whatever the row length (a 4096-element Q4_K row is about 1 us of one CPU
 * core's work).  A loop over the rows of a matrix (the
 * reference's logit_score, src/native.c:500-514) belongs on
 * edgexpu_hip_logits / edgexpu_hip_dot_*_rows or the linear entry points,
 * which take all rows in one call. */
float edgexpu_gguf_dot_quant(uint32_t type, const uint8_t *row, const float *x, int n);
float edgexpu_gguf_dot_quant_q8(uint32_t type, const uint8_t *wrow, const uint8_t *x_q8, int n);
float edgexpu_gguf_dot_quant_q8k(uint32_t type, const uint8_t *wrow, const uint8_t *x_q8k, int n);

/* include/edgexpu/cpu_kernel.h:60-67,71-80 (src/cpu_kernel.c:545-656):
 * out[t*n_out + o] = bias[o] + W[o]·q8(x[t]).  Returns silently on bad
 * arguments like the reference.  When `weight` was registered with
 * edgexpu_kernels_register_weight the device-resident copy is used; otherwise
 * the rows are uploaded for the call. */
void edgexpu_cpu_linear_quant(float *out, const float *x, const uint8_t *weight, uint32_t type, const float *bias,
                              int n_out, int n_in);
void edgexpu_cpu_linear_quant_batch(float *out, const float *x, const uint8_t *weight, uint32_t type,
                                    const float *bias, int m, int n_out, int n_in);

/* include/edgexpu/cpu_kernel.h:24 (src/cpu_kernel.c:328-353): softmax in
 * place; and include/edgexpu/cpu_kernel.h:86-94 (src/cpu_kernel.c:762-849):
 * softmax in place, then one draw (top_p in (0,1): nucleus) with the
 * reference's xorshift state *rng.  Returns 0 on bad arguments, 1 otherwise.
 * Computed on the GPU, for n <= 2^24 (16 777 216, a vocabulary 100 times the
 * largest in use): a larger n, or a failing GPU call, leaves io / logits as
 * given (edgexpu_cpu_softmax cannot return a status; the sticky error of
 * edgexpu_hip_last_error() names the cause) and edgexpu_cpu_sample_softmax
 * returns 0, where the reference would normalise. */
void edgexpu_cpu_softmax(float *io, int n);
int edgexpu_cpu_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out);

/* ---- device residency for host-pointer callers (no reference counterpart:
 * replaces the per-token staging copies of src/native.c:350-380) ---- */

/* Uploads n_out rows at `blocks` (and `bias`, may be NULL) once; later linear
 * calls passing the same (blocks, type, n_out, n_in, bias) use the device copy.
 * The caller promises the bytes do not change while registered (the
 * reference's reused weight_stage buffer must NOT be registered).  Returns 1
 * on success. */
int edgexpu_kernels_register_weight(const uint8_t *blocks, uint32_t type, int n_out, int n_in, const float *bias);
/* Drops the device copy registered for `blocks`; returns 1 if one existed. */
int edgexpu_kernels_unregister_weight(const uint8_t *blocks);
/* Device handle registered for `blocks`, or NULL. */
const edgexpu_hip_weight *edgexpu_kernels_lookup_weight(const uint8_t *blocks);

/* ---- edgexpu_layer_kind dispatch (include/edgexpu/arch.h:28-33) ---- */
#ifndef EDGEXPU_ARCH_H
typedef enum edgexpu_layer_kind {
    EDGEXPU_LAYER_ATTN_SWIGLU = 0,
    EDGEXPU_LAYER_UNSUPPORTED = 1,
    EDGEXPU_LAYER_GATED_DELTA = 2,
    EDGEXPU_LAYER_ATTN_QK_NORM = 3
} edgexpu_layer_kind;
#endif

/* Projection slots of edgexpu_native_layer (include/edgexpu/native.h:30-73)
 * that go through the matrix path. */
typedef enum edgexpu_proj_slot {
    EDGEXPU_PROJ_WQ = 0,
    EDGEXPU_PROJ_WK,
    EDGEXPU_PROJ_WV,
    EDGEXPU_PROJ_WO,
    EDGEXPU_PROJ_WGATE,
    EDGEXPU_PROJ_WUP,
    EDGEXPU_PROJ_WDOWN,
    EDGEXPU_PROJ_WQKV,
    EDGEXPU_PROJ_WATTN_GATE,
    EDGEXPU_PROJ_WSSM_ALPHA,
    EDGEXPU_PROJ_WSSM_BETA,
    EDGEXPU_PROJ_WSSM_OUT,
    EDGEXPU_PROJ_COUNT
} edgexpu_proj_slot;

/* Writes, in call order, the slots a decode step of a layer of `kind` runs
 * through edgexpu_cpu_linear_quant (src/native.c:2487-2581 and the layer
 * bodies at :1557-1565, :1660-1710, :1792-1895); returns the count, 0 for
 * EDGEXPU_LAYER_UNSUPPORTED or an unknown kind. */
int edgexpu_kernels_layer_projections(int kind, edgexpu_proj_slot *slots, int max_slots);

/* The kernel set as a function table, for hosts that select kernels at run
 * time instead of at link time. */
typedef struct edgexpu_kernel_set {
    const char *name;
    void (*linear_quant)(float *, const float *, const uint8_t *, uint32_t, const float *, int, int);
    void (*linear_quant_batch)(float *, const float *, const uint8_t *, uint32_t, const float *, int, int, int);
    int (*dequantize)(const uint8_t *, uint32_t, uint64_t, float *, char *, size_t);
    int (*quantize_q8_0)(const float *, int, uint8_t *);
    int (*quantize_q8_k)(const float *, int, uint8_t *);
    float (*dot_quant)(uint32_t, const uint8_t *, const float *, int);
    float (*dot_quant_q8)(uint32_t, const uint8_t *, const uint8_t *, int);
    float (*dot_quant_q8k)(uint32_t, const uint8_t *, const uint8_t *, int);
} edgexpu_kernel_set;

const edgexpu_kernel_set *edgexpu_kernels_hip(void);

#ifdef __cplusplus
}
#endif

#endif
