/*
 * libedgexpu_kernels.so: the reference's quantized-weight entry points
 * (include/edgexpu/cpu_kernel.h:60-80, include/edgexpu/gguf_quant.h:26-102)
 * re-implemented as a C11 host layer over libedgexpu_hip.so.  Argument
 * checks and error strings follow the reference; every computation runs on
 * the GPU.
 */
#include "edgexpu_kernels.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void set_msg(char *error, size_t error_size, const char *msg) {
    if (error != NULL && error_size > 0) {
        snprintf(error, error_size, "%s", msg);
    }
}

/* ------------------------------------------------------------ layouts */

size_t edgexpu_gguf_type_block_size(uint32_t type) {
    switch (type) {
        case EDGEXPU_GGUF_TYPE_F32:
        case EDGEXPU_GGUF_TYPE_F16:
            return 1;
        case EDGEXPU_GGUF_TYPE_Q4_0:
        case EDGEXPU_GGUF_TYPE_Q5_0:
        case EDGEXPU_GGUF_TYPE_Q8_0:
            return 32;
        case EDGEXPU_GGUF_TYPE_Q4_K:
        case EDGEXPU_GGUF_TYPE_Q5_K:
        case EDGEXPU_GGUF_TYPE_Q6_K:
            return 256;
        default:
            return 0;
    }
}

size_t edgexpu_gguf_type_block_bytes(uint32_t type) {
    switch (type) {
        case EDGEXPU_GGUF_TYPE_F32: return 4;
        case EDGEXPU_GGUF_TYPE_F16: return 2;
        case EDGEXPU_GGUF_TYPE_Q4_0: return 18;
        case EDGEXPU_GGUF_TYPE_Q5_0: return 22;
        case EDGEXPU_GGUF_TYPE_Q8_0: return 34;
        case EDGEXPU_GGUF_TYPE_Q4_K: return 144;
        case EDGEXPU_GGUF_TYPE_Q5_K: return 176;
        case EDGEXPU_GGUF_TYPE_Q6_K: return 210;
        default: return 0;
    }
}

size_t edgexpu_gguf_row_bytes(uint32_t type, int n) {
    size_t bs;
    size_t bb;
    if (n <= 0) {
        return 0;
    }
    bs = edgexpu_gguf_type_block_size(type);
    bb = edgexpu_gguf_type_block_bytes(type);
    if (bs == 0 || bb == 0 || (size_t)n % bs != 0) {
        return 0;
    }
    return (size_t)n / bs * bb;
}

size_t edgexpu_gguf_q8_0_nbytes(int n) {
    return (n <= 0 || n % 32 != 0) ? 0 : (size_t)n / 32 * 34;
}

size_t edgexpu_gguf_q8_k_nbytes(int n) {
    return (n <= 0 || n % 256 != 0) ? 0 : (size_t)n / 256 * 292;
}

int edgexpu_gguf_can_dot_q8(uint32_t type) {
    return type == EDGEXPU_GGUF_TYPE_Q4_0 || type == EDGEXPU_GGUF_TYPE_Q5_0 || type == EDGEXPU_GGUF_TYPE_Q8_0;
}

int edgexpu_gguf_can_dot_q8k(uint32_t type) {
    return type == EDGEXPU_GGUF_TYPE_Q4_K || type == EDGEXPU_GGUF_TYPE_Q5_K || type == EDGEXPU_GGUF_TYPE_Q6_K;
}

/* ------------------------------------------------------------ registry */

typedef struct reg_entry {
    const uint8_t *blocks;
    const float *bias;
    uint32_t type;
    int n_out;
    int n_in;
    edgexpu_hip_weight *w;
    struct reg_entry *next;
} reg_entry;

static reg_entry *g_registry;

static reg_entry *reg_find(const uint8_t *blocks) {
    reg_entry *e;
    for (e = g_registry; e != NULL; e = e->next) {
        if (e->blocks == blocks) {
            return e;
        }
    }
    return NULL;
}

int edgexpu_kernels_register_weight(const uint8_t *blocks, uint32_t type, int n_out, int n_in, const float *bias) {
    reg_entry *e;
    edgexpu_hip_weight *w;
    if (blocks == NULL || reg_find(blocks) != NULL) {
        return 0;
    }
    w = edgexpu_hip_weight_upload(blocks, type, n_out, n_in, bias);
    if (w == NULL) {
        return 0;
    }
    e = (reg_entry *)calloc(1, sizeof(*e));
    if (e == NULL) {
        edgexpu_hip_weight_free(w);
        return 0;
    }
    e->blocks = blocks;
    e->bias = bias;
    e->type = type;
    e->n_out = n_out;
    e->n_in = n_in;
    e->w = w;
    e->next = g_registry;
    g_registry = e;
    return 1;
}

int edgexpu_kernels_unregister_weight(const uint8_t *blocks) {
    reg_entry **pp;
    for (pp = &g_registry; *pp != NULL; pp = &(*pp)->next) {
        if ((*pp)->blocks == blocks) {
            reg_entry *e = *pp;
            *pp = e->next;
            edgexpu_hip_weight_free(e->w);
            free(e);
            return 1;
        }
    }
    return 0;
}

const edgexpu_hip_weight *edgexpu_kernels_lookup_weight(const uint8_t *blocks) {
    reg_entry *e = reg_find(blocks);
    return e != NULL ? e->w : NULL;
}

uint64_t edgexpu_gguf_tensor_elements(const edgexpu_gguf_tensor *tensor) {
    uint64_t n = 1;
    uint32_t i;
    if (tensor == NULL) {
        return 0;
    }
    for (i = 0; i < tensor->n_dims && i < 4; i++) {
        n *= tensor->dims[i];
    }
    return n;
}

size_t edgexpu_gguf_tensor_nbytes(const edgexpu_gguf_tensor *tensor) {
    uint64_t n;
    size_t bs;
    size_t bb;
    if (tensor == NULL) {
        return 0;
    }
    n = edgexpu_gguf_tensor_elements(tensor);
    bs = edgexpu_gguf_type_block_size(tensor->type);
    bb = edgexpu_gguf_type_block_bytes(tensor->type);
    if (bs == 0 || bb == 0 || n % bs != 0) {
        return 0;
    }
    return (size_t)(n / bs) * bb;
}

/* ------------------------------------------------------------ dequant */

int edgexpu_gguf_dequantize(const uint8_t *src, uint32_t type, uint64_t n_elements, float *dst, char *error,
                            size_t error_size) {
    size_t bs;
    char msg[256];
    if (src == NULL || dst == NULL || n_elements == 0) {
        set_msg(error, error_size, "dequantize 参数为空");
        return 0;
    }
    bs = edgexpu_gguf_type_block_size(type);
    if (bs == 0 || n_elements % bs != 0) {
        set_msg(error, error_size, "不支持的 GGUF 量化类型或元素数不对齐");
        return 0;
    }
    if (!edgexpu_hip_supports_type(type)) {
        snprintf(msg, sizeof(msg), "GGUF type %u is not supported (F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)", type);
        set_msg(error, error_size, msg);
        return 0;
    }
    if (!edgexpu_hip_dequantize(src, type, n_elements, dst)) {
        edgexpu_hip_last_error(msg, sizeof(msg));
        set_msg(error, error_size, msg);
        return 0;
    }
    return 1;
}

int edgexpu_gguf_dequantize_q8_0_rows(const uint8_t *src, uint64_t row, int n_embd, float *dst) {
    size_t rb;
    if (src == NULL || dst == NULL || n_embd <= 0 || n_embd % 32 != 0) {
        return 0; /* src/gguf_quant.c:420-422 */
    }
    rb = (size_t)(n_embd / 32) * 34;
    return edgexpu_gguf_dequantize(src + row * rb, EDGEXPU_GGUF_TYPE_Q8_0, (uint64_t)n_embd, dst, NULL, 0);
}

int edgexpu_gguf_dequantize_row(const uint8_t *src, const edgexpu_gguf_tensor *tensor, uint64_t row, int n_embd,
                                float *dst, char *error, size_t error_size) {
    uint64_t n;
    uint64_t rows;
    size_t nbytes;
    /* the checks and messages of src/gguf_quant.c:442-463 */
    if (src == NULL || tensor == NULL || dst == NULL || n_embd <= 0) {
        set_msg(error, error_size, "dequantize_row 参数为空");
        return 0;
    }
    n = edgexpu_gguf_tensor_elements(tensor);
    if (n == 0 || n % (uint64_t)n_embd != 0) {
        set_msg(error, error_size, "tensor 行宽与 embedding_length 不匹配");
        return 0;
    }
    rows = n / (uint64_t)n_embd;
    if (row >= rows) {
        set_msg(error, error_size, "tensor 行越界");
        return 0;
    }
    if (tensor->type == EDGEXPU_GGUF_TYPE_Q8_0) {
        return edgexpu_gguf_dequantize_q8_0_rows(src, row, n_embd, dst);
    }
    nbytes = edgexpu_gguf_tensor_nbytes(tensor);
    if (nbytes == 0 || nbytes % rows != 0) {
        set_msg(error, error_size, "tensor 字节数无法按行切分");
        return 0;
    }
    return edgexpu_gguf_dequantize(src + row * (nbytes / rows), tensor->type, (uint64_t)n_embd, dst, error,
                                   error_size);
}

/* ------------------------------------------------------------ quantizers */

int edgexpu_gguf_quantize_q8_0(const float *x, int n, uint8_t *dst) {
    if (x == NULL || dst == NULL || n <= 0 || n % 32 != 0) {
        return 0;
    }
    return edgexpu_hip_quantize_q8_0(x, n, dst);
}

int edgexpu_gguf_quantize_q8_k(const float *x, int n, uint8_t *dst) {
    if (x == NULL || dst == NULL || n <= 0 || n % 256 != 0) {
        return 0;
    }
    return edgexpu_hip_quantize_q8_k(x, n, dst);
}

/* ------------------------------------------------------------ row dots */

float edgexpu_gguf_dot_quant(uint32_t type, const uint8_t *row, const float *x, int n) {
    float out = 0.0f;
    if (row == NULL || x == NULL || n <= 0 || edgexpu_gguf_row_bytes(type, n) == 0) {
        return 0.0f;
    }
    if (!edgexpu_hip_supports_type(type) || !edgexpu_hip_dot_f32_rows(&out, row, type, x, 1, n)) {
        return 0.0f;
    }
    return out;
}

float edgexpu_gguf_q8_0_dot_row(const uint8_t *src, uint64_t row, int n_embd, const float *x) {
    if (src == NULL || x == NULL || n_embd <= 0 || n_embd % 32 != 0) {
        return 0.0f; /* src/gguf_quant.c:927-929 */
    }
    return edgexpu_gguf_dot_quant(EDGEXPU_GGUF_TYPE_Q8_0, src + row * edgexpu_gguf_row_bytes(EDGEXPU_GGUF_TYPE_Q8_0,
                                                                                             n_embd),
                                  x, n_embd);
}

float edgexpu_gguf_dot_quant_q8(uint32_t type, const uint8_t *wrow, const uint8_t *x_q8, int n) {
    float out = 0.0f;
    if (wrow == NULL || x_q8 == NULL || n <= 0 || n % 32 != 0) {
        return 0.0f;
    }
    /* the Q8_0-activation family of src/gguf_dot_q8.c:1004-1023 */
    if ((type != EDGEXPU_GGUF_TYPE_Q8_0 && type != EDGEXPU_GGUF_TYPE_Q4_0 && type != EDGEXPU_GGUF_TYPE_Q5_0) ||
        !edgexpu_hip_dot_q8_rows(&out, wrow, type, x_q8, 1, n)) {
        return 0.0f;
    }
    return out;
}

float edgexpu_gguf_dot_quant_q8k(uint32_t type, const uint8_t *wrow, const uint8_t *x_q8k, int n) {
    float out = 0.0f;
    if (wrow == NULL || x_q8k == NULL || n <= 0 || n % 256 != 0) {
        return 0.0f;
    }
    /* the Q8_K-activation family of src/gguf_dot_q8.c:1025-1044 */
    if ((type != EDGEXPU_GGUF_TYPE_Q4_K && type != EDGEXPU_GGUF_TYPE_Q5_K && type != EDGEXPU_GGUF_TYPE_Q6_K) ||
        !edgexpu_hip_dot_q8_rows(&out, wrow, type, x_q8k, 1, n)) {
        return 0.0f;
    }
    return out;
}

/* ---------------------------------------------------------- sampling */

void edgexpu_cpu_softmax(float *io, int n) {
    if (io == NULL || n <= 0) {
        return; /* src/cpu_kernel.c:333-335 */
    }
    (void)edgexpu_hip_softmax(io, n);
}

int edgexpu_cpu_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out) {
    if (logits == NULL || rng == NULL || out == NULL || n <= 0) {
        return 0; /* src/cpu_kernel.c:776-778 */
    }
    return edgexpu_hip_sample_softmax(logits, n, top_p, rng, out);
}

/* ------------------------------------------------------------ linear */

void edgexpu_cpu_linear_quant_batch(float *out, const float *x, const uint8_t *weight, uint32_t type,
                                    const float *bias, int m, int n_out, int n_in) {
    reg_entry *e;
    if (out == NULL || x == NULL || weight == NULL || m <= 0 || n_out <= 0 || n_in <= 0) {
        return; /* src/cpu_kernel.c:562-564 */
    }
    if (edgexpu_gguf_row_bytes(type, n_in) == 0) {
        return; /* src/cpu_kernel.c:571-574 */
    }
    /* every type with a row layout runs on the GPU, F32 included (its
     * one-token sum starts at the bias in double, src/cpu_kernel.c:566-569) */
    e = reg_find(weight);
    if (e != NULL && e->type == type && e->n_out == n_out && e->n_in == n_in && e->bias == bias) {
        edgexpu_hip_linear_quant_batch(out, x, e->w, m);
        return;
    }
    edgexpu_hip_linear_quant_batch_host(out, x, weight, type, bias, m, n_out, n_in);
}

void edgexpu_cpu_linear_quant(float *out, const float *x, const uint8_t *weight, uint32_t type, const float *bias,
                              int n_out, int n_in) {
    edgexpu_cpu_linear_quant_batch(out, x, weight, type, bias, 1, n_out, n_in);
}

/* ------------------------------------------------------------ layer kinds */

int edgexpu_kernels_layer_projections(int kind, edgexpu_proj_slot *slots, int max_slots) {
    static const edgexpu_proj_slot swiglu[] = {
        EDGEXPU_PROJ_WQ, EDGEXPU_PROJ_WK, EDGEXPU_PROJ_WV, EDGEXPU_PROJ_WO,
        EDGEXPU_PROJ_WGATE, EDGEXPU_PROJ_WUP, EDGEXPU_PROJ_WDOWN};
    static const edgexpu_proj_slot delta[] = {
        EDGEXPU_PROJ_WQKV, EDGEXPU_PROJ_WATTN_GATE, EDGEXPU_PROJ_WSSM_ALPHA, EDGEXPU_PROJ_WSSM_BETA,
        EDGEXPU_PROJ_WSSM_OUT, EDGEXPU_PROJ_WGATE, EDGEXPU_PROJ_WUP, EDGEXPU_PROJ_WDOWN};
    const edgexpu_proj_slot *src;
    int n;
    int i;
    switch (kind) {
        case EDGEXPU_LAYER_ATTN_SWIGLU:
        case EDGEXPU_LAYER_ATTN_QK_NORM: /* q (with its gate half), k, v, o, then the FFN */
            src = swiglu;
            n = (int)(sizeof(swiglu) / sizeof(swiglu[0]));
            break;
        case EDGEXPU_LAYER_GATED_DELTA:
            src = delta;
            n = (int)(sizeof(delta) / sizeof(delta[0]));
            break;
        default:
            return 0;
    }
    if (slots == NULL || max_slots < n) {
        return slots == NULL ? n : 0;
    }
    for (i = 0; i < n; i++) {
        slots[i] = src[i];
    }
    return n;
}

static const edgexpu_kernel_set g_hip_set = {
    "hip.gfx950",
    edgexpu_cpu_linear_quant,
    edgexpu_cpu_linear_quant_batch,
    edgexpu_gguf_dequantize,
    edgexpu_gguf_quantize_q8_0,
    edgexpu_gguf_quantize_q8_k,
    edgexpu_gguf_dot_quant,
    edgexpu_gguf_dot_quant_q8,
    edgexpu_gguf_dot_quant_q8k,
};

const edgexpu_kernel_set *edgexpu_kernels_hip(void) {
    return &g_hip_set;
}

/* ------------------------------------------------------------ self-test */

/* The known-answer checks of src/gguf_quant.c:934-1061, each built here and
 * run through this kernel set (so on the GPU). */
int edgexpu_gguf_quant_selftest(char *error, size_t error_size) {
    const uint16_t one = 0x3c00; /* fp16 1.0 */
    const uint16_t two = 0x4000; /* fp16 2.0 */
    char msg[160];
    float fused;
    int i;
    { /* Q4_K: d = 1, sc0 = 1, code 2 at element 0; x[0] = 3 -> 6 */
        uint8_t blk[144];
        float x[256];
        memset(blk, 0, sizeof(blk));
        memset(x, 0, sizeof(x));
        memcpy(blk, &one, 2);
        blk[4] = 1;
        blk[16] = 0x02;
        x[0] = 3.0f;
        fused = edgexpu_gguf_dot_quant(EDGEXPU_GGUF_TYPE_Q4_K, blk, x, 256);
        if (!(fused > 6.0f - 1e-3f && fused < 6.0f + 1e-3f)) {
            snprintf(msg, sizeof(msg), "q4_k fused dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
    }
    { /* Q4_0: low nibble 9 (value 1) at element 0; x[0] = 3 -> 3 */
        uint8_t blk[18];
        float x[32];
        memset(blk, 0, sizeof(blk));
        memset(x, 0, sizeof(x));
        memcpy(blk, &one, 2);
        for (i = 0; i < 16; i++) {
            blk[2 + i] = 0x88; /* value 0 */
        }
        blk[2] = 0x89;
        x[0] = 3.0f;
        fused = edgexpu_gguf_dot_quant(EDGEXPU_GGUF_TYPE_Q4_0, blk, x, 32);
        if (!(fused > 3.0f - 1e-3f && fused < 3.0f + 1e-3f)) {
            snprintf(msg, sizeof(msg), "q4_0 fused dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
    }
    { /* F16: {1, 2} . {2, 3} = 8 */
        uint8_t h[64];
        float x[32];
        memset(h, 0, sizeof(h));
        memset(x, 0, sizeof(x));
        memcpy(h, &one, 2);
        memcpy(h + 2, &two, 2);
        x[0] = 2.0f;
        x[1] = 3.0f;
        fused = edgexpu_gguf_dot_quant(EDGEXPU_GGUF_TYPE_F16, h, x, 32);
        if (!(fused > 8.0f - 1e-3f && fused < 8.0f + 1e-3f)) {
            snprintf(msg, sizeof(msg), "f16 fused dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
    }
    { /* Q5_K: d = 1, sc0 = 1, code 2 at element 0; x[0] = 3 -> 6 */
        uint8_t blk[176];
        float x[256];
        memset(blk, 0, sizeof(blk));
        memset(x, 0, sizeof(x));
        memcpy(blk, &one, 2);
        blk[4] = 1;
        blk[48] = 0x02;
        x[0] = 3.0f;
        fused = edgexpu_gguf_dot_quant(EDGEXPU_GGUF_TYPE_Q5_K, blk, x, 256);
        if (!(fused > 6.0f - 1e-3f && fused < 6.0f + 1e-3f)) {
            snprintf(msg, sizeof(msg), "q5_k fused dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
    }
    { /* Q8_0 x Q8_0: all-ones codes, d = 1, x = 1 -> 32; Q5_0 zero codes -> -512 */
        uint8_t w[34];
        uint8_t xq[34];
        float x[32];
        for (i = 0; i < 32; i++) {
            x[i] = 1.0f;
        }
        memset(w, 0, sizeof(w));
        memcpy(w, &one, 2);
        for (i = 0; i < 32; i++) {
            w[2 + i] = 1;
        }
        if (!edgexpu_gguf_quantize_q8_0(x, 32, xq)) {
            set_msg(error, error_size, "q8_0 quantize selftest failed");
            return 0;
        }
        fused = edgexpu_gguf_dot_quant_q8(EDGEXPU_GGUF_TYPE_Q8_0, w, xq, 32);
        if (!(fused > 32.0f - 0.5f && fused < 32.0f + 0.5f)) {
            snprintf(msg, sizeof(msg), "q8_0 integer dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
        memset(w, 0, 22);
        memcpy(w, &one, 2);
        fused = edgexpu_gguf_dot_quant_q8(EDGEXPU_GGUF_TYPE_Q5_0, w, xq, 32);
        if (!(fused > -512.0f - 1.0f && fused < -512.0f + 1.0f)) {
            snprintf(msg, sizeof(msg), "q5_0 integer dot selftest failed fused=%.6f", fused);
            set_msg(error, error_size, msg);
            return 0;
        }
    }
    return 1;
}
