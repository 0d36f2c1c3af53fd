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
        snprintf(msg, sizeof(msg), "GGUF type %u is not on the GPU path (F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)", type);
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
    if (!edgexpu_hip_supports_type(type)) {
        /* refuse explicitly: the caller keeps its CPU kernel for this type */
        edgexpu_hip_linear_quant_batch_host(out, x, weight, type, bias, m, n_out, n_in);
        return;
    }
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
