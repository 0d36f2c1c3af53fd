/* Test infrastructure only: a driver that runs the logits product of the
 * reference's greedy decode step (src/native.c:2292-2401) on the reference's
 * own row kernels, linked into oracle/_ref/libedgexpu_ref.so beside them.
 *
 * The reference keeps this loop inside a static function of src/native.c
 * (sample_next_token), which needs the whole session/GGUF/tokenizer machinery
 * to build; the loop itself is short, so it is stated here over the exported
 * row kernels of src/gguf_quant.c and src/gguf_dot_q8.c:
 *   - the hidden state goes through edgexpu_gguf_quantize_q8_0 when
 *     edgexpu_gguf_can_dot_q8(type) (src/native.c:2317-2319, 483-498), and each
 *     row then through edgexpu_gguf_dot_quant_q8 (src/native.c:464-481),
 *     otherwise through edgexpu_gguf_dot_quant on the f32 hidden state
 *     (src/native.c:445-462);
 *   - the output bias is added to the row dot (src/native.c:500-514);
 *   - rows are taken in chunks of chunk_rows (0 = the 48 MiB output-chunk
 *     budget of include/edgexpu/scheduler.h:34 over the row bytes,
 *     src/native.c:2262-2274), each chunk an OpenMP static loop with a
 *     per-thread best merged under a critical section, lowest index on ties,
 *     parallel only for chunks of 256 rows or more (src/native.c:2358-2391).
 * Returns the argmax; scores (optional) receives every row's score. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "edgexpu/gguf_quant.h"

#define REFDRV_CHUNK_BYTES ((size_t)48u * 1024u * 1024u)

uint32_t edgexpu_refdrv_logits(float *scores, const float *hidden, const uint8_t *w, uint32_t type,
                               const float *bias, int vocab, int n_embd, size_t chunk_rows) {
    size_t rb = edgexpu_gguf_row_bytes(type, n_embd);
    uint8_t *xq = NULL;
    uint32_t best = 0;
    float best_score = -INFINITY;
    uint32_t begin;
    if (rb == 0 || vocab <= 0 || hidden == NULL || w == NULL) {
        return 0;
    }
    if (edgexpu_gguf_can_dot_q8(type)) {
        xq = (uint8_t *)malloc(edgexpu_gguf_q8_0_nbytes(n_embd));
        if (xq != NULL && !edgexpu_gguf_quantize_q8_0(hidden, n_embd, xq)) {
            free(xq);
            xq = NULL;
        }
    }
    if (chunk_rows == 0) {
        chunk_rows = REFDRV_CHUNK_BYTES / rb;
        if (chunk_rows < 1) {
            chunk_rows = 1;
        }
    }
    for (begin = 0; begin < (uint32_t)vocab; begin += (uint32_t)chunk_rows) {
        uint32_t end = begin + (uint32_t)chunk_rows;
        if (end > (uint32_t)vocab) {
            end = (uint32_t)vocab;
        }
#pragma omp parallel if ((end - begin) >= 256)
        {
            uint32_t lbest = 0;
            float lscore = -INFINITY;
            int i;
#pragma omp for nowait schedule(static)
            for (i = (int)begin; i < (int)end; i++) {
                const uint8_t *row = w + (size_t)i * rb;
                float s = xq != NULL ? edgexpu_gguf_dot_quant_q8(type, row, xq, n_embd)
                                     : edgexpu_gguf_dot_quant(type, row, hidden, n_embd);
                if (bias != NULL) {
                    s += bias[i];
                }
                if (scores != NULL) {
                    scores[i] = s;
                }
                if (s > lscore) {
                    lscore = s;
                    lbest = (uint32_t)i;
                }
            }
#pragma omp critical
            {
                if (lscore > best_score || (lscore == best_score && lbest < best)) {
                    best_score = lscore;
                    best = lbest;
                }
            }
        }
    }
    free(xq);
    return best;
}
