/*
 * Device-resident GGUF blocks for the quantized-weight path.
 *
 * The reference maps the GGUF file (src/native.c:115-178) and, per layer and
 * per token, copies each weight tensor into a reused staging buffer before
 * its matvec (stage_copy_bytes, src/native.c:350-380, reached from
 * load_qweight, src/native.c:593-655).  This header replaces that with one
 * upload per model:
 *
 *   - edgexpu_gguf_up_read_table reads the file's GGUF v3 tensor directory
 *     (the table edgexpu_gguf_load builds in src/gguf.c:359-610): header,
 *     every metadata key/value skipped by type, the tensor infos, and the
 *     data section offset, which is the end of the infos rounded up to 32
 *     as src/gguf.c:595 computes it (a general.alignment key is reported in
 *     the table but, as in the reference, not applied: a file whose writer
 *     padded to 64 is read where the reference reads it);
 *   - edgexpu_gguf_device_upload copies the whole data section to the GPU
 *     once (one allocation holding the file's own bytes, so tensor t lives at
 *     base + t.offset, unchanged from the file), and
 *     edgexpu_gguf_device_weight hands out weight handles over it with the
 *     shape checks of load_qweight (element count n_out * n_in, a known
 *     block layout for rows of n_in).
 *
 * Host C (libedgexpu_kernels.so); the device copy goes through
 * libedgexpu_hip.so.  Not reentrant, like the rest of the library.
 */
#ifndef EDGEXPU_GGUF_UPLOAD_H
#define EDGEXPU_GGUF_UPLOAD_H

#include <stddef.h>
#include <stdint.h>

#include "edgexpu_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define EDGEXPU_GGUF_UP_NAME 96 /* the reference's EDGEXPU_GGUF_TENSOR_NAME (include/edgexpu/gguf.h:19) */

/* One tensor info (include/edgexpu/gguf.h:21-27) plus its byte size. */
typedef struct edgexpu_gguf_up_tensor {
    char name[EDGEXPU_GGUF_UP_NAME]; /* truncated like the reference's read_string_into */
    uint32_t n_dims;
    uint32_t type;     /* GGUF type id (gguf_quant.h:17-24) */
    uint64_t dims[4];  /* dims[0] = row length, dims[1] = rows for matrices */
    uint64_t offset;   /* bytes from the data section start */
    uint64_t nbytes;   /* elements / block size * block bytes; 0 for a type without a block layout here */
} edgexpu_gguf_up_tensor;

typedef struct edgexpu_gguf_up_table {
    uint32_t version;
    uint32_t alignment;     /* general.alignment as declared (32 when absent); not applied */
    uint64_t tensor_count;
    uint64_t kv_count;
    uint64_t data_offset;   /* file offset of the data section */
    uint64_t file_size;
    uint32_t n_tensors;
    edgexpu_gguf_up_tensor *tensors;
} edgexpu_gguf_up_table;

/* Reads the tensor table of the GGUF v3 file at path.  1 on success; 0 and a
 * message in error otherwise (not a GGUF file, unsupported version, a
 * truncated header or table, more than 4 dims, a tensor whose element count
 * or byte size overflows 64 bits, a tensor whose bytes lie past the end of
 * the file).  Free with edgexpu_gguf_up_table_free. */
int edgexpu_gguf_up_read_table(const char *path, edgexpu_gguf_up_table *table, char *error, size_t error_size);
void edgexpu_gguf_up_table_free(edgexpu_gguf_up_table *table);
/* The tensor with this exact name, or NULL (edgexpu_gguf_find_tensor). */
const edgexpu_gguf_up_tensor *edgexpu_gguf_up_find(const edgexpu_gguf_up_table *table, const char *name);

typedef struct edgexpu_gguf_device edgexpu_gguf_device;

/* Reads the table, maps the file and copies its data section to the current
 * GPU (initialising device 0 if the library is not initialised yet).  NULL
 * and a message on failure. */
edgexpu_gguf_device *edgexpu_gguf_device_upload(const char *path, char *error, size_t error_size);
const edgexpu_gguf_up_table *edgexpu_gguf_device_table(const edgexpu_gguf_device *d);
/* Device address of a tensor's blocks, or NULL when the name is unknown. */
const void *edgexpu_gguf_device_tensor(const edgexpu_gguf_device *d, const char *name);
/* A weight handle (edgexpu_hip_weight_wrap; not owning) over a tensor used as
 * an [n_out x n_in] matrix: NULL and a message when the name is unknown, the
 * element count is not n_out * n_in, rows of n_in have no block layout, or
 * the tensor's byte size is 0 or not n_out rows of n_in (the checks of
 * load_qweight, src/native.c:611-644).  Free the handle with
 * edgexpu_hip_weight_free before edgexpu_gguf_device_free. */
edgexpu_hip_weight *edgexpu_gguf_device_weight(const edgexpu_gguf_device *d, const char *name, int n_out, int n_in,
                                               char *error, size_t error_size);
void edgexpu_gguf_device_free(edgexpu_gguf_device *d);

#ifdef __cplusplus
}
#endif

#endif
