/*
 * GGUF v3 tensor table and the one-time device upload of a model's blocks
 * (include/edgexpu_gguf_upload.h).  The table is the one edgexpu_gguf_load
 * builds (src/gguf.c:359-610); the upload replaces the per-token staging
 * copy of src/native.c:350-380,593-655.
 *
 * File layout read here (GGUF v3, little-endian):
 *   "GGUF" | u32 version | u64 tensor_count | u64 kv_count
 *   kv_count x { string key | u32 value type | value }
 *   tensor_count x { string name | u32 n_dims | u64 dims[n_dims] | u32 type | u64 offset }
 *   padding to a multiple of 32 (src/gguf.c:595; general.alignment is
 *   reported, not used) | data section
 * where a string is u64 length + bytes, and a value is a scalar, a string, or
 * an array (u32 element type | u64 count | elements, arrays nesting).
 */
#define _POSIX_C_SOURCE 200809L
#include "edgexpu_gguf_upload.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include "edgexpu_kernels.h"

enum {
    GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7,
    GV_STRING = 8, GV_ARRAY = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12
};

/* Bytes of a scalar value type; 0 for string, array and unknown ids. */
static size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        default: return 0;
    }
}

/* A bounds-checked reader over the file (buffered stdio; positions are
 * 64-bit). */
typedef struct {
    FILE *f;
    uint64_t pos, size;
    int bad;
} rd;

static int rd_bytes(rd *r, void *dst, uint64_t n) {
    if (r->bad || n > r->size - r->pos) {
        r->bad = 1;
        return 0;
    }
    if (n != 0 && fread(dst, 1, (size_t)n, r->f) != (size_t)n) {
        r->bad = 1;
        return 0;
    }
    r->pos += n;
    return 1;
}

static int rd_skip(rd *r, uint64_t n) {
    if (r->bad || n > r->size - r->pos) {
        r->bad = 1;
        return 0;
    }
    if (fseeko(r->f, (off_t)(r->pos + n), SEEK_SET) != 0) {
        r->bad = 1;
        return 0;
    }
    r->pos += n;
    return 1;
}

static int rd_u32(rd *r, uint32_t *v) {
    uint8_t b[4];
    if (!rd_bytes(r, b, 4)) return 0;
    *v = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
    return 1;
}

static int rd_u64(rd *r, uint64_t *v) {
    uint32_t lo, hi;
    if (!rd_u32(r, &lo) || !rd_u32(r, &hi)) return 0;
    *v = (uint64_t)lo | ((uint64_t)hi << 32);
    return 1;
}

/* A string into dst (truncated to cap - 1 bytes, the rest skipped). */
static int rd_string(rd *r, char *dst, size_t cap) {
    uint64_t n;
    uint64_t keep;
    if (!rd_u64(r, &n)) return 0;
    keep = n < (uint64_t)(cap - 1) ? n : (uint64_t)(cap - 1);
    if (!rd_bytes(r, dst, keep)) return 0;
    dst[keep] = '\0';
    return rd_skip(r, n - keep);
}

/* Skips one value of type t; depth bounds nested arrays. */
static int rd_skip_value(rd *r, uint32_t t, int depth) {
    uint64_t n, i;
    uint32_t et;
    size_t sb = scalar_bytes(t);
    if (sb != 0) return rd_skip(r, sb);
    if (t == GV_STRING) return rd_u64(r, &n) && rd_skip(r, n);
    if (t != GV_ARRAY || depth > 8) {
        r->bad = 1;
        return 0;
    }
    if (!rd_u32(r, &et) || !rd_u64(r, &n)) return 0;
    sb = scalar_bytes(et);
    if (sb != 0) {
        if (n > (r->size - r->pos) / sb) {
            r->bad = 1;
            return 0;
        }
        return rd_skip(r, n * sb);
    }
    for (i = 0; i < n; i++) {
        if (!rd_skip_value(r, et, depth + 1)) return 0;
    }
    return 1;
}

static void set_msg(char *error, size_t error_size, const char *msg) {
    if (error != NULL && error_size > 0) {
        snprintf(error, error_size, "%s", msg);
    }
}

void edgexpu_gguf_up_table_free(edgexpu_gguf_up_table *table) {
    if (table == NULL) return;
    free(table->tensors);
    memset(table, 0, sizeof(*table));
}

/* The element count of t (the product of its dims), or 0 when the product
 * does not fit 64 bits; *ok = 0 then. */
static uint64_t tensor_elements(const edgexpu_gguf_up_tensor *t, int *ok) {
    uint64_t n = 1;
    uint32_t d;
    *ok = 1;
    for (d = 0; d < t->n_dims; d++) {
        if (t->dims[d] != 0 && n > UINT64_MAX / t->dims[d]) {
            *ok = 0;
            return 0;
        }
        n *= t->dims[d];
    }
    return n;
}

/* Byte size of t's blocks: elements / block size * block bytes; 0 for a type
 * without a block layout here, an element count that is not whole blocks, or
 * a size that does not fit 64 bits (*ok = 0 for the last). */
static uint64_t tensor_nbytes(const edgexpu_gguf_up_tensor *t, int *ok) {
    size_t bs = edgexpu_gguf_type_block_size(t->type);
    size_t bb = edgexpu_gguf_type_block_bytes(t->type);
    uint64_t n = tensor_elements(t, ok);
    if (!*ok || bs == 0 || bb == 0 || n % bs != 0) return 0;
    if (n / bs > UINT64_MAX / bb) {
        *ok = 0;
        return 0;
    }
    return n / bs * bb;
}

int edgexpu_gguf_up_read_table(const char *path, edgexpu_gguf_up_table *table, char *error, size_t error_size) {
    rd r = {0};
    char magic[4];
    char key[256];
    uint64_t i;
    if (path == NULL || table == NULL) {
        set_msg(error, error_size, "GGUF table: path and table are required");
        return 0;
    }
    memset(table, 0, sizeof(*table));
    table->alignment = 32;
    r.f = fopen(path, "rb");
    if (r.f == NULL) {
        set_msg(error, error_size, "GGUF table: cannot open the file");
        return 0;
    }
    if (fseeko(r.f, 0, SEEK_END) != 0) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: cannot size the file");
        return 0;
    }
    r.size = (uint64_t)ftello(r.f);
    rewind(r.f);
    table->file_size = r.size;
    if (!rd_bytes(&r, magic, 4) || memcmp(magic, "GGUF", 4) != 0) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: not a GGUF file");
        return 0;
    }
    if (!rd_u32(&r, &table->version) || !rd_u64(&r, &table->tensor_count) || !rd_u64(&r, &table->kv_count)) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: truncated header");
        return 0;
    }
    if (table->version != 3) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: only GGUF version 3 is read");
        return 0;
    }
    for (i = 0; i < table->kv_count; i++) {
        uint32_t t;
        if (!rd_string(&r, key, sizeof(key)) || !rd_u32(&r, &t)) break;
        if (strcmp(key, "general.alignment") == 0 && t == GV_U32) {
            if (!rd_u32(&r, &table->alignment)) break; /* reported only */
        } else if (!rd_skip_value(&r, t, 0)) {
            break;
        }
    }
    if (r.bad) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: truncated or malformed metadata");
        return 0;
    }
    /* a tensor info takes at least 24 bytes: bound the allocation by the file */
    if (table->tensor_count > (r.size - r.pos) / 24 || table->tensor_count > 0xFFFFFFFFu) {
        fclose(r.f);
        set_msg(error, error_size, "GGUF table: tensor count exceeds the file");
        return 0;
    }
    if (table->tensor_count > 0) {
        table->tensors = (edgexpu_gguf_up_tensor *)calloc((size_t)table->tensor_count, sizeof(*table->tensors));
        if (table->tensors == NULL) {
            fclose(r.f);
            set_msg(error, error_size, "GGUF table: out of memory");
            return 0;
        }
    }
    for (i = 0; i < table->tensor_count; i++) {
        edgexpu_gguf_up_tensor *t = &table->tensors[i];
        uint32_t d;
        if (!rd_string(&r, t->name, sizeof(t->name)) || !rd_u32(&r, &t->n_dims)) break;
        if (t->n_dims > 4) {
            fclose(r.f);
            edgexpu_gguf_up_table_free(table);
            set_msg(error, error_size, "GGUF table: a tensor has more than 4 dims");
            return 0;
        }
        for (d = 0; d < t->n_dims; d++) {
            if (!rd_u64(&r, &t->dims[d])) break;
        }
        if (!rd_u32(&r, &t->type) || !rd_u64(&r, &t->offset)) break;
        {
            int ok;
            t->nbytes = tensor_nbytes(t, &ok);
            if (!ok) {
                fclose(r.f);
                edgexpu_gguf_up_table_free(table);
                set_msg(error, error_size, "GGUF table: a tensor's element count or byte size overflows 64 bits");
                return 0;
            }
        }
        table->n_tensors++;
    }
    fclose(r.f);
    if (r.bad) {
        edgexpu_gguf_up_table_free(table);
        set_msg(error, error_size, "GGUF table: truncated tensor infos");
        return 0;
    }
    /* src/gguf.c:595: the data section starts at the end of the infos
     * rounded up to 32, whatever general.alignment says */
    table->data_offset = (r.pos + 31u) & ~(uint64_t)31u;
    for (i = 0; i < table->n_tensors; i++) {
        const edgexpu_gguf_up_tensor *t = &table->tensors[i];
        const uint64_t avail = table->data_offset <= r.size ? r.size - table->data_offset : 0;
        if (t->offset > avail || t->nbytes > avail - t->offset) {
            edgexpu_gguf_up_table_free(table);
            set_msg(error, error_size, "GGUF table: a tensor's bytes lie past the end of the file");
            return 0;
        }
    }
    return 1;
}

const edgexpu_gguf_up_tensor *edgexpu_gguf_up_find(const edgexpu_gguf_up_table *table, const char *name) {
    uint32_t i;
    if (table == NULL || name == NULL) return NULL;
    for (i = 0; i < table->n_tensors; i++) {
        if (strcmp(table->tensors[i].name, name) == 0) return &table->tensors[i];
    }
    return NULL;
}

/* ------------------------------------------------------------ device copy */

struct edgexpu_gguf_device {
    edgexpu_gguf_up_table table;
    void *dev;        /* the data section, file bytes [data_offset, file_size) */
    uint64_t bytes;
};

edgexpu_gguf_device *edgexpu_gguf_device_upload(const char *path, char *error, size_t error_size) {
    edgexpu_gguf_device *d = (edgexpu_gguf_device *)calloc(1, sizeof(*d));
    int fd;
    void *map;
    if (d == NULL) {
        set_msg(error, error_size, "GGUF upload: out of memory");
        return NULL;
    }
    if (!edgexpu_gguf_up_read_table(path, &d->table, error, error_size)) {
        free(d);
        return NULL;
    }
    d->bytes = d->table.file_size > d->table.data_offset ? d->table.file_size - d->table.data_offset : 0;
    if (d->bytes == 0) {
        return d; /* no tensor data: nothing to upload */
    }
    fd = open(path, O_RDONLY);
    if (fd < 0) {
        edgexpu_gguf_up_table_free(&d->table);
        free(d);
        set_msg(error, error_size, "GGUF upload: cannot open the file");
        return NULL;
    }
    map = mmap(NULL, (size_t)d->table.file_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        edgexpu_gguf_up_table_free(&d->table);
        free(d);
        set_msg(error, error_size, "GGUF upload: mmap failed");
        return NULL;
    }
    d->dev = edgexpu_hip_upload_bytes((const uint8_t *)map + d->table.data_offset, (size_t)d->bytes);
    munmap(map, (size_t)d->table.file_size);
    if (d->dev == NULL) {
        char msg[200];
        edgexpu_hip_last_error(msg, sizeof(msg));
        if (error != NULL && error_size > 0) snprintf(error, error_size, "GGUF upload: %s", msg);
        edgexpu_gguf_up_table_free(&d->table);
        free(d);
        return NULL;
    }
    return d;
}

const edgexpu_gguf_up_table *edgexpu_gguf_device_table(const edgexpu_gguf_device *d) {
    return d != NULL ? &d->table : NULL;
}

const void *edgexpu_gguf_device_tensor(const edgexpu_gguf_device *d, const char *name) {
    const edgexpu_gguf_up_tensor *t = d != NULL ? edgexpu_gguf_up_find(&d->table, name) : NULL;
    if (t == NULL || d->dev == NULL) return NULL;
    return (const uint8_t *)d->dev + t->offset;
}

edgexpu_hip_weight *edgexpu_gguf_device_weight(const edgexpu_gguf_device *d, const char *name, int n_out, int n_in,
                                               char *error, size_t error_size) {
    const edgexpu_gguf_up_tensor *t = d != NULL ? edgexpu_gguf_up_find(&d->table, name) : NULL;
    uint64_t n;
    size_t rb;
    int ok;
    if (t == NULL || d->dev == NULL || n_out <= 0 || n_in <= 0) {
        if (error != NULL && error_size > 0)
            snprintf(error, error_size, "GGUF weight: missing tensor or bad shape: %s", name != NULL ? name : "");
        return NULL;
    }
    n = tensor_elements(t, &ok);
    if (!ok || n != (uint64_t)n_out * (uint64_t)n_in) {
        if (error != NULL && error_size > 0)
            snprintf(error, error_size, "GGUF weight: shape mismatch: %s (have %llu want %d*%d)", name,
                     (unsigned long long)n, n_out, n_in);
        return NULL;
    }
    rb = edgexpu_gguf_row_bytes(t->type, n_in);
    if (rb == 0) {
        if (error != NULL && error_size > 0) snprintf(error, error_size, "GGUF weight: unsupported type: %s", name);
        return NULL;
    }
    /* load_qweight's size check (src/native.c:624-633): the blocks the
     * handle reads, n_out rows of rb bytes, are exactly the tensor's bytes,
     * which the table already bounded by the file */
    if (t->nbytes == 0 || t->nbytes != (uint64_t)n_out * rb) {
        if (error != NULL && error_size > 0)
            snprintf(error, error_size, "GGUF weight: byte size mismatch: %s (have %llu want %d rows of %zu)", name,
                     (unsigned long long)t->nbytes, n_out, rb);
        return NULL;
    }
    return edgexpu_hip_weight_wrap((const uint8_t *)d->dev + t->offset, t->type, n_out, n_in, NULL);
}

void edgexpu_gguf_device_free(edgexpu_gguf_device *d) {
    if (d == NULL) return;
    edgexpu_hip_free_bytes(d->dev);
    edgexpu_gguf_up_table_free(&d->table);
    free(d);
}
