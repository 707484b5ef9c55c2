/*
 * q4k_gguf.h -- C ABI of the GGUF model-file reader of the MI355X K-quant
 * GEMV library.
 *
 * Reads the metadata and tensor directory of a GGUF file (versions 2 and 3,
 * little-endian) and maps its tensor data read-only, so that Q4_K / Q6_K
 * weights of a model can be uploaded to the GPU and multiplied with
 * q4k_mul_mat_vec_q / q6k_mul_mat_vec_q.  Counterpart of ggml's
 * gguf_init_from_file and gguf_get_* accessors (upstream ggml, which
 * llama-cli uses to load the model the reference's capture ran; not vendored
 * by the reference).
 *
 * Every entry point returns a q4k_status (include/q4k_gemv.h) or a value
 * documented below; none throws or aborts.  A handle is immutable after
 * q4k_gguf_open and may be read from several threads; the pointers it hands
 * out (names, strings, tensor data) stay valid until q4k_gguf_close.
 */
#ifndef Q4K_GGUF_H
#define Q4K_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "q4k_gemv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Metadata value types (gguf_type) */
#define Q4K_GGUF_UINT8 0
#define Q4K_GGUF_INT8 1
#define Q4K_GGUF_UINT16 2
#define Q4K_GGUF_INT16 3
#define Q4K_GGUF_UINT32 4
#define Q4K_GGUF_INT32 5
#define Q4K_GGUF_FLOAT32 6
#define Q4K_GGUF_BOOL 7
#define Q4K_GGUF_STRING 8
#define Q4K_GGUF_ARRAY 9
#define Q4K_GGUF_UINT64 10
#define Q4K_GGUF_INT64 11
#define Q4K_GGUF_FLOAT64 12

typedef struct q4k_gguf q4k_gguf; /* opaque */

typedef struct q4k_gguf_tensor_info {
    const char *name;   /* NUL-terminated, owned by the handle */
    int32_t type;       /* ggml type id (Q4K_GGML_TYPE_*) */
    int32_t n_dims;     /* 1..4 */
    int64_t ne[4];      /* elements per dimension, ggml order (ne[0] = row length); 1 past n_dims */
    uint64_t offset;    /* byte offset of the data from the start of the file */
    uint64_t nbytes;    /* bytes of the data (whole blocks of its type) */
    const void *data;   /* the data in the read-only mapping of the file */
} q4k_gguf_tensor_info;

/* Opens and validates a GGUF file.  Q4K_EFORMAT: not a GGUF v2/v3 file, a
 * count, length or dimension that does not fit the file, a tensor type
 * whose block size is unknown (including the types ggml removed), or tensor
 * offsets other than ggml's layout (each tensor right after the previous
 * one, padded to the alignment, in directory order; ggml's loader refuses
 * the same files); Q4K_EIO: the file cannot be opened, inspected or mapped;
 * Q4K_ENOMEM; Q4K_EINVAL: null arguments. */
int q4k_gguf_open(const char *path, q4k_gguf **out);
void q4k_gguf_close(q4k_gguf *g);

uint32_t q4k_gguf_version(const q4k_gguf *g);
/* general.alignment (32 when absent) and the data section's file offset */
uint64_t q4k_gguf_alignment(const q4k_gguf *g);
uint64_t q4k_gguf_data_offset(const q4k_gguf *g);

/* tensors */
int64_t q4k_gguf_tensor_count(const q4k_gguf *g);
int64_t q4k_gguf_find_tensor(const q4k_gguf *g, const char *name); /* index, -1 if absent */
int q4k_gguf_get_tensor(const q4k_gguf *g, int64_t i, q4k_gguf_tensor_info *out);
/* Bytes of n elements of a ggml type (whole blocks), 0 for unknown types or
 * n not a multiple of the type's block size. */
uint64_t q4k_ggml_row_size(int32_t type, int64_t n);

/* metadata */
int64_t q4k_gguf_kv_count(const q4k_gguf *g);
int64_t q4k_gguf_find_key(const q4k_gguf *g, const char *key); /* index, -1 if absent */
const char *q4k_gguf_key(const q4k_gguf *g, int64_t i);        /* NULL if out of range */
int32_t q4k_gguf_kv_type(const q4k_gguf *g, int64_t i);        /* Q4K_GGUF_*, -1 if out of range */
/* Scalar values converted to the asked kind: integers and bools to int64,
 * any numeric to double; Q4K_EINVAL if the value is not of such a type
 * (or an int64 read of a uint64 above INT64_MAX). */
int q4k_gguf_get_int(const q4k_gguf *g, int64_t i, int64_t *out);
int q4k_gguf_get_float(const q4k_gguf *g, int64_t i, double *out);
/* NUL-terminated copy of a string value, owned by the handle */
int q4k_gguf_get_str(const q4k_gguf *g, int64_t i, const char **out);
/* Arrays: element type and length; numeric elements as one contiguous
 * little-endian block in the mapping (data NULL for string arrays, read
 * those with q4k_gguf_get_arr_str). */
int q4k_gguf_get_arr(const q4k_gguf *g, int64_t i, int32_t *elem_type, int64_t *n, const void **data);
int q4k_gguf_get_arr_str(const q4k_gguf *g, int64_t i, int64_t j, const char **out);

#ifdef __cplusplus
}
#endif

#endif /* Q4K_GGUF_H */
