/*
 * rxq4_gguf.h -- caller-side GGUF tensor ingest for the MI355X Q4_K weight
 * path: read-only mmap of a GGUF file (versions 2 and 3, little-endian),
 * tensor and metadata lookup, and the device copy that serves as the
 * `weights_device` alias of the mapped weights.
 *
 * None of these entry points has a counterpart in the reference: reflex-infer
 * leaves GGUF parsing to its caller (reference docs/library-architecture.md:60,
 * 154-158) and takes "runtime-owned quantized weight pointers and CUDA-visible
 * aliases for mmap-backed weights" (infer.h:94-95 `weights` / `weights_device`).
 * This header is for such callers.  The kernel entry points of rxq4.h never
 * read GGUF.
 *
 * Format (GGUF specification, ggml docs/gguf.md): "GGUF" magic, uint32
 * version, uint64 tensor count, uint64 key/value count; key/value pairs
 * (string key, uint32 value type, value); tensor infos (string name, uint32
 * n_dims, uint64 ne[n_dims], uint32 ggml type, uint64 offset); padding to
 * `general.alignment` (default 32); tensor data.  Strings are a uint64
 * length and bytes without a terminator.
 *
 * Every entry point returns an RXQ4_STATUS_* value; on failure
 * rxq4_last_error() says why.  A handle is read-only after open and may be
 * shared between threads.
 */
#ifndef RXQ4_GGUF_H
#define RXQ4_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types. */
#define RXQ4_GGUF_UINT8 0
#define RXQ4_GGUF_INT8 1
#define RXQ4_GGUF_UINT16 2
#define RXQ4_GGUF_INT16 3
#define RXQ4_GGUF_UINT32 4
#define RXQ4_GGUF_INT32 5
#define RXQ4_GGUF_FLOAT32 6
#define RXQ4_GGUF_BOOL 7
#define RXQ4_GGUF_STRING 8
#define RXQ4_GGUF_ARRAY 9
#define RXQ4_GGUF_UINT64 10
#define RXQ4_GGUF_INT64 11
#define RXQ4_GGUF_FLOAT64 12

typedef struct rxq4_gguf rxq4_gguf; /* opaque file handle */

typedef struct rxq4_gguf_tensor {
    const char *name;  /* NUL-terminated, owned by the handle */
    int ggml_type;     /* GGML type id (12 = Q4_K, 13 = Q5_K, 14 = Q6_K, 0 = F32, ...) */
    int n_dims;        /* 1..4 */
    int64_t ne[4];     /* GGUF order: ne[0] = row length (K), ne[1] = rows (M); unused = 1 */
    uint64_t offset;   /* byte offset from the start of the data section */
    uint64_t nbytes;   /* ne[0] / block_elems * block_bytes * ne[1] * ne[2] * ne[3] */
    const void *host;  /* mapped address of the data (read-only) */
} rxq4_gguf_tensor;

/* Maps `path` read-only and parses header, metadata and tensor infos.  Every
 * field is bounds-checked against the file: counts, string lengths, n_dims,
 * element counts, the ggml type (known types only), row lengths that are a
 * whole number of blocks, unique tensor names, aligned offsets and data that
 * lies inside the file.  Version 1 and big-endian files are rejected. */
int rxq4_gguf_open(const char *path, rxq4_gguf **out);
void rxq4_gguf_close(rxq4_gguf *g);

uint32_t rxq4_gguf_version(const rxq4_gguf *g);
uint32_t rxq4_gguf_alignment(const rxq4_gguf *g);
int64_t rxq4_gguf_n_tensors(const rxq4_gguf *g);
int64_t rxq4_gguf_n_kv(const rxq4_gguf *g);
/* The data section: host address and size (the size of the device copy). */
const void *rxq4_gguf_data(const rxq4_gguf *g);
uint64_t rxq4_gguf_data_bytes(const rxq4_gguf *g);

/* Tensor i (file order), or the index of a name (-1 when absent). */
int rxq4_gguf_tensor_info(const rxq4_gguf *g, int64_t i, rxq4_gguf_tensor *out);
int64_t rxq4_gguf_find_tensor(const rxq4_gguf *g, const char *name);

/* Metadata.  rxq4_gguf_find_kv returns the index of a key or -1.  For arrays
 * *type is RXQ4_GGUF_ARRAY; the element type and count come from
 * rxq4_gguf_kv_array. */
int64_t rxq4_gguf_find_kv(const rxq4_gguf *g, const char *key);
int rxq4_gguf_kv_key(const rxq4_gguf *g, int64_t i, const char **key, int *type);
/* Any integer or bool value as int64 (UINT64 above INT64_MAX fails). */
int rxq4_gguf_kv_int(const rxq4_gguf *g, int64_t i, int64_t *out);
/* FLOAT32 / FLOAT64 as double. */
int rxq4_gguf_kv_float(const rxq4_gguf *g, int64_t i, double *out);
/* STRING: pointer into the mapping (not NUL-terminated) and length. */
int rxq4_gguf_kv_str(const rxq4_gguf *g, int64_t i, const char **s, uint64_t *len);
/* ARRAY: element type, count, and for fixed-size elements the address of
 * the packed little-endian elements in the mapping (NULL for strings). */
int rxq4_gguf_kv_array(const rxq4_gguf *g, int64_t i, int *elem_type, uint64_t *n,
                       const void **data);
/* Elements [first, first + count) of a string array: pointers into the
 * mapping (not NUL-terminated) and lengths.  Walks the array once: O(first +
 * count). */
int rxq4_gguf_kv_array_strs(const rxq4_gguf *g, int64_t i, uint64_t first, uint64_t count,
                            const char **s, uint64_t *len);

/* Copies the whole data section into device memory `dst` (at least
 * rxq4_gguf_data_bytes bytes, 256-byte aligned) through pinned staging
 * buffers on `stream` (hipStream_t, NULL = null stream), and returns when the
 * copy is complete.  Tensor i then lives at dst + offset_i: that address is
 * the `weights_device` alias of tensor_info.host. */
int rxq4_gguf_upload(const rxq4_gguf *g, void *dst, uint64_t dst_bytes, void *stream);

/* Block geometry of a GGML type: elements and bytes per block (0 if unknown). */
int rxq4_ggml_block_elems(int ggml_type);
int rxq4_ggml_block_bytes(int ggml_type);

#ifdef __cplusplus
}
#endif

#endif /* RXQ4_GGUF_H */
