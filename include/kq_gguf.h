/* GGUF wire-byte reader of libgmlx_amd (host code, no GPU).
 *
 * Replaces the C++ GGUF reader inside mlx-kquant that kq.load_gguf(path,
 * zero_copy) wraps (gmlx/loader.py:92-142, one call per shard at :124), and
 * the metadata scan of gmlx/headerscan.py:122-176.  The file is mapped
 * read-only while the handle is open; keys, string values, arrays and tensor
 * bytes are returned as pointers into the mapping (GGUF wire bytes,
 * unchanged: the kernels consume K-quant rows as they lie in the file).
 *
 * Status codes are those of kq_capi.h; malformed headers give
 * KQ_ERR_BAD_FORMAT, an unreadable file KQ_ERR_IO. */
#ifndef KQ_GGUF_H
#define KQ_GGUF_H

#include <stdint.h>

#include "kq_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kq_gguf kq_gguf;

/* Open and parse a GGUF v2/v3 file: header, every metadata entry, the tensor
 * table.  A file cut short inside the tensor data opens (its expected size
 * exceeds its size; such tensors have data == NULL). */
int kq_gguf_open(const char *path, kq_gguf **out);
void kq_gguf_close(kq_gguf *g);

/* expected_size = data_offset + the end of the last tensor (0 without
 * tensors); a file shorter than that is truncated. */
int kq_gguf_header(const kq_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv,
                   int64_t *data_offset, int64_t *alignment, int64_t *file_size,
                   int64_t *expected_size);

/* Metadata entry i.  type is the GGUF value type (0 u8, 1 i8, 2 u16, 3 i16,
 * 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64).
 * Scalars: count 1, data -> the value.  Strings: count = byte length, data ->
 * the bytes.  Arrays: elem_type, count = elements, data -> the first element
 * (string elements are u64 length + bytes, one after the other). */
int kq_gguf_kv(const kq_gguf *g, int64_t i, const char **key, int64_t *key_len, uint32_t *type,
               uint32_t *elem_type, int64_t *count, const void **data);

/* Tensor i: dims[4] in GGUF order (dims[0] varies fastest: the row length),
 * unused dims 1; ggml_type the GGML type id (12 Q4_K, 14 Q6_K, 16 IQ2_XXS,
 * 0 F32, 1 F16, 30 BF16, ...); offset relative to the data section; data ->
 * the bytes in the mapping, NULL when they lie past the end of the file. */
int kq_gguf_tensor(const kq_gguf *g, int64_t i, const char **name, int64_t *name_len,
                   uint32_t *n_dims, int64_t *dims, uint32_t *ggml_type, int64_t *offset,
                   int64_t *nbytes, const void **data);

/* Values and bytes per block of a GGML type id; KQ_ERR_UNSUPPORTED_CODEC
 * for ids the table does not assign. */
int kq_gguf_type_size(uint32_t ggml_type, int32_t *block, int32_t *bytes);

#ifdef __cplusplus
}
#endif

#endif /* KQ_GGUF_H */
