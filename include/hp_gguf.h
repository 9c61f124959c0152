/*
 * hp_gguf.h -- C ABI of the GGUF v3 reader that feeds the HIP runner.
 *
 * Restates the engine's parser, parseGguf (packages/engine/src/gguf.ts:150-215),
 * and its tensor byte-length contract, tensorByteLength / ggmlTypeStorage
 * (packages/engine/src/tensor-reader.ts:268-293), in C++ so that tensors can
 * be streamed from the file into HBM by hp_hip_weight_upload_gguf (hp_hip.h)
 * without passing through a JS heap.  Semantics kept from gguf.ts:
 *   - magic "GGUF" checked, version read but not checked;
 *   - counts, string and array lengths, dimensions and 64-bit metadata values
 *     must be JS-safe integers (<= 2^53 - 1 in magnitude), as bigintToSafeNumber
 *     (gguf.ts:372-378) requires;
 *   - arrays keep the first max_array_sample elements (all of them for the
 *     keys in complete_array_keys) and skip the rest (gguf.ts:302-365);
 *   - a duplicate metadata key keeps its first position and its last value,
 *     like assignment into a JS object; a duplicate tensor name resolves to
 *     the last tensor, like the Map in tensor-reader.ts:61;
 *   - data start = cursor aligned up to general.alignment (default 32); an
 *     alignment that is not an integer in 1..2^32 is an error (the TS parser
 *     throws a RangeError for a fraction or zero).
 * Arrays nest at most 64 deep here (the TS parser is bounded by its stack).
 * Error messages are C strings, so a NUL byte inside a quoted name ends them.
 * Strings are returned as the file's bytes (the TS parser decodes them as
 * UTF-8; the two agree for valid UTF-8).  Errors carry the TS messages
 * ("Invalid GGUF magic: ...", "Unexpected EOF at offset N", ...).
 */
#ifndef HP_GGUF_H
#define HP_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Metadata value types (gguf.ts:96-110). */
#define HP_GGUF_UINT8 0
#define HP_GGUF_INT8 1
#define HP_GGUF_UINT16 2
#define HP_GGUF_INT16 3
#define HP_GGUF_UINT32 4
#define HP_GGUF_INT32 5
#define HP_GGUF_FLOAT32 6
#define HP_GGUF_BOOL 7
#define HP_GGUF_STRING 8
#define HP_GGUF_ARRAY 9
#define HP_GGUF_UINT64 10
#define HP_GGUF_INT64 11
#define HP_GGUF_FLOAT64 12

/* ggml tensor type ids of the blocks the runner implements (gguf.ts:113-148). */
#define HP_GGML_Q4_K 12
#define HP_GGML_Q6_K 14

/* Status codes beyond hp_hip.h's. */
#define HP_ERR_FORMAT 21 /* malformed GGUF (see hp_gguf_last_error) */
#define HP_ERR_IO 22     /* the file could not be opened or read */

typedef struct hp_gguf hp_gguf_t;

typedef struct hp_gguf_value {
  int32_t type;            /* HP_GGUF_* */
  double number;           /* numeric types; bool as 0 / 1 */
  const char *string;      /* HP_GGUF_STRING: the bytes (NUL-terminated copy) */
  uint64_t string_length;
  int32_t element_type;    /* HP_GGUF_ARRAY: element type id as stored */
  uint64_t length;         /* HP_GGUF_ARRAY: element count in the file */
  uint64_t sample_count;   /* HP_GGUF_ARRAY: elements kept */
  int32_t truncated;       /* HP_GGUF_ARRAY: length > sample_count */
  uint64_t node;           /* HP_GGUF_ARRAY: id for hp_gguf_array_element */
} hp_gguf_value_t;

typedef struct hp_gguf_tensor {
  const char *name;        /* NUL-terminated copy of the stored bytes */
  uint64_t name_length;
  uint32_t n_dims;
  const uint64_t *dims;    /* dims[0] = input size, dims[1] = rows for a 2-D weight */
  uint32_t type_id;        /* ggml type id */
  uint64_t offset;         /* relative to the data start, as stored */
  uint64_t data_offset;    /* absolute file offset */
  uint64_t byte_length;    /* tensorByteLength; 0 when storage_known == 0 */
  int32_t storage_known;   /* the type is in ggmlTypeStorage and the element count divides */
} hp_gguf_tensor_t;

/* Parse the header, metadata and tensor table of a GGUF file.  The file stays
 * open for hp_gguf_read and hp_hip_weight_upload_gguf until hp_gguf_close.
 * max_array_sample: elements kept per array (the engine passes 16 by default,
 * 300000 for chat sessions); complete_array_keys: keys kept whole. */
int32_t hp_gguf_open(const char *path, uint64_t max_array_sample, const char *const *complete_array_keys,
                     size_t complete_key_count, hp_gguf_t **out);
/* Same over bytes in host memory, which must outlive the returned object. */
int32_t hp_gguf_open_memory(const uint8_t *data, size_t size, uint64_t max_array_sample,
                            const char *const *complete_array_keys, size_t complete_key_count, hp_gguf_t **out);
void hp_gguf_close(hp_gguf_t *g);
/* Message of the last failure on the calling thread ("" if none). */
const char *hp_gguf_last_error(void);

int32_t hp_gguf_header(const hp_gguf_t *g, uint32_t *version, uint64_t *tensor_count, uint64_t *metadata_count,
                       uint64_t *data_start, uint64_t *alignment, uint64_t *file_size);
/* Distinct metadata keys, in first-appearance order. */
uint64_t hp_gguf_metadata_count(const hp_gguf_t *g);
int32_t hp_gguf_metadata_entry(const hp_gguf_t *g, uint64_t index, const char **key, uint64_t *key_length,
                               hp_gguf_value_t *value);
/* HP_ERR_ARG when the key is absent. */
int32_t hp_gguf_metadata_find(const hp_gguf_t *g, const char *key, hp_gguf_value_t *value);
/* Element `index` (< sample_count) of an array value. */
int32_t hp_gguf_array_element(const hp_gguf_t *g, uint64_t node, uint64_t index, hp_gguf_value_t *value);

int32_t hp_gguf_tensor_info(const hp_gguf_t *g, uint64_t index, hp_gguf_tensor_t *out);
/* Index of the tensor of that name (the last one when repeated), or -1. */
int64_t hp_gguf_find_tensor(const hp_gguf_t *g, const char *name);
/* Name of a ggml type id ("Q4_K", ..., "UNKNOWN_<id>").  Known names are
 * static; an UNKNOWN_ name lives in a per-thread buffer until the next call. */
const char *hp_gguf_type_name(uint32_t type_id);
/* Copy bytes [offset, offset + length) of the file into host memory
 * (readTensorRange, tensor-reader.ts:120-156).  HP_ERR_IO past the end. */
int32_t hp_gguf_read(const hp_gguf_t *g, uint64_t offset, void *dst, uint64_t length);

#ifdef __cplusplus
}
#endif

#endif
