/* GGUF model store: the container reader and read-only mapping the K-quant
 * path's weights come from (GgufModelStore, src/model.rs:583-681, and
 * parse_gguf, src/model.rs:1034-1240), with uploads of a tensor's packed
 * bytes as-is to HBM as a si_hip_quant_weight.
 *
 * All entry points return SI_HIP_OK or a negative SI_HIP_ERR_* code; on
 * failure si_hip_last_error() holds the reference's message (for example
 * "GGUF header has invalid magic", "unsupported GGUF version 4",
 * "unknown GGUF tensor blk.9.ffn_up.weight").  A store is immutable once
 * opened and may be read from several threads. */
#ifndef SI_HIP_GGUF_H
#define SI_HIP_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "si_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct si_hip_gguf si_hip_gguf;

/* GGUF metadata value types (model.rs:304-318, read_value 1198-1231). */
#define SI_HIP_GGUF_U8 0u
#define SI_HIP_GGUF_I8 1u
#define SI_HIP_GGUF_U16 2u
#define SI_HIP_GGUF_I16 3u
#define SI_HIP_GGUF_U32 4u
#define SI_HIP_GGUF_I32 5u
#define SI_HIP_GGUF_F32 6u
#define SI_HIP_GGUF_BOOL 7u
#define SI_HIP_GGUF_STRING 8u
#define SI_HIP_GGUF_ARRAY 9u
#define SI_HIP_GGUF_U64 10u
#define SI_HIP_GGUF_I64 11u
#define SI_HIP_GGUF_F64 12u

/* One metadata value.  Exactly one payload field is meaningful, by type:
 * u64 (U8/U16/U32/U64, BOOL as 0/1), i64 (I8/I16/I32/I64), f64 (F32 widened
 * exactly, F64), str + count (STRING: count bytes of UTF-8 followed by a NUL
 * the file does not hold), count + array_type (ARRAY: read its items with
 * si_hip_gguf_value_item).  Pointers live as long as the store. */
typedef struct si_hip_gguf_value {
  uint32_t type;
  uint32_t array_type;
  uint64_t count;
  uint64_t u64;
  int64_t i64;
  double f64;
  const char *str;
  const void *node; /* internal: the array an ARRAY value refers to */
} si_hip_gguf_value;

/* One tensor of the index (GgufTensorInfo, model.rs:498-505).  shape has
 * n_dims entries, shape[0] being the contiguous (column) dimension as GGUF
 * stores it.  data_start/data_end are byte offsets in the file: data_start
 * = aligned data base + offset, data_end = the next tensor's start in offset
 * order, or the end of the file for the last one (model.rs:1094-1133). */
typedef struct si_hip_gguf_tensor {
  const char *name;
  uint32_t n_dims;
  uint32_t ggml_type;
  const uint64_t *shape;
  uint64_t offset;
  uint64_t data_start;
  uint64_t data_end;
} si_hip_gguf_tensor;

/* GgufModelStore::open (model.rs:625-666): map the file read-only and parse
 * it.  The mapping stays valid until si_hip_gguf_close. */
int si_hip_gguf_open(const char *path, si_hip_gguf **out_store);
/* parse_gguf over a caller buffer (copied; the caller may free it). */
int si_hip_gguf_parse(const uint8_t *bytes, size_t len, si_hip_gguf **out_store);
void si_hip_gguf_close(si_hip_gguf *store);

uint32_t si_hip_gguf_version(const si_hip_gguf *store);
uint64_t si_hip_gguf_alignment(const si_hip_gguf *store);
uint64_t si_hip_gguf_data_base(const si_hip_gguf *store);
uint64_t si_hip_gguf_file_bytes(const si_hip_gguf *store);

/* Tensors, in the file's index order. */
uint64_t si_hip_gguf_tensor_count(const si_hip_gguf *store);
int si_hip_gguf_tensor_info(const si_hip_gguf *store, uint64_t index, si_hip_gguf_tensor *out);
/* GgufModelStore::tensor lookup (model.rs:668-673): "unknown GGUF tensor <name>". */
int si_hip_gguf_find_tensor(const si_hip_gguf *store, const char *name, uint64_t *out_index);
/* The tensor's bytes [data_start, data_end) inside the mapping (GgufTensorView). */
int si_hip_gguf_tensor_data(const si_hip_gguf *store, uint64_t index, const uint8_t **out_data,
                            uint64_t *out_len);
/* GgufTensorInfo::element_count (model.rs:512-518). */
int si_hip_gguf_tensor_elements(const si_hip_gguf *store, uint64_t index, uint64_t *out_elements);
/* GgufTensorInfo::expected_payload_bytes (model.rs:532-573): F32, F16/BF16
 * and the K-quants; *out_known = 0 (and *out_bytes = 0) for other types, an
 * error for a K-quant whose element count is not a multiple of 256. */
int si_hip_gguf_expected_payload_bytes(const si_hip_gguf *store, uint64_t index,
                                       uint64_t *out_bytes, int *out_known);

/* Metadata, keys in byte order (the reference keeps a BTreeMap). */
uint64_t si_hip_gguf_metadata_count(const si_hip_gguf *store);
int si_hip_gguf_metadata_key(const si_hip_gguf *store, uint64_t index, const char **out_key);
/* "GGUF metadata is missing <key>" (model.rs:450) when absent. */
int si_hip_gguf_metadata_get(const si_hip_gguf *store, const char *key, si_hip_gguf_value *out);
/* Item i of an ARRAY value (arrays may nest). */
int si_hip_gguf_value_item(const si_hip_gguf_value *array, uint64_t index, si_hip_gguf_value *out);

/* Upload (upload_quant_weight_private, metal.rs:2502-2542) or bind
 * (bind_quant_weight_mapped, metal.rs:2549-2580) one K-quant tensor: its
 * type must be Q4_K/Q5_K/Q6_K and its byte range must hold the expected
 * payload (model.rs:790-850 messages); exactly the payload bytes become the
 * weight (alignment padding after it is not copied). */
int si_hip_gguf_upload_tensor(si_hip_context *ctx, const si_hip_gguf *store, uint64_t index,
                              si_hip_quant_weight **out_weight);
int si_hip_gguf_bind_tensor_mapped(si_hip_context *ctx, const si_hip_gguf *store, uint64_t index,
                                   si_hip_quant_weight **out_weight);

/* F32 matvec over rows [row_start, row_start + row_count) of a rank-2 F32
 * tensor (f32_matvec_tensor_rows, metal.rs:3074-3110): "F32 matvec requires a
 * rank-2 F32 tensor", "F32 row range is invalid", "F32 tensor columns or
 * input length is invalid", "F32 tensor payload is shorter than its shape". */
int si_hip_gguf_f32_matvec_tensor_rows(si_hip_context *ctx, const si_hip_gguf *store,
                                       uint64_t index, size_t row_start, size_t row_count,
                                       const float *x, size_t x_len, float *y);
/* F32 matvecs of several rank-2 F32 tensors with the same columns and one
 * input, one submission (f32_matvec_many_gguf_tensors, metal.rs:4780-4870);
 * outputs[i] receives tensor indices[i]'s rows.  A tensor's byte range must
 * hold exactly its payload ("GGUF F32 matvec group tensor is truncated"). */
int si_hip_gguf_f32_matvec_many_tensors(si_hip_context *ctx, const si_hip_gguf *store,
                                        const uint64_t *indices, size_t count, const float *x,
                                        size_t x_len, float *const *outputs);
/* gguf_matvec_tensor_rows (metal.rs:5003-5015): rows [row_start, row_start +
 * row_count) of a rank-2 F32, Q4_K, Q5_K or Q6_K tensor of the store (the
 * quantized checks of q4_k_matvec_tensor_rows / quant_k_matvec_tensor_rows,
 * metal.rs:4346-4467). */
int si_hip_gguf_matvec_tensor_rows(si_hip_context *ctx, const si_hip_gguf *store, uint64_t index,
                                   size_t row_start, size_t row_count, const float *input,
                                   size_t input_len, float *output);
/* gguf_quant_matvec_many_tensors (metal.rs:4532-4646): several Q4_K / Q5_K /
 * Q6_K tensors of the store (indices) over one input, one submission. */
int si_hip_gguf_quant_matvec_many_tensors(si_hip_context *ctx, const si_hip_gguf *store,
                                          const uint64_t *indices, size_t count,
                                          const float *input, size_t input_len,
                                          float *const *outputs);

#ifdef __cplusplus
}
#endif
#endif /* SI_HIP_GGUF_H */
