/*
 * ullm/weights_io.h -- on-disk weights: safetensors files in, packed device
 * weights out (gfx950 build).
 *
 * The reference plans to load safetensors checkpoints (reference
 * docs/plans/main-plan.md:26,53) and to verify every consumed byte against a
 * model lock that records each file's size and SHA-256
 * (docs/models/model-lock.md, "Required lock contents" and "Resolution
 * procedure" step 7: reject a missing file or a content mismatch).  It has no
 * loader yet.  These entry points are the native side of that loader for the
 * quantized linear layer: open (and optionally verify) a safetensors file,
 * inspect its tensors, build ullm_linear_weight_t handles from them, and write
 * device weights back out in their canonical encodings.
 *
 * Conventions are those of include/ullm/linear.h (ABI v1 headers, zero
 * reserved words, error sink, no exceptions, handle table).  The safetensors
 * format is the published one: an 8-byte little-endian header length, a JSON
 * header mapping tensor names to {dtype, shape, data_offsets} plus an optional
 * "__metadata__" map of strings, then the tensor bytes; offsets are relative
 * to the end of the header and the tensors tile the data region exactly.
 */
#ifndef ULLM_WEIGHTS_IO_H
#define ULLM_WEIGHTS_IO_H

#include "ullm/linear.h"

/* safetensors element types (the format's dtype strings). */
#define ULLM_ST_DTYPE_BOOL UINT32_C(1)
#define ULLM_ST_DTYPE_U8 UINT32_C(2)
#define ULLM_ST_DTYPE_I8 UINT32_C(3)
#define ULLM_ST_DTYPE_F8_E4M3 UINT32_C(4)
#define ULLM_ST_DTYPE_F8_E5M2 UINT32_C(5)
#define ULLM_ST_DTYPE_U16 UINT32_C(6)
#define ULLM_ST_DTYPE_I16 UINT32_C(7)
#define ULLM_ST_DTYPE_F16 UINT32_C(8)
#define ULLM_ST_DTYPE_BF16 UINT32_C(9)
#define ULLM_ST_DTYPE_U32 UINT32_C(10)
#define ULLM_ST_DTYPE_I32 UINT32_C(11)
#define ULLM_ST_DTYPE_F32 UINT32_C(12)
#define ULLM_ST_DTYPE_U64 UINT32_C(13)
#define ULLM_ST_DTYPE_I64 UINT32_C(14)
#define ULLM_ST_DTYPE_F64 UINT32_C(15)

#define ULLM_ST_MAX_RANK 8

typedef struct ullm_safetensors_t ullm_safetensors_t;

typedef struct ullm_safetensors_open_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  const char *path;
  /* 32 bytes: the file's SHA-256 must equal this (model-lock check); null =
   * not checked.  A mismatch is ULLM_STATUS_INVALID_ARGUMENT. */
  const uint8_t *expected_sha256;
  uint64_t expected_size; /* file bytes that must match; 0 = not checked */
  uint64_t reserved[4];
} ullm_safetensors_open_desc_t;

typedef struct ullm_safetensors_tensor_info_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t dtype; /* ULLM_ST_DTYPE_* */
  uint32_t rank;
  uint64_t shape[ULLM_ST_MAX_RANK];
  uint64_t offset; /* byte offset of the data from the start of the file */
  uint64_t bytes;
  uint64_t reserved[4];
} ullm_safetensors_tensor_info_t;

/* A linear weight from safetensors tensors.
 *   Float sources (F32, BF16, F16 values): `values` names value_parts tensors
 *   [N_i][K] stacked along N in the given order (q/k/v into a fused qkv, gate
 *   and up into a gated pair); the weight is quantized on the GPU with the
 *   encoding's recipe.  scales and zeros must be null.
 *   Encoded sources (one part): FP8_E4M3_ROW takes F8_E4M3 values [N][K] and
 *   F32 scales of shape [N], [N][1] (per row) or [] / [1] (one scale for all
 *   rows); AQ4_G128 takes U32 values [N][K/8], F16 scales and F16 zeros
 *   [N][K/128] (the canonical encodings of linear.h). */
typedef struct ullm_linear_weight_load_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  const ullm_safetensors_t *file;
  uint32_t encoding; /* ULLM_LINEAR_ENCODING_* */
  uint32_t layout;   /* ULLM_LINEAR_LAYOUT_* */
  const char *const *values;
  uint32_t value_parts;
  int32_t device;
  const char *scales;
  const char *zeros;
  void *stream; /* creation blocks until the weight is ready */
  uint64_t reserved[4];
} ullm_linear_weight_load_desc_t;

/* Write device weights in their canonical encodings.  Tensor names per weight
 * `name`: FP8 "<name>.weight" (F8_E4M3 [N][K]) and "<name>.weight_scale"
 * (F32 [N]); AQ4 "<name>.qweight" (U32 [N][K/8]), "<name>.scales" and
 * "<name>.zeros" (F16 [N][K/128]).  "__metadata__" records "format" =
 * "ullm-linear", and per weight "<name>.encoding" ("fp8_e4m3_row" or
 * "aq4_g128") and "<name>.layout" ("plain" or "gated_pairs"), followed by the
 * caller's key/value pairs. */
typedef struct ullm_linear_weights_save_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  const char *path;
  const char *const *names;
  const ullm_linear_weight_t *const *weights;
  uint64_t count;
  const char *const *metadata_keys;
  const char *const *metadata_values;
  uint64_t metadata_count;
  uint64_t reserved[4];
} ullm_linear_weights_save_desc_t;

#ifdef __cplusplus
extern "C" {
#endif

/* Open and validate a safetensors file (header, dtypes, shapes, offsets);
 * with expected_sha256/expected_size set, hash the whole file first. */
ULLM_HIP_API ullm_status_t ullm_safetensors_open(
    const ullm_safetensors_open_desc_t *desc, ullm_safetensors_t **file,
    ullm_error_sink_t *error_sink);

ULLM_HIP_API ullm_status_t ullm_safetensors_close(
    ullm_safetensors_t **file, ullm_error_sink_t *error_sink);

ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_count(
    const ullm_safetensors_t *file, uint64_t *count,
    ullm_error_sink_t *error_sink);

/* Name of tensor `index` in byte order of the names (NUL-terminated; length
 * receives the full length; a short buffer is ULLM_STATUS_BUFFER_TOO_SMALL). */
ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_name(
    const ullm_safetensors_t *file, uint64_t index, char *name,
    uint64_t capacity, uint64_t *length, ullm_error_sink_t *error_sink);

/* A missing tensor is ULLM_STATUS_INVALID_ARGUMENT. */
ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_info(
    const ullm_safetensors_t *file, const char *name,
    ullm_safetensors_tensor_info_t *info, ullm_error_sink_t *error_sink);

/* Value of a "__metadata__" key (same string conventions as tensor_name; a
 * missing key is ULLM_STATUS_INVALID_ARGUMENT). */
ULLM_HIP_API ullm_status_t ullm_safetensors_metadata(
    const ullm_safetensors_t *file, const char *key, char *value,
    uint64_t capacity, uint64_t *length, ullm_error_sink_t *error_sink);

/* SHA-256 of the whole file (computed on first use if open did not). */
ULLM_HIP_API ullm_status_t ullm_safetensors_file_sha256(
    const ullm_safetensors_t *file, uint8_t sha256[32],
    ullm_error_sink_t *error_sink);

ULLM_HIP_API ullm_status_t ullm_linear_weight_load(
    const ullm_linear_weight_load_desc_t *desc, ullm_linear_weight_t **weight,
    ullm_error_sink_t *error_sink);

/* sha256 (32 bytes, may be null) receives the written file's SHA-256. */
ULLM_HIP_API ullm_status_t ullm_linear_weights_save(
    const ullm_linear_weights_save_desc_t *desc, uint8_t *sha256,
    ullm_error_sink_t *error_sink);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* ULLM_WEIGHTS_IO_H */
