/*
 * C ABI of the QWENBIN1 model archive: the reader (src/archive.cpp:49-102,
 * include/infer/archive.hpp of Greedy-cy/qwen2.5-jetson-inference), the
 * W8A16 / W16A16 exporter (tools/export_model.py:202-396) and the
 * config.json loader (src/model_config.cpp:15-46).  Host-only code: none of
 * these calls touches the GPU.
 *
 * Format (the reference's, kept so that the same files serve both engines):
 *   - a 32-byte packed header `<8sIIQQ>`: magic "QWENBIN1", version 1, the
 *     JSON metadata's byte size, the data offset, a reserved word;
 *   - UTF-8 JSON metadata right after the header: {"format", "version",
 *     "source", "precision", "group_size", "tensors": [{"name", "shape",
 *     "dtype" ("float32" | "bfloat16" | "int8"), "offset", "nbytes", "sha256",
 *     "quant"?}]};
 *   - tensor payloads at data offset + offset (the exporter uses a 1 MiB data
 *     offset and 256-byte alignment relative to it).
 * A W8A16 Linear weight is an int8 [out, in] record whose "quant" object
 * names its BF16 [out, ceil(in / group_size)] scale tensor "<name>.scale".
 *
 * Every entry point that returns int returns a status code of
 * include/infer_linear.h, with the message in infer_hip_last_error.
 */
#ifndef INFER_ARCHIVE_H
#define INFER_ARCHIVE_H

#include <stddef.h>
#include <stdint.h>

#include "infer_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* include/infer/common.hpp:10 (DType). */
enum infer_hip_dtype {
  INFER_HIP_DTYPE_FLOAT32 = 0,
  INFER_HIP_DTYPE_BFLOAT16 = 1,
  INFER_HIP_DTYPE_INT8 = 2
};

#define INFER_HIP_ARCHIVE_MAX_DIMS 8

/* include/infer/archive.hpp:7-20 (QuantizationInfo, TensorRecord).  The
 * strings point into the archive object and live as long as it. */
typedef struct infer_hip_tensor_record {
  const char* name;
  int ndim;
  int64_t shape[INFER_HIP_ARCHIVE_MAX_DIMS];
  int dtype;               /* infer_hip_dtype */
  uint64_t offset;         /* from the data offset */
  uint64_t nbytes;
  int quant_group_size;    /* 0: not quantised */
  int quant_axis;          /* 1 when quantised (the "axis" default) */
  const char* scale_tensor; /* NULL when not quantised */
  const char* sha256;      /* hex digest of the payload; "" when absent */
} infer_hip_tensor_record;

typedef struct infer_hip_archive infer_hip_archive;

/* ModelArchive::open (src/archive.cpp:49-102): maps the file read-only and
 * validates the header, the metadata and every record (size = numel x dtype
 * size, payload inside the file, no duplicate name).  Same error cases as
 * the reference. */
int infer_hip_archive_open(const char* path, infer_hip_archive** archive);
/* Never fails (NULL is accepted) and leaves the last error message as it is. */
int infer_hip_archive_close(infer_hip_archive* archive);
int infer_hip_archive_tensor_count(const infer_hip_archive* archive);
int infer_hip_archive_record(const infer_hip_archive* archive, int index,
                             infer_hip_tensor_record* record);
/* ModelArchive::contains / record lookup: the record's index, or -1. */
int infer_hip_archive_find(const infer_hip_archive* archive, const char* name);
/* ModelArchive::data: the payload of record `index` in the mapping. */
const void* infer_hip_archive_data(const infer_hip_archive* archive, int index);
uint64_t infer_hip_archive_data_offset(const infer_hip_archive* archive);
size_t infer_hip_archive_mapped_bytes(const infer_hip_archive* archive);
/* verify_archive (tools/export_model.py:148-199): every record's offset is a
 * multiple of 256 and its payload's SHA-256 equals the recorded digest. */
int infer_hip_archive_verify(const infer_hip_archive* archive);
/* The metadata's "precision" ("w8a16", "w16a16", "fp32"; "" when absent). */
const char* infer_hip_archive_precision(const infer_hip_archive* archive);

/* One FP32 source tensor of an export (the safetensors tensors the
 * reference's exporter reads, in file order). */
typedef struct infer_hip_export_tensor {
  const char* name;
  int ndim;
  const int64_t* shape;
  const float* data; /* numel values, row-major */
} infer_hip_export_tensor;

/* The counts and errors of export()'s report (export_model.py:370-395). */
typedef struct infer_hip_export_report {
  int tensor_count;
  int quantized_count;
  int int8_count;
  int bfloat16_count;
  int float32_count;
  double max_groupwise_abs_error; /* |w - q * bf16(scale)| over quantised tensors */
  double max_bfloat16_abs_error;  /* |x - bf16(x)| over BF16-stored tensors */
  uint64_t bytes;                 /* archive file size */
} infer_hip_export_report;

/* export() (export_model.py:273-368): precision "w8a16" (group_size must be
 * 64), "w16a16" or "fp32".  Under W8A16 every 2-D tensor except
 * model.embed_tokens.weight and lm_head.weight is quantised symmetric per
 * group of group_size columns (scale = max|w| / 127, 1 where the group is all
 * zero; q = clip(round-half-even(w / scale), -127, 127)) and followed by its
 * BF16 "<name>.scale" tensor; the other tensors are stored BF16 (RNE), or FP32
 * under "fp32".  `source` is recorded in the metadata; report may be NULL.
 * max_bfloat16_abs_error covers the BF16 scale tensors too, as the reference's
 * report does. */
int infer_hip_archive_export(const char* path, const char* precision, int group_size,
                             const infer_hip_export_tensor* tensors, int count,
                             const char* source, infer_hip_export_report* report);

/* ModelConfig::load (src/model_config.cpp:15-37): a Hugging Face
 * config.json with model_type "qwen2".  max_position_embeddings may be NULL. */
int infer_hip_model_config_load(const char* path, infer_hip_model_config* config,
                                int* max_position_embeddings);

/* Qwen2Model::Qwen2Model(model_directory, options) (src/qwen2.cpp:30-78):
 * loads <dir>/config.json and <dir>/model.<precision>.qbin
 * (archive_filename, include/infer/common.hpp:49-55), checks
 * max_sequence_length <= max_position_embeddings, uploads every tensor into
 * one device allocation owned by the model (freed by
 * infer_hip_model_destroy) and creates the model on the current device. */
int infer_hip_model_open(const char* model_directory, const infer_hip_runtime_options* options,
                         infer_hip_model** model);

#ifdef __cplusplus
}
#endif

#endif /* INFER_ARCHIVE_H */
