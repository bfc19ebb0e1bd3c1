/*
 * nspeech_gguf.h — GGUF model files for the MI355X kernels (C ABI of
 * libnspeech_rocm_host.so).
 *
 * Reads a GGUF file (versions 1-3: header, metadata key/values, tensor
 * infos, aligned tensor data) from disk (memory-mapped) or from a caller's
 * buffer, and copies tensors to the GPU as stored: a Q8_0 table or weight
 * goes to HBM as its 34-byte blocks, ready for nsr_q8_0_embed_gather and
 * for nsr_q8_0_to_gemv_q8 / nsr_q8_0_to_t4 (include/nspeech_rocm.h), with
 * no host-side dequantisation.
 *
 * Replaces, for this path, candle's gguf_file::Content::read and
 * quantized_var_builder::VarBuilder::from_gguf_buffer as the reference uses
 * them (examples/bench_triton_encoder.rs:69-73, src/moonshine/model.rs:
 * 133-163, src/parakeet/transducer.rs:1616-1620) and the host dequantise +
 * index_select of the decoder's embedding tables
 * (src/moonshine/gpu_decoder.rs:244-248). The files are those the
 * reference's quantizer writes (tools/quantize-moonshine/src/main.rs:63-150).
 *
 * Every length, count and offset read from the file is checked against the
 * file size before use: a malformed file yields NSR_ERR_BAD_ARG and a
 * message, never an out-of-bounds read.
 */
#ifndef NSPEECH_GGUF_H
#define NSPEECH_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "nspeech_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types (the ids GGUF stores). */
typedef enum nsr_ggml_type {
  NSR_GGML_F32 = 0,
  NSR_GGML_F16 = 1,
  NSR_GGML_Q4_0 = 2,
  NSR_GGML_Q4_1 = 3,
  NSR_GGML_Q5_0 = 6,
  NSR_GGML_Q5_1 = 7,
  NSR_GGML_Q8_0 = 8,
  NSR_GGML_Q8_1 = 9,
  NSR_GGML_Q2_K = 10,
  NSR_GGML_Q3_K = 11,
  NSR_GGML_Q4_K = 12,
  NSR_GGML_Q5_K = 13,
  NSR_GGML_Q6_K = 14,
  NSR_GGML_Q8_K = 15,
  NSR_GGML_BF16 = 30
} nsr_ggml_type;

/* GGUF metadata value types. */
typedef enum nsr_gguf_value_type {
  NSR_GGUF_U8 = 0,
  NSR_GGUF_I8 = 1,
  NSR_GGUF_U16 = 2,
  NSR_GGUF_I16 = 3,
  NSR_GGUF_U32 = 4,
  NSR_GGUF_I32 = 5,
  NSR_GGUF_F32 = 6,
  NSR_GGUF_BOOL = 7,
  NSR_GGUF_STRING = 8,
  NSR_GGUF_ARRAY = 9,
  NSR_GGUF_U64 = 10,
  NSR_GGUF_I64 = 11,
  NSR_GGUF_F64 = 12
} nsr_gguf_value_type;

typedef struct nsr_gguf nsr_gguf;

typedef struct nsr_gguf_tensor {
  const char* name;  /* NUL-terminated; valid until nsr_gguf_close */
  uint32_t type;     /* nsr_ggml_type */
  uint32_t n_dims;   /* 1..4 */
  int64_t shape[4];  /* outermost first (candle's Shape order; GGUF stores the
                        innermost dimension first); entries past n_dims are 1 */
  uint64_t offset;   /* byte offset of the data from the start of the file */
  uint64_t nbytes;   /* bytes of data */
  const void* data;  /* host pointer to the data (inside the mapping) */
} nsr_gguf_tensor;

/* Opens and parses a GGUF file (memory-mapped, read-only). */
nsr_status nsr_gguf_open(const char* path, nsr_gguf** out);

/* Parses a GGUF image held by the caller (which keeps it alive until
 * nsr_gguf_close), as candle's VarBuilder::from_gguf_buffer does. */
nsr_status nsr_gguf_open_buffer(const void* data, uint64_t size, nsr_gguf** out);

void nsr_gguf_close(nsr_gguf* g);

/* Message of the last failure of an nsr_gguf_* call on this thread. */
const char* nsr_gguf_last_error(void);

uint32_t nsr_gguf_version(const nsr_gguf* g);
uint64_t nsr_gguf_alignment(const nsr_gguf* g);
uint64_t nsr_gguf_data_offset(const nsr_gguf* g);

int64_t nsr_gguf_tensor_count(const nsr_gguf* g);
nsr_status nsr_gguf_tensor_at(const nsr_gguf* g, int64_t index, nsr_gguf_tensor* out);
/* NSR_ERR_BAD_ARG when no tensor has that name. */
nsr_status nsr_gguf_find_tensor(const nsr_gguf* g, const char* name, nsr_gguf_tensor* out);

/* Copies a tensor's bytes, as stored, to device memory (nbytes at dst) on
 * `stream`; returns once the copy is enqueued (the source is the mapping,
 * which lives until nsr_gguf_close: synchronise before closing). */
nsr_status nsr_gguf_upload(const nsr_gguf* g, const nsr_gguf_tensor* t, void* device_dst,
                           nsr_stream_t stream);

int64_t nsr_gguf_metadata_count(const nsr_gguf* g);
/* Key and value type of entry `index` (file order). */
nsr_status nsr_gguf_metadata_at(const nsr_gguf* g, int64_t index, const char** key,
                                 uint32_t* value_type);
/* Scalar getters: any integer or bool type as int64, F32/F64 as double, a
 * STRING as a NUL-terminated pointer valid until close. */
nsr_status nsr_gguf_get_int(const nsr_gguf* g, const char* key, int64_t* out);
nsr_status nsr_gguf_get_float(const nsr_gguf* g, const char* key, double* out);
nsr_status nsr_gguf_get_string(const nsr_gguf* g, const char* key, const char** out);
/* Arrays: element type and length, then element i by the same conversions. */
nsr_status nsr_gguf_get_array(const nsr_gguf* g, const char* key, uint32_t* elem_type,
                              uint64_t* count);
nsr_status nsr_gguf_get_array_int(const nsr_gguf* g, const char* key, uint64_t i, int64_t* out);
nsr_status nsr_gguf_get_array_float(const nsr_gguf* g, const char* key, uint64_t i, double* out);
nsr_status nsr_gguf_get_array_string(const nsr_gguf* g, const char* key, uint64_t i,
                                     const char** out);

#ifdef __cplusplus
}
#endif

#endif /* NSPEECH_GGUF_H */
