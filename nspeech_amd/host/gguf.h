// nspeech::rocm::gguf — GGUF reader (C++ side of include/nspeech_gguf.h).
//
// Mirrors the part of candle's quantized::gguf_file the reference uses:
// Content::read (header, metadata, tensor infos; src/parakeet/transducer.rs:
// 1616) and per-tensor access (Content::tensor, :1620), plus
// VarBuilder::from_gguf_buffer's shape-checked lookup (src/moonshine/
// model.rs:163, `vb.get((vocab, dim), "weight")` at
// src/moonshine/gpu_decoder.rs:244). Tensors go to the GPU as stored
// (upload), not dequantised on the host.
//
// The format (ggml's published GGUF specification, versions 1-3):
//   u32 magic "GGUF" | u32 version | n_tensors | n_kv        (u64; u32 in v1)
//   n_kv x { string key | u32 value_type | value }
//   n_tensors x { string name | u32 n_dims | n_dims x dim | u32 type | u64 offset }
//   padding to `general.alignment` (default 32) | tensor data
// with string = length (u64; u32 in v1) + bytes, dims innermost first, and
// each offset relative to the data section and aligned.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "rocm_kernels.h"

namespace nspeech {
namespace rocm {
namespace gguf {

enum ValueType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7, STRING = 8, ARRAY = 9,
  U64 = 10, I64 = 11, F64 = 12
};

struct Value {
  uint32_t type = U8;
  uint64_t u = 0;      // unsigned integers and bool
  int64_t i = 0;       // signed integers
  double f = 0.0;      // F32 / F64
  std::string s;       // STRING
  uint32_t elem_type = 0;          // ARRAY
  std::vector<Value> arr;          // ARRAY

  bool is_int() const;
  int64_t as_int() const;   // throws Error unless an integer or bool type
  double as_float() const;  // throws Error unless F32 / F64
};

// Block size (elements) and bytes per block of a ggml type; false when the
// type id is not a ggml type this reader knows.
bool ggml_type_layout(uint32_t type, uint64_t* block, uint64_t* type_size);
const char* ggml_type_name(uint32_t type);

struct TensorInfo {
  std::string name;
  uint32_t type = 0;
  std::vector<uint64_t> shape;  // outermost first
  uint64_t offset = 0;          // relative to the data section
  uint64_t nbytes = 0;
};

class Content {
 public:
  // Parses an in-memory GGUF image; `keepalive` owns the bytes (may be null
  // when the caller keeps them alive).
  static Content read(const uint8_t* data, uint64_t size, std::shared_ptr<void> keepalive = nullptr);
  // Memory-maps and parses a file.
  static Content open(const std::string& path);

  uint32_t version() const { return version_; }
  uint64_t alignment() const { return alignment_; }
  uint64_t data_offset() const { return data_offset_; }
  const std::vector<std::pair<std::string, Value>>& metadata() const { return metadata_; }
  const Value* find_metadata(const std::string& key) const;
  const std::vector<TensorInfo>& tensor_infos() const { return tensors_; }
  const TensorInfo* find_tensor(const std::string& name) const;
  const uint8_t* tensor_data(const TensorInfo& t) const { return base_ + data_offset_ + t.offset; }

  // Copies a tensor's stored bytes to a new device tensor (U8, shape
  // [nbytes]) on the device's stream (Content::tensor(.., device)).
  Tensor upload(const TensorInfo& t, const RocmDevice& device) const;
  // VarBuilder::get: the tensor `name` with exactly `shape` (outermost
  // first), uploaded; throws Error on a missing name or a shape mismatch.
  Tensor get(const std::vector<uint64_t>& shape, const std::string& name, const RocmDevice& device,
             uint32_t* type = nullptr) const;

 private:
  std::shared_ptr<void> keep_;
  const uint8_t* base_ = nullptr;
  uint64_t size_ = 0;
  uint32_t version_ = 0;
  uint64_t alignment_ = 32;
  uint64_t data_offset_ = 0;
  std::vector<std::pair<std::string, Value>> metadata_;
  std::map<std::string, size_t> meta_index_;
  std::vector<TensorInfo> tensors_;
  std::map<std::string, size_t> tensor_index_;
};

}  // namespace gguf
}  // namespace rocm
}  // namespace nspeech
