// nspeech::rocm — C++ host side of the MI355X fused layer kernels.
//
// Mirrors the host interface nspeech uses for these ops, over the C ABI of
// libnspeech_rocm.so (include/nspeech_rocm.h):
//   * the Tensor-level triton_* functions and buffer-level enc_* functions of
//     src/triton_kernels.rs (same names, argument order and meaning; the
//     Metal device/pipeline pair becomes RocmDevice/RocmKernels and a
//     ComputeCommandEncoder becomes an Encoder = the device's HIP stream);
//   * KokoroGpuBackend::adain_snake_f32 (src/kokoro/gpu_backend.rs:181-185);
//   * QEmbedding::forward (src/parakeet/quantized_layers.rs:65-71);
//   * RotaryEmbedding + apply_rotary_pos_emb (src/moonshine/decoder.rs:85-183).
//
// Error behaviour follows the reference's anyhow::Result: every fallible
// call throws nspeech::rocm::Error with a message (the reference bails with
// "All tensors must be on Metal device" on a storage mismatch,
// src/triton_kernels.rs:138; here "... on the ROCm device"). Launches are
// asynchronous on the device's stream, as Candle's pooled command buffer is;
// RocmDevice::synchronize() is the wait_until_completed() equivalent.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace nspeech {
namespace rocm {

class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

enum class DType { F32, F16, BF16, U8, U32, I64 };
size_t dtype_size(DType d);
const char* dtype_name(DType d);

// One GPU and its stream (candle's MetalDevice + pooled command buffer).
class RocmDevice {
 public:
  // Device `ordinal`, with a default-priority stream of its own.
  static RocmDevice create(int ordinal = 0);
  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_->s; }
  void synchronize() const;  // wait_until_completed()

 private:
  struct Stream {
    hipStream_t s = nullptr;
    ~Stream();
  };
  int ordinal_ = 0;
  std::shared_ptr<Stream> stream_;
};

// Device buffer + byte offset (candle_core::GpuBuffer, src/triton_kernels.rs:9).
struct GpuBuffer {
  void* ptr = nullptr;
  size_t offset = 0;
  void* at() const { return static_cast<char*>(ptr) + offset; }
};

// Contiguous tensor in device memory (or, for the error paths, host memory).
class Tensor {
 public:
  static Tensor empty(const RocmDevice& dev, std::vector<size_t> shape, DType dtype);
  static Tensor from_host(const RocmDevice& dev, const void* data, std::vector<size_t> shape, DType dtype);
  // A host-resident tensor: passing it to a kernel entry point is an error.
  static Tensor cpu(const void* data, std::vector<size_t> shape, DType dtype);

  DType dtype() const { return dtype_; }
  const std::vector<size_t>& shape() const { return shape_; }
  size_t dim(int i) const;
  size_t elem_count() const;
  size_t size_bytes() const { return elem_count() * dtype_size(dtype_); }
  bool on_device() const { return storage_ && storage_->device; }
  GpuBuffer buffer() const;  // the enc_* view of a device tensor
  std::vector<uint8_t> to_host_bytes() const;
  template <class T>
  std::vector<T> to_vec() const {
    std::vector<uint8_t> b = to_host_bytes();
    std::vector<T> v(b.size() / sizeof(T));
    std::copy(b.data(), b.data() + v.size() * sizeof(T), reinterpret_cast<uint8_t*>(v.data()));
    return v;
  }

 private:
  struct Storage {
    void* ptr = nullptr;
    bool device = false;
    std::vector<uint8_t> host;
    ~Storage();
  };
  std::shared_ptr<Storage> storage_;
  std::vector<size_t> shape_;
  DType dtype_ = DType::F32;
};

// The loaded kernel set (TritonKernels::load / DecoderKernels::load /
// KokoroKernels::load, kernels/out/generated/triton_metal_gen.rs:39-106).
class RocmKernels {
 public:
  static RocmKernels load(const RocmDevice& dev);
  int kernel_count() const { return kernel_count_; }
  // The t4 tile copy of a repacked-Q8 weight (qs u32 [K, NW/4], scales f16 [K/32, NW]) that the enc_gemv_q8*
  // calls multiply with. The decoder passes the same weight buffers for every token: each is packed once
  // (nsr_q8_pack_t4, on `stream`, ahead of that call's GEMV) on its first call and the copy reused, so the
  // GEMVs read whole 128-byte lines (the [K, N/4] layout makes a workgroup that owns a few columns read 8 bytes
  // of every weight row) and later calls allocate nothing. Returns the t4 qs and scales.
  std::pair<const uint32_t*, const uint16_t*> t4_weight(hipStream_t stream, const void* qs, const void* scales,
                                                        size_t k, size_t nw, bool glu) const;
  // Drop the t4 copies (for a caller that rewrites or frees a weight buffer).
  void forget_gemv_weights() const;
  size_t gemv_weights_cached() const;

 private:
  struct T4Weight {
    const void* qs;
    const void* scales;
    size_t k, nw;
    bool glu;
    Tensor tq, ts;
  };
  struct GemvWeightCache {
    std::mutex mu;
    std::vector<T4Weight> entries;
  };
  int kernel_count_ = 0;
  RocmDevice device_;
  std::shared_ptr<GemvWeightCache> gemv_weights_;
};

// The encoder of the enc_* API: launches go onto this stream.
using Encoder = hipStream_t;

// ---- Tensor-level API (src/triton_kernels.rs) ------------------------------

// out = LN(x) * (gamma + 1), f16 out [n_rows, n_cols] (:312).
Tensor triton_layernorm_unit_offset(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                                    const Tensor& gamma, size_t n_rows, size_t n_cols);
// out = (x - mean) / sqrt(var + eps), f16 out (:345).
Tensor triton_layernorm_bare(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x, size_t n_rows,
                             size_t n_cols);
// out = x + residual, f16 (:383).
Tensor triton_residual_add(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                           const Tensor& residual, size_t n_elements);
// out = gelu(x), f16 (:412).
Tensor triton_gelu(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x, size_t n_elements);
// out = LN(x) * weight: f32 x, f16 weight, f16 out (:598).
void triton_layernorm_std_f32in(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                                const Tensor& weight, const Tensor& out, size_t n_rows, size_t n_cols);
// out = x + residual, f32 (:625).
void triton_residual_add_f32(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                             const Tensor& residual, const Tensor& out, size_t n_elements);
// out[i] = silu(fc1[n + i]) * fc1[i], f16 (:713).
void triton_glu_silu(const RocmDevice& device, const RocmKernels& kernels, const Tensor& fc1, const Tensor& out,
                     size_t n_elements);
// f32_out = f16_proj + f32_residual; f16_norm = LN(f32_out) * weight (:742).
void triton_residual_add_layernorm(const RocmDevice& device, const RocmKernels& kernels, const Tensor& f16_proj,
                                   const Tensor& f32_residual, const Tensor& f32_out, const Tensor& weight,
                                   const Tensor& f16_norm, size_t n_rows, size_t dim);
// Decode attention over f16 tensors (:648-678): q [n_q_heads, head_dim], K/V
// with the given element strides, out [n_q_heads, head_dim].
void triton_attention_decode(const RocmDevice& device, const RocmKernels& kernels, const Tensor& q, const Tensor& k,
                             const Tensor& v, const Tensor& out, size_t kv_len, size_t head_dim, size_t n_kv_heads,
                             size_t n_q_heads, float sm_scale, size_t stride_kv_head, size_t stride_kv_seq);
// new_kv [n_kv_heads, head_dim] f16 into row `pos` of cache [n_kv_heads, max_kv_len, head_dim] (:680-711).
void triton_kv_cache_append(const RocmDevice& device, const RocmKernels& kernels, const Tensor& new_kv,
                            const Tensor& cache, size_t n_kv_heads, size_t head_dim, size_t max_kv_len, size_t pos);

// ---- Buffer-level API (src/triton_kernels.rs:862-1423) ----------------------

void enc_layernorm_std_f32in(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& weight,
                             const GpuBuffer& out, size_t n_rows, size_t n_cols);
void enc_residual_add_layernorm(Encoder enc, const RocmKernels& kernels, const GpuBuffer& f16_proj,
                                const GpuBuffer& f32_residual, const GpuBuffer& f32_out, const GpuBuffer& weight,
                                const GpuBuffer& f16_norm, size_t n_rows, size_t dim);
void enc_layernorm_bare(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& out,
                        size_t n_rows, size_t n_cols);
void enc_layernorm_unit_offset(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& gamma,
                               const GpuBuffer& out, size_t n_rows, size_t n_cols);
void enc_gelu(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& out, size_t n_elements);
void enc_residual_add(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& residual,
                      const GpuBuffer& out, size_t n_elements);

// Decoder step (src/triton_kernels.rs:900-1010). The reference bakes the head
// count, head_dim and rotary dim into the compiled rope kernel
// (kernels/kernel_configs.py:102-104); here they are arguments.
// enc_rope_qk_cache_fused (:975-991): RoPE on q [n_q_heads, head_dim] and
// k [n_kv_heads, head_dim] f16 in place at `pos` (table row `pos` of the
// [max_kv_len, rotary_dim] f32 RoPE table), rotated k into cache_k
// [n_kv_heads, max_kv_len, head_dim].
void enc_rope_qk_cache_fused(Encoder enc, const RocmKernels& kernels, const GpuBuffer& q, const GpuBuffer& k,
                             const GpuBuffer& rope_table, const GpuBuffer& cache_k, size_t pos, size_t max_kv_len,
                             size_t n_q_heads, size_t n_kv_heads, size_t head_dim, size_t rotary_dim);
// enc_kv_cache_append (:993-1010): new_kv [n_kv_heads, head_dim] f16 into row `pos` of the cache.
void enc_kv_cache_append(Encoder enc, const RocmKernels& kernels, const GpuBuffer& new_kv, const GpuBuffer& cache,
                         size_t n_kv_heads, size_t head_dim, size_t max_kv_len, size_t pos);
// enc_attention_decode (:900-923): f16 q [n_q_heads, head_dim] against kv_len
// cached positions (strides in elements) -> f16 out [n_q_heads, head_dim].
void enc_attention_decode(Encoder enc, const RocmKernels& kernels, const GpuBuffer& q, const GpuBuffer& k,
                          const GpuBuffer& v, const GpuBuffer& out, size_t kv_len, size_t head_dim,
                          size_t n_kv_heads, size_t n_q_heads, float sm_scale, size_t stride_kv_head,
                          size_t stride_kv_seq);
// enc_attention_splitkv (:925-973): as above over n_splits ranges with the
// caller's partial buffer (3 * 128 f32 per head and split is enough).
void enc_attention_splitkv(Encoder enc, const RocmKernels& kernels, const GpuBuffer& q, const GpuBuffer& k,
                           const GpuBuffer& v, const GpuBuffer& out, const GpuBuffer& partial_buf, size_t kv_len,
                           size_t head_dim, size_t n_kv_heads, size_t n_q_heads, float sm_scale,
                           size_t stride_kv_head, size_t stride_kv_seq, size_t n_splits);

// Decoder MLP GEMVs at M = 1 over the reference's repacked-Q8 layout (qs u32 [K, NW/4], scales f16 [K/32, NW]),
// the kernels of kernels/moonshine_kernels.py:616-677, 1721-1819 (the reference's Triton source has them; its
// Metal decoder does not dispatch them). x and the f16 outputs as the decoder holds them.
// enc_gemv_q8: out [N] f16 = x [K] f16 @ W + bias (bias f32 [N] or an empty buffer).
void enc_gemv_q8(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                 const GpuBuffer& scales, const GpuBuffer* bias, const GpuBuffer& out, size_t k, size_t n);
// enc_gemv_q8_bias_glu: out [N] f16 = silu(gate) * up over fc1's 2N columns (+ bias f32 [2N]).
void enc_gemv_q8_bias_glu(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                          const GpuBuffer& scales, const GpuBuffer& bias, const GpuBuffer& out, size_t k, size_t n);
// enc_gemv_q8_resadd_ln: out_f32 [dim] = f16(x @ W) + residual f32; norm [dim] f16 = LN(out_f32) * weight f16.
void enc_gemv_q8_resadd_ln(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                           const GpuBuffer& scales, const GpuBuffer& residual, const GpuBuffer& out_f32,
                           const GpuBuffer& ln_weight, const GpuBuffer& norm, size_t k, size_t dim, float eps);

// ---- Kokoro backend (src/kokoro/gpu_backend.rs) ------------------------------

// The AdaIN+Snake part of KokoroGpuBackend for the ROCm device: Buf = GpuBuffer.
class RocmKokoroBackend {
 public:
  RocmKokoroBackend(const RocmDevice& device, const RocmKernels& kernels)
      : device_(device), kernels_(kernels), conv_weights_(std::make_shared<ConvWeightCache>()) {}
  // out = snake(AdaIN(x)) over x [channels, seq_len] f32; gamma, beta, alpha
  // [channels] f16 (the precomputed style parameters, decoder.rs:966-981).
  void adain_snake_f32(const GpuBuffer& x, const GpuBuffer& gamma, const GpuBuffer& beta, const GpuBuffer& alpha,
                       const GpuBuffer& out, size_t channels, size_t seq_len) const;
  // The f16-activation variant (gpu_backend.rs:55-57): x, out [channels,
  // seq_len] f16, parameters f16; seq_len up to 131072.
  void adain_snake(const GpuBuffer& x, const GpuBuffer& gamma, const GpuBuffer& beta, const GpuBuffer& alpha,
                   const GpuBuffer& out, size_t channels, size_t seq_len) const;
  // snake (gpu_backend.rs:51-52): out = x + sin^2(alpha_c x) / (alpha_c + 1e-9), x/out f16 [channels,
  // seq_len] (n_elements = channels * seq_len), alpha [channels] f16.
  void snake(const GpuBuffer& x, const GpuBuffer& alpha, const GpuBuffer& out, size_t n_elements, size_t channels,
             size_t seq_len) const;
  // The f32-intermediate path (gpu_backend.rs:134-225): this backend has it.
  bool has_f32_intermediates() const { return true; }
  // conv1d_f32 (:165-177): x f32 [c_in, t_in], w f16 [c_out, c_in, k], bias f16 [c_out] -> f32 [c_out, t_out];
  // stride 1 (the decoder's only stride), t_out must be what padding and dilation give. The decoder passes the
  // same weight buffers on every call: each is packed once (nsr_conv1d_pack_f16) on its first call and the
  // packed copy reused, so later calls are one launch (nsr_conv1d_f16w_packed) and allocate nothing.
  void conv1d_f32(const GpuBuffer& x, const GpuBuffer& w, const GpuBuffer& bias, const GpuBuffer& out, size_t c_in,
                  size_t c_out, size_t t_in, size_t t_out, size_t k, size_t stride, size_t padding,
                  size_t dilation) const;
  // Drop the packed weights conv1d_f32 keeps (for a caller that rewrites a weight buffer in place).
  void forget_conv_weights() const;
  // add_f32 (:186-190), scale_third_f32 (:191-195), leaky_relu_f32 (:196-200): f32 elementwise over n.
  void add_f32(const GpuBuffer& a, const GpuBuffer& b, const GpuBuffer& out, size_t n) const;
  void scale_third_f32(const GpuBuffer& x, const GpuBuffer& out, size_t n) const;
  void leaky_relu_f32(const GpuBuffer& x, const GpuBuffer& out, size_t n, float slope) const;
  // istft_gpu (:220-225): conv_post output [22, n_frames] f32 -> audio [out_len] f32 (n_fft 20, hop 5).
  void istft_gpu(const GpuBuffer& x, const GpuBuffer& out, size_t n_frames, size_t out_len) const;

 private:
  struct PackedConvWeight {
    const void* w;
    size_t c_out, c_in, k;
    Tensor packed;
  };
  struct ConvWeightCache {
    std::mutex mu;
    std::vector<PackedConvWeight> entries;
  };
  RocmDevice device_;
  RocmKernels kernels_;
  std::shared_ptr<ConvWeightCache> conv_weights_;
};

// ---- Embedding and rotary (model-side entry points the GPU also serves) ------

// GGUF Q8_0 embedding table on the device (QEmbedding, quantized_layers.rs).
class QEmbedding {
 public:
  // table: U8 bytes of vocab rows x hidden/32 blocks {f16 d; i8 qs[32]}.
  QEmbedding(const RocmDevice& device, const RocmKernels& kernels, Tensor table, size_t vocab, size_t hidden);
  size_t hidden_size() const { return hidden_; }
  // indexes: U32 or I64 device tensor of any shape -> f32 [..., hidden].
  // An index outside [0, vocab) is an error (as Candle's index_select).
  Tensor forward(const Tensor& indexes) const;

 private:
  RocmDevice device_;
  RocmKernels kernels_;
  Tensor table_;
  size_t vocab_, hidden_;
};

// inv_freq and the f32 cos/sin table of RotaryEmbedding::new, built on the
// host with the reference's f32 operations (decoder.rs:85-95).
class RotaryEmbedding {
 public:
  RotaryEmbedding(const RocmDevice& device, const RocmKernels& kernels, size_t rotary_dim, size_t max_positions,
                  float theta);
  size_t rotary_dim() const { return rotary_dim_; }
  const Tensor& table() const { return table_; }  // [max_positions, rotary_dim]: cos | sin
  // apply_rotary_pos_emb for q [B, Hq, T, Dh], k [B, Hk, T, Dh] f32 at
  // positions pos0 .. pos0 + T - 1; dims >= rotary_dim pass through.
  std::pair<Tensor, Tensor> apply(const Tensor& q, const Tensor& k, size_t pos0) const;

 private:
  RocmDevice device_;
  RocmKernels kernels_;
  size_t rotary_dim_, max_positions_;
  float theta_;
  Tensor table_;
};

}  // namespace rocm
}  // namespace nspeech
