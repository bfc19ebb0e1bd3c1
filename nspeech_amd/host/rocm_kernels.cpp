// nspeech::rocm host side: see rocm_kernels.h. Every launch goes through the
// C ABI of libnspeech_rocm.so; this file only validates, allocates outputs
// and maps the reference's argument conventions onto that ABI.
#include "rocm_kernels.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

#include "nspeech_rocm.h"

namespace nspeech {
namespace rocm {

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    (void)hipGetLastError();
    throw Error(std::string(what) + ": " + hipGetErrorString(e));
  }
}

void nsr_check(nsr_status st, const char* what) {
  if (st != NSR_OK) throw Error(std::string(what) + ": " + nsr_last_error());
}

nsr_dtype to_nsr(DType d, const char* what) {
  switch (d) {
    case DType::F32: return NSR_F32;
    case DType::F16: return NSR_F16;
    case DType::BF16: return NSR_BF16;
    default: throw Error(std::string(what) + ": unsupported dtype " + dtype_name(d));
  }
}

// The reference's storage check (src/triton_kernels.rs:138 and siblings).
void require_device(std::initializer_list<const Tensor*> ts) {
  for (const Tensor* t : ts)
    if (!t->on_device()) throw Error("All tensors must be on the ROCm device");
}

void require_dtype(const Tensor& t, DType d, const char* what) {
  if (t.dtype() != d)
    throw Error(std::string(what) + ": expected " + dtype_name(d) + ", got " + dtype_name(t.dtype()));
}

void require_elems(const Tensor& t, size_t n, const char* what) {
  if (t.elem_count() < n)
    throw Error(std::string(what) + ": tensor holds " + std::to_string(t.elem_count()) + " elements, need " +
                std::to_string(n));
}

}  // namespace

size_t dtype_size(DType d) {
  switch (d) {
    case DType::F32: case DType::U32: return 4;
    case DType::F16: case DType::BF16: return 2;
    case DType::U8: return 1;
    case DType::I64: return 8;
  }
  return 0;
}

const char* dtype_name(DType d) {
  switch (d) {
    case DType::F32: return "f32";
    case DType::F16: return "f16";
    case DType::BF16: return "bf16";
    case DType::U8: return "u8";
    case DType::U32: return "u32";
    case DType::I64: return "i64";
  }
  return "?";
}

// ---------------------------------------------------------------- device --

RocmDevice::Stream::~Stream() {
  if (s) (void)hipStreamDestroy(s);
}

RocmDevice RocmDevice::create(int ordinal) {
  int n = 0;
  hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (ordinal < 0 || ordinal >= n) throw Error("ROCm device " + std::to_string(ordinal) + " not present");
  hip_check(hipSetDevice(ordinal), "hipSetDevice");
  RocmDevice d;
  d.ordinal_ = ordinal;
  d.stream_ = std::make_shared<Stream>();
  hip_check(hipStreamCreateWithFlags(&d.stream_->s, hipStreamNonBlocking), "hipStreamCreate");
  return d;
}

void RocmDevice::synchronize() const { hip_check(hipStreamSynchronize(stream_->s), "hipStreamSynchronize"); }

// ---------------------------------------------------------------- tensor --

Tensor::Storage::~Storage() {
  if (device && ptr) (void)hipFree(ptr);
}

size_t Tensor::dim(int i) const {
  const int n = (int)shape_.size();
  const int k = i < 0 ? n + i : i;
  if (k < 0 || k >= n) throw Error("dimension index out of range");
  return shape_[k];
}

size_t Tensor::elem_count() const {
  return std::accumulate(shape_.begin(), shape_.end(), (size_t)1, [](size_t a, size_t b) { return a * b; });
}

Tensor Tensor::empty(const RocmDevice& dev, std::vector<size_t> shape, DType dtype) {
  Tensor t;
  t.shape_ = std::move(shape);
  t.dtype_ = dtype;
  t.storage_ = std::make_shared<Storage>();
  t.storage_->device = true;
  hip_check(hipSetDevice(dev.ordinal()), "hipSetDevice");
  const size_t bytes = std::max<size_t>(t.size_bytes(), 16);
  hip_check(hipMalloc(&t.storage_->ptr, bytes), "hipMalloc");
  return t;
}

Tensor Tensor::from_host(const RocmDevice& dev, const void* data, std::vector<size_t> shape, DType dtype) {
  Tensor t = empty(dev, std::move(shape), dtype);
  hip_check(hipMemcpyAsync(t.storage_->ptr, data, t.size_bytes(), hipMemcpyHostToDevice, dev.stream()),
            "upload");
  dev.synchronize();
  return t;
}

Tensor Tensor::cpu(const void* data, std::vector<size_t> shape, DType dtype) {
  Tensor t;
  t.shape_ = std::move(shape);
  t.dtype_ = dtype;
  t.storage_ = std::make_shared<Storage>();
  t.storage_->host.resize(t.size_bytes());
  if (t.size_bytes()) std::memcpy(t.storage_->host.data(), data, t.size_bytes());
  t.storage_->ptr = t.storage_->host.data();
  return t;
}

GpuBuffer Tensor::buffer() const {
  if (!on_device()) throw Error("All tensors must be on the ROCm device");
  return GpuBuffer{storage_->ptr, 0};
}

std::vector<uint8_t> Tensor::to_host_bytes() const {
  std::vector<uint8_t> out(size_bytes());
  if (!storage_ || out.empty()) return out;
  if (storage_->device) {
    hip_check(hipMemcpy(out.data(), storage_->ptr, out.size(), hipMemcpyDeviceToHost), "download");
  } else {
    std::memcpy(out.data(), storage_->host.data(), out.size());
  }
  return out;
}

// --------------------------------------------------------------- kernels --

RocmKernels RocmKernels::load(const RocmDevice& dev) {
  hip_check(hipSetDevice(dev.ordinal()), "hipSetDevice");
  nsr_check(nsr_init(nullptr), "RocmKernels::load");
  RocmKernels k;
  k.kernel_count_ = nsr_kernel_count();
  k.device_ = dev;
  k.gemv_weights_ = std::make_shared<GemvWeightCache>();
  return k;
}

std::pair<const uint32_t*, const uint16_t*> RocmKernels::t4_weight(hipStream_t stream, const void* qs,
                                                                   const void* scales, size_t k, size_t nw,
                                                                   bool glu) const {
  if (!gemv_weights_) throw Error("RocmKernels: not loaded (RocmKernels::load)");
  std::lock_guard<std::mutex> lk(gemv_weights_->mu);
  for (const T4Weight& e : gemv_weights_->entries)
    if (e.qs == qs && e.scales == scales && e.k == k && e.nw == nw && e.glu == glu)
      return {static_cast<const uint32_t*>(e.tq.buffer().at()), static_cast<const uint16_t*>(e.ts.buffer().at())};
  // first call with this weight: pack it once, in stream order before the caller's GEMV
  Tensor tq = Tensor::empty(device_, {k * nw / 4}, DType::U32);
  Tensor ts = Tensor::empty(device_, {k / 32 * nw}, DType::F16);
  nsr_check(nsr_q8_pack_t4(static_cast<const uint32_t*>(qs), static_cast<const uint16_t*>(scales), (int64_t)k,
                           (int64_t)nw, glu ? 1 : 0, static_cast<uint32_t*>(tq.buffer().at()),
                           static_cast<uint16_t*>(ts.buffer().at()), stream),
            "enc_gemv_q8 (t4 packing)");
  gemv_weights_->entries.push_back(T4Weight{qs, scales, k, nw, glu, tq, ts});
  return {static_cast<const uint32_t*>(tq.buffer().at()), static_cast<const uint16_t*>(ts.buffer().at())};
}

void RocmKernels::forget_gemv_weights() const {
  if (!gemv_weights_) return;
  std::lock_guard<std::mutex> lk(gemv_weights_->mu);
  gemv_weights_->entries.clear();
}

size_t RocmKernels::gemv_weights_cached() const {
  if (!gemv_weights_) return 0;
  std::lock_guard<std::mutex> lk(gemv_weights_->mu);
  return gemv_weights_->entries.size();
}

// --------------------------------------------------- Tensor-level (triton_*) --

Tensor triton_layernorm_unit_offset(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                                    const Tensor& gamma, size_t n_rows, size_t n_cols) {
  (void)kernels;
  require_device({&x, &gamma});
  require_elems(x, n_rows * n_cols, "triton_layernorm_unit_offset x");
  require_elems(gamma, n_cols, "triton_layernorm_unit_offset gamma");
  if (gamma.dtype() != DType::F16 && gamma.dtype() != DType::F32)
    throw Error("triton_layernorm_unit_offset: gamma must be f16 or f32");
  Tensor out = Tensor::empty(device, {n_rows, n_cols}, DType::F16);
  nsr_check(nsr_layernorm(x.buffer().at(), to_nsr(x.dtype(), "triton_layernorm_unit_offset"), gamma.buffer().at(),
                          nullptr, to_nsr(gamma.dtype(), "triton_layernorm_unit_offset"), out.buffer().at(), NSR_F16,
                          (int64_t)n_rows, (int64_t)n_cols, (int64_t)n_cols, (int64_t)n_cols, 1e-5f,
                          NSR_LN_UNIT_OFFSET, NSR_ACT_NONE, device.stream()),
            "triton_layernorm_unit_offset");
  return out;
}

Tensor triton_layernorm_bare(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x, size_t n_rows,
                             size_t n_cols) {
  (void)kernels;
  require_device({&x});
  require_elems(x, n_rows * n_cols, "triton_layernorm_bare x");
  Tensor out = Tensor::empty(device, {n_rows, n_cols}, DType::F16);
  nsr_check(nsr_layernorm(x.buffer().at(), to_nsr(x.dtype(), "triton_layernorm_bare"), nullptr, nullptr, NSR_F16,
                          out.buffer().at(), NSR_F16, (int64_t)n_rows, (int64_t)n_cols, (int64_t)n_cols,
                          (int64_t)n_cols, 1e-5f, 0, NSR_ACT_NONE, device.stream()),
            "triton_layernorm_bare");
  return out;
}

Tensor triton_residual_add(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                           const Tensor& residual, size_t n_elements) {
  (void)kernels;
  require_device({&x, &residual});
  require_dtype(x, DType::F16, "triton_residual_add x");
  require_dtype(residual, DType::F16, "triton_residual_add residual");
  require_elems(x, n_elements, "triton_residual_add x");
  require_elems(residual, n_elements, "triton_residual_add residual");
  Tensor out = Tensor::empty(device, x.shape(), DType::F16);
  enc_residual_add(device.stream(), kernels, x.buffer(), residual.buffer(), out.buffer(), n_elements);
  return out;
}

Tensor triton_gelu(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x, size_t n_elements) {
  (void)kernels;
  require_device({&x});
  require_dtype(x, DType::F16, "triton_gelu x");
  require_elems(x, n_elements, "triton_gelu x");
  Tensor out = Tensor::empty(device, x.shape(), DType::F16);
  enc_gelu(device.stream(), kernels, x.buffer(), out.buffer(), n_elements);
  return out;
}

void triton_layernorm_std_f32in(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                                const Tensor& weight, const Tensor& out, size_t n_rows, size_t n_cols) {
  (void)kernels;
  require_device({&x, &weight, &out});
  require_dtype(x, DType::F32, "triton_layernorm_std_f32in x");
  require_dtype(weight, DType::F16, "triton_layernorm_std_f32in weight");
  require_dtype(out, DType::F16, "triton_layernorm_std_f32in out");
  require_elems(x, n_rows * n_cols, "triton_layernorm_std_f32in x");
  require_elems(weight, n_cols, "triton_layernorm_std_f32in weight");
  require_elems(out, n_rows * n_cols, "triton_layernorm_std_f32in out");
  enc_layernorm_std_f32in(device.stream(), kernels, x.buffer(), weight.buffer(), out.buffer(), n_rows, n_cols);
}

void triton_residual_add_f32(const RocmDevice& device, const RocmKernels& kernels, const Tensor& x,
                             const Tensor& residual, const Tensor& out, size_t n_elements) {
  (void)kernels;
  require_device({&x, &residual, &out});
  for (const Tensor* t : {&x, &residual, &out}) {
    require_dtype(*t, DType::F32, "triton_residual_add_f32");
    require_elems(*t, n_elements, "triton_residual_add_f32");
  }
  nsr_check(nsr_residual_add(x.buffer().at(), residual.buffer().at(), out.buffer().at(), NSR_F32,
                             (int64_t)n_elements, device.stream()),
            "triton_residual_add_f32");
}

void triton_glu_silu(const RocmDevice& device, const RocmKernels& kernels, const Tensor& fc1, const Tensor& out,
                     size_t n_elements) {
  (void)kernels;
  require_device({&fc1, &out});
  require_dtype(fc1, DType::F16, "triton_glu_silu fc1");
  require_dtype(out, DType::F16, "triton_glu_silu out");
  require_elems(fc1, 2 * n_elements, "triton_glu_silu fc1");
  require_elems(out, n_elements, "triton_glu_silu out");
  nsr_check(nsr_glu_silu(fc1.buffer().at(), out.buffer().at(), NSR_F16, (int64_t)n_elements, device.stream()),
            "triton_glu_silu");
}

void triton_residual_add_layernorm(const RocmDevice& device, const RocmKernels& kernels, const Tensor& f16_proj,
                                   const Tensor& f32_residual, const Tensor& f32_out, const Tensor& weight,
                                   const Tensor& f16_norm, size_t n_rows, size_t dim) {
  (void)kernels;
  require_device({&f16_proj, &f32_residual, &f32_out, &weight, &f16_norm});
  require_dtype(f16_proj, DType::F16, "triton_residual_add_layernorm f16_proj");
  require_dtype(f32_residual, DType::F32, "triton_residual_add_layernorm f32_residual");
  require_dtype(f32_out, DType::F32, "triton_residual_add_layernorm f32_out");
  require_dtype(weight, DType::F16, "triton_residual_add_layernorm weight");
  require_dtype(f16_norm, DType::F16, "triton_residual_add_layernorm f16_norm");
  for (const Tensor* t : {&f16_proj, &f32_residual, &f32_out, &f16_norm})
    require_elems(*t, n_rows * dim, "triton_residual_add_layernorm");
  require_elems(weight, dim, "triton_residual_add_layernorm weight");
  enc_residual_add_layernorm(device.stream(), kernels, f16_proj.buffer(), f32_residual.buffer(), f32_out.buffer(),
                             weight.buffer(), f16_norm.buffer(), n_rows, dim);
}

// ------------------------------------------------------ buffer-level (enc_*) --

void enc_layernorm_std_f32in(Encoder enc, const RocmKernels&, const GpuBuffer& x, const GpuBuffer& weight,
                             const GpuBuffer& out, size_t n_rows, size_t n_cols) {
  nsr_check(nsr_layernorm(x.at(), NSR_F32, weight.at(), nullptr, NSR_F16, out.at(), NSR_F16, (int64_t)n_rows,
                          (int64_t)n_cols, (int64_t)n_cols, (int64_t)n_cols, 1e-5f, 0, NSR_ACT_NONE, enc),
            "enc_layernorm_std_f32in");
}

void enc_residual_add_layernorm(Encoder enc, const RocmKernels&, const GpuBuffer& f16_proj,
                                const GpuBuffer& f32_residual, const GpuBuffer& f32_out, const GpuBuffer& weight,
                                const GpuBuffer& f16_norm, size_t n_rows, size_t dim) {
  nsr_check(nsr_residual_add_layernorm(f16_proj.at(), NSR_F16, f32_residual.at(), NSR_F32, f32_out.at(), NSR_F32,
                                       weight.at(), nullptr, NSR_F16, f16_norm.at(), NSR_F16, (int64_t)n_rows,
                                       (int64_t)dim, 1e-5f, 0, NSR_ACT_NONE, enc),
            "enc_residual_add_layernorm");
}

void enc_layernorm_bare(Encoder enc, const RocmKernels&, const GpuBuffer& x, const GpuBuffer& out, size_t n_rows,
                        size_t n_cols) {
  nsr_check(nsr_layernorm(x.at(), NSR_F16, nullptr, nullptr, NSR_F16, out.at(), NSR_F16, (int64_t)n_rows,
                          (int64_t)n_cols, (int64_t)n_cols, (int64_t)n_cols, 1e-5f, 0, NSR_ACT_NONE, enc),
            "enc_layernorm_bare");
}

void enc_layernorm_unit_offset(Encoder enc, const RocmKernels&, const GpuBuffer& x, const GpuBuffer& gamma,
                               const GpuBuffer& out, size_t n_rows, size_t n_cols) {
  nsr_check(nsr_layernorm(x.at(), NSR_F16, gamma.at(), nullptr, NSR_F16, out.at(), NSR_F16, (int64_t)n_rows,
                          (int64_t)n_cols, (int64_t)n_cols, (int64_t)n_cols, 1e-5f, NSR_LN_UNIT_OFFSET,
                          NSR_ACT_NONE, enc),
            "enc_layernorm_unit_offset");
}

void enc_gelu(Encoder enc, const RocmKernels&, const GpuBuffer& x, const GpuBuffer& out, size_t n_elements) {
  nsr_check(nsr_activation(x.at(), out.at(), NSR_F16, (int64_t)n_elements, NSR_ACT_GELU_ERF, enc), "enc_gelu");
}

void enc_residual_add(Encoder enc, const RocmKernels&, const GpuBuffer& x, const GpuBuffer& residual,
                      const GpuBuffer& out, size_t n_elements) {
  nsr_check(nsr_residual_add(x.at(), residual.at(), out.at(), NSR_F16, (int64_t)n_elements, enc),
            "enc_residual_add");
}

// ------------------------------------------------------------ decoder step --

void enc_rope_qk_cache_fused(Encoder enc, const RocmKernels&, const GpuBuffer& q, const GpuBuffer& k,
                             const GpuBuffer& rope_table, const GpuBuffer& cache_k, size_t pos, size_t max_kv_len,
                             size_t n_q_heads, size_t n_kv_heads, size_t head_dim, size_t rotary_dim) {
  nsr_check(nsr_rope_qk_cache_append(q.at(), k.at(), nullptr, NSR_F16, static_cast<const float*>(rope_table.at()),
                                     (int64_t)max_kv_len, cache_k.at(), nullptr, (int64_t)n_q_heads,
                                     (int64_t)n_kv_heads, (int64_t)head_dim, (int)rotary_dim, (int64_t)pos,
                                     (int64_t)max_kv_len, enc),
            "enc_rope_qk_cache_fused");
}

void triton_attention_decode(const RocmDevice& device, const RocmKernels& kernels, const Tensor& q, const Tensor& k,
                             const Tensor& v, const Tensor& out, size_t kv_len, size_t head_dim, size_t n_kv_heads,
                             size_t n_q_heads, float sm_scale, size_t stride_kv_head, size_t stride_kv_seq) {
  require_device({&q, &k, &v, &out});
  for (const Tensor* t : {&q, &k, &v, &out}) require_dtype(*t, DType::F16, "triton_attention_decode");
  require_elems(q, n_q_heads * head_dim, "triton_attention_decode q");
  require_elems(out, n_q_heads * head_dim, "triton_attention_decode out");
  if (kv_len > 0 && n_kv_heads > 0) {
    const size_t last = (n_kv_heads - 1) * stride_kv_head + (kv_len - 1) * stride_kv_seq + head_dim;
    require_elems(k, last, "triton_attention_decode k");
    require_elems(v, last, "triton_attention_decode v");
  }
  enc_attention_decode(device.stream(), kernels, q.buffer(), k.buffer(), v.buffer(), out.buffer(), kv_len, head_dim,
                       n_kv_heads, n_q_heads, sm_scale, stride_kv_head, stride_kv_seq);
}

void triton_kv_cache_append(const RocmDevice& device, const RocmKernels& kernels, const Tensor& new_kv,
                            const Tensor& cache, size_t n_kv_heads, size_t head_dim, size_t max_kv_len, size_t pos) {
  require_device({&new_kv, &cache});
  require_dtype(new_kv, DType::F16, "triton_kv_cache_append new_kv");
  require_dtype(cache, DType::F16, "triton_kv_cache_append cache");
  require_elems(new_kv, n_kv_heads * head_dim, "triton_kv_cache_append new_kv");
  require_elems(cache, n_kv_heads * max_kv_len * head_dim, "triton_kv_cache_append cache");
  enc_kv_cache_append(device.stream(), kernels, new_kv.buffer(), cache.buffer(), n_kv_heads, head_dim, max_kv_len,
                      pos);
}

void enc_kv_cache_append(Encoder enc, const RocmKernels&, const GpuBuffer& new_kv, const GpuBuffer& cache,
                         size_t n_kv_heads, size_t head_dim, size_t max_kv_len, size_t pos) {
  nsr_check(nsr_kv_cache_append(new_kv.at(), cache.at(), NSR_F16, (int64_t)n_kv_heads, (int64_t)head_dim,
                                (int64_t)max_kv_len, (int64_t)pos, enc),
            "enc_kv_cache_append");
}

void enc_attention_decode(Encoder enc, const RocmKernels&, const GpuBuffer& q, const GpuBuffer& k, const GpuBuffer& v,
                          const GpuBuffer& out, size_t kv_len, size_t head_dim, size_t n_kv_heads, size_t n_q_heads,
                          float sm_scale, size_t stride_kv_head, size_t stride_kv_seq) {
  nsr_check(nsr_attention_decode_f16(q.at(), k.at(), v.at(), out.at(), (int64_t)kv_len, (int64_t)head_dim,
                                     (int64_t)n_kv_heads, (int64_t)n_q_heads, sm_scale, (int64_t)stride_kv_head,
                                     (int64_t)stride_kv_seq, enc),
            "enc_attention_decode");
}

void enc_attention_splitkv(Encoder enc, const RocmKernels&, const GpuBuffer& q, const GpuBuffer& k,
                           const GpuBuffer& v, const GpuBuffer& out, const GpuBuffer& partial_buf, size_t kv_len,
                           size_t head_dim, size_t n_kv_heads, size_t n_q_heads, float sm_scale,
                           size_t stride_kv_head, size_t stride_kv_seq, size_t n_splits) {
  nsr_check(nsr_attention_splitkv_f16(q.at(), k.at(), v.at(), out.at(), static_cast<float*>(partial_buf.at()),
                                      (int64_t)kv_len, (int64_t)head_dim, (int64_t)n_kv_heads, (int64_t)n_q_heads,
                                      sm_scale, (int64_t)stride_kv_head, (int64_t)stride_kv_seq, (int64_t)n_splits,
                                      enc),
            "enc_attention_splitkv");
}

// The three decoder GEMVs multiply with the t4 copy of their weight (RocmKernels::t4_weight: packed on the first
// call with a weight buffer, reused after). x is read 4 elements at a time there; an x not 8-byte aligned takes
// the [K, N/4] kernels on the caller's layout instead.
static bool t4_ok(const GpuBuffer& x) { return (reinterpret_cast<uintptr_t>(x.at()) & 7) == 0; }

void enc_gemv_q8(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                 const GpuBuffer& scales, const GpuBuffer* bias, const GpuBuffer& out, size_t k, size_t n) {
  const float* b = bias ? static_cast<const float*>(bias->at()) : nullptr;
  if (t4_ok(x) && k % 32 == 0 && n % 16 == 0) {
    const auto w = kernels.t4_weight(enc, qs.at(), scales.at(), k, n, false);
    nsr_check(nsr_gemv_q8_t4(x.at(), NSR_F16, w.first, w.second, b, out.at(), NSR_F16, (int64_t)k, (int64_t)n, enc),
              "enc_gemv_q8");
    return;
  }
  nsr_check(nsr_gemv_q8(x.at(), NSR_F16, static_cast<const uint32_t*>(qs.at()), static_cast<const uint16_t*>(scales.at()),
                        b, out.at(), NSR_F16, (int64_t)k, (int64_t)n, enc),
            "enc_gemv_q8");
}

void enc_gemv_q8_bias_glu(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                          const GpuBuffer& scales, const GpuBuffer& bias, const GpuBuffer& out, size_t k, size_t n) {
  if (t4_ok(x) && k % 32 == 0 && n % 16 == 0) {
    const auto w = kernels.t4_weight(enc, qs.at(), scales.at(), k, 2 * n, true);
    nsr_check(nsr_gemv_q8_t4_bias_glu(x.at(), NSR_F16, w.first, w.second, static_cast<const float*>(bias.at()),
                                      out.at(), NSR_F16, (int64_t)k, (int64_t)n, enc),
              "enc_gemv_q8_bias_glu");
    return;
  }
  nsr_check(nsr_gemv_q8_bias_glu(x.at(), NSR_F16, static_cast<const uint32_t*>(qs.at()),
                                 static_cast<const uint16_t*>(scales.at()), static_cast<const float*>(bias.at()),
                                 out.at(), NSR_F16, (int64_t)k, (int64_t)n, enc),
            "enc_gemv_q8_bias_glu");
}

void enc_gemv_q8_resadd_ln(Encoder enc, const RocmKernels& kernels, const GpuBuffer& x, const GpuBuffer& qs,
                           const GpuBuffer& scales, const GpuBuffer& residual, const GpuBuffer& out_f32,
                           const GpuBuffer& ln_weight, const GpuBuffer& norm, size_t k, size_t dim, float eps) {
  if (t4_ok(x) && k % 32 == 0 && dim % 16 == 0) {
    const auto w = kernels.t4_weight(enc, qs.at(), scales.at(), k, dim, false);
    nsr_check(nsr_gemv_q8_t4_resadd_ln(x.at(), NSR_F16, w.first, w.second, static_cast<const float*>(residual.at()),
                                       static_cast<float*>(out_f32.at()), ln_weight.at(), NSR_F16, norm.at(), NSR_F16,
                                       (int64_t)k, (int64_t)dim, eps, enc),
              "enc_gemv_q8_resadd_ln");
    return;
  }
  nsr_check(nsr_gemv_q8_resadd_ln(x.at(), NSR_F16, static_cast<const uint32_t*>(qs.at()),
                                  static_cast<const uint16_t*>(scales.at()), static_cast<const float*>(residual.at()),
                                  static_cast<float*>(out_f32.at()), ln_weight.at(), NSR_F16, norm.at(), NSR_F16,
                                  (int64_t)k, (int64_t)dim, eps, enc),
            "enc_gemv_q8_resadd_ln");
}

// ---------------------------------------------------------------- Kokoro --

void RocmKokoroBackend::adain_snake_f32(const GpuBuffer& x, const GpuBuffer& gamma, const GpuBuffer& beta,
                                        const GpuBuffer& alpha, const GpuBuffer& out, size_t channels,
                                        size_t seq_len) const {
  nsr_check(nsr_adain_snake_f32(static_cast<const float*>(x.at()), gamma.at(), beta.at(), alpha.at(), NSR_F16, 0, 0,
                                static_cast<float*>(out.at()), 1, (int64_t)channels, (int64_t)seq_len, 1e-5f,
                                device_.stream()),
            "adain_snake_f32");
}

void RocmKokoroBackend::adain_snake(const GpuBuffer& x, const GpuBuffer& gamma, const GpuBuffer& beta,
                                    const GpuBuffer& alpha, const GpuBuffer& out, size_t channels,
                                    size_t seq_len) const {
  nsr_check(nsr_adain_snake_f16(x.at(), gamma.at(), beta.at(), alpha.at(), NSR_F16, 0, 0, out.at(), 1,
                                (int64_t)channels, (int64_t)seq_len, 1e-5f, device_.stream()),
            "adain_snake");
}

void RocmKokoroBackend::snake(const GpuBuffer& x, const GpuBuffer& alpha, const GpuBuffer& out, size_t n_elements,
                              size_t channels, size_t seq_len) const {
  nsr_check(nsr_snake(x.at(), NSR_F16, alpha.at(), NSR_F16, out.at(), (int64_t)n_elements, (int64_t)channels,
                      (int64_t)seq_len, device_.stream()),
            "snake");
}

void RocmKokoroBackend::conv1d_f32(const GpuBuffer& x, const GpuBuffer& w, const GpuBuffer& bias,
                                   const GpuBuffer& out, size_t c_in, size_t c_out, size_t t_in, size_t t_out,
                                   size_t k, size_t stride, size_t padding, size_t dilation) const {
  if ((int64_t)t_out != (int64_t)t_in + 2 * (int64_t)padding - (int64_t)dilation * ((int64_t)k - 1))
    throw Error("conv1d_f32: t_out does not match t_in, k, padding and dilation");
  if (stride != 1) throw Error("conv1d_f32: only stride 1 is built");
  const void* packed = nullptr;
  {
    std::lock_guard<std::mutex> lk(conv_weights_->mu);
    for (const PackedConvWeight& e : conv_weights_->entries)
      if (e.w == w.at() && e.c_out == c_out && e.c_in == c_in && e.k == k) packed = e.packed.buffer().at();
    if (!packed) {
      // first call with this weight buffer: pack it once, in stream order before the conv below
      Tensor t = Tensor::empty(device_, {c_out, k, c_in}, DType::F16);
      nsr_check(nsr_conv1d_pack_f16(w.at(), (int64_t)c_out, (int64_t)c_in, (int64_t)k, t.buffer().at(),
                                    device_.stream()),
                "conv1d_f32");
      packed = t.buffer().at();
      conv_weights_->entries.push_back(PackedConvWeight{w.at(), c_out, c_in, k, t});
    }
  }
  nsr_check(nsr_conv1d_f16w_packed(static_cast<const float*>(x.at()), packed, bias.at(), nullptr,
                                   static_cast<float*>(out.at()), 1, (int64_t)c_in, (int64_t)c_out, (int64_t)t_in,
                                   (int64_t)k, (int64_t)padding, (int64_t)dilation, device_.stream()),
            "conv1d_f32");
}

void RocmKokoroBackend::forget_conv_weights() const {
  std::lock_guard<std::mutex> lk(conv_weights_->mu);
  conv_weights_->entries.clear();
}

void RocmKokoroBackend::add_f32(const GpuBuffer& a, const GpuBuffer& b, const GpuBuffer& out, size_t n) const {
  nsr_check(nsr_residual_add(a.at(), b.at(), out.at(), NSR_F32, (int64_t)n, device_.stream()), "add_f32");
}

void RocmKokoroBackend::scale_third_f32(const GpuBuffer& x, const GpuBuffer& out, size_t n) const {
  nsr_check(nsr_scale_f32(static_cast<const float*>(x.at()), static_cast<float*>(out.at()), (int64_t)n,
                          (float)0.3333333333333333, device_.stream()),
            "scale_third_f32");
}

void RocmKokoroBackend::leaky_relu_f32(const GpuBuffer& x, const GpuBuffer& out, size_t n, float slope) const {
  nsr_check(nsr_leaky_relu_f32(static_cast<const float*>(x.at()), static_cast<float*>(out.at()), (int64_t)n, slope,
                               device_.stream()),
            "leaky_relu_f32");
}

void RocmKokoroBackend::istft_gpu(const GpuBuffer& x, const GpuBuffer& out, size_t n_frames, size_t out_len) const {
  nsr_check(nsr_istft_f32(static_cast<const float*>(x.at()), static_cast<float*>(out.at()), (int64_t)n_frames,
                          (int64_t)out_len, 20, 5, device_.stream()),
            "istft_gpu");
}

// ------------------------------------------------------------- embedding --

QEmbedding::QEmbedding(const RocmDevice& device, const RocmKernels& kernels, Tensor table, size_t vocab,
                       size_t hidden)
    : device_(device), kernels_(kernels), table_(std::move(table)), vocab_(vocab), hidden_(hidden) {
  require_device({&table_});
  require_dtype(table_, DType::U8, "QEmbedding table");
  if (hidden % 32 != 0) throw Error("QEmbedding: hidden size must be a multiple of 32 (Q8_0 blocks)");
  if (table_.size_bytes() < vocab * (hidden / 32) * 34) throw Error("QEmbedding: table smaller than vocab rows");
}

Tensor QEmbedding::forward(const Tensor& indexes) const {
  require_device({&indexes});
  if (indexes.dtype() != DType::U32 && indexes.dtype() != DType::I64)
    throw Error("QEmbedding::forward: indexes must be u32 or i64");
  std::vector<size_t> shape = indexes.shape();
  shape.push_back(hidden_);
  Tensor out = Tensor::empty(device_, shape, DType::F32);
  Tensor flag = Tensor::empty(device_, {1}, DType::U32);
  hip_check(hipMemsetAsync(flag.buffer().at(), 0, 4, device_.stream()), "hipMemsetAsync");
  nsr_check(nsr_q8_0_embed_gather(table_.buffer().at(), (int64_t)vocab_, (int64_t)hidden_, indexes.buffer().at(),
                                  indexes.dtype() == DType::I64 ? NSR_IDX_I64 : NSR_IDX_U32,
                                  (int64_t)indexes.elem_count(), static_cast<float*>(out.buffer().at()),
                                  NSR_ACT_NONE, static_cast<int32_t*>(flag.buffer().at()), device_.stream()),
            "QEmbedding::forward");
  device_.synchronize();
  if (flag.to_vec<uint32_t>()[0] != 0)
    throw Error("QEmbedding::forward: index out of range for vocabulary of " + std::to_string(vocab_));
  return out;
}

// ---------------------------------------------------------------- rotary --

RotaryEmbedding::RotaryEmbedding(const RocmDevice& device, const RocmKernels& kernels, size_t rotary_dim,
                                 size_t max_positions, float theta)
    : device_(device), kernels_(kernels), rotary_dim_(rotary_dim), max_positions_(max_positions), theta_(theta) {
  std::vector<float> host(max_positions * rotary_dim);
  nsr_check(nsr_rope_table_f32(host.data(), (int64_t)max_positions, (int)rotary_dim, theta), "RotaryEmbedding");
  table_ = Tensor::from_host(device, host.data(), {max_positions, rotary_dim}, DType::F32);
}

std::pair<Tensor, Tensor> RotaryEmbedding::apply(const Tensor& q, const Tensor& k, size_t pos0) const {
  require_device({&q, &k});
  require_dtype(q, DType::F32, "apply_rotary_pos_emb q");
  require_dtype(k, DType::F32, "apply_rotary_pos_emb k");
  if (q.shape().size() != 4 || k.shape().size() != 4)
    throw Error("apply_rotary_pos_emb: q and k must be [batch, heads, seq_len, head_dim]");
  if (q.dim(0) != k.dim(0) || q.dim(2) != k.dim(2) || q.dim(3) != k.dim(3))
    throw Error("apply_rotary_pos_emb: q and k shapes disagree");
  if (pos0 + q.dim(2) > max_positions_) throw Error("apply_rotary_pos_emb: positions beyond the RoPE table");
  Tensor qo = Tensor::empty(device_, q.shape(), DType::F32);
  Tensor ko = Tensor::empty(device_, k.shape(), DType::F32);
  nsr_check(nsr_rotary_partial_interleaved_f32(
                static_cast<const float*>(q.buffer().at()), static_cast<const float*>(k.buffer().at()),
                static_cast<float*>(qo.buffer().at()), static_cast<float*>(ko.buffer().at()), (int64_t)q.dim(0),
                (int64_t)q.dim(1), (int64_t)k.dim(1), (int64_t)q.dim(2), (int64_t)q.dim(3), (int)rotary_dim_, theta_,
                (int64_t)pos0, static_cast<const float*>(table_.buffer().at()), (int64_t)max_positions_,
                device_.stream()),
            "apply_rotary_pos_emb");
  return {qo, ko};
}

}  // namespace rocm
}  // namespace nspeech
