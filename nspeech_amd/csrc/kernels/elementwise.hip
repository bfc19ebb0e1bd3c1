/*
 * Elementwise kernels: SiLU / GELU(erf) activation, GLU-SiLU, residual add.
 *
 * Reference semantics:
 *   gelu_erf: x * 0.5 * (1 + erf(x / sqrt(2)))  (Tensor::gelu_erf,
 *     src/moonshine/encoder.rs:106; gelu_forward kernels/moonshine_kernels.py:388-400)
 *   silu: x / (1 + exp(-x))  (candle_nn::ops::silu, src/moonshine/decoder.rs:409;
 *     silu kernels/moonshine_kernels.py:96-98)
 *   glu_silu: out[i] = silu(fc1[n + i]) * fc1[i]  (glu_silu_fused,
 *     kernels/moonshine_kernels.py:846-862; DecoderMLP::forward decoder.rs:403-411)
 *   residual add: out = x + res  (FastAddOp, src/fast_ops.rs:16-36)
 *   combine (f32): out = lrelu?(((a + b) + c) * scale), the Kokoro
 *     generator's resblock average and conv_post input, as the reference GPU
 *     path computes it in four dispatches: add_f32 (r0 + r1), add_f32 (+ r2),
 *     scale_third_f32 (x * f32(1/3), kernels/kokoro_kernels.py:941-969) and
 *     leaky_relu_f32 (x > 0 ? x : x * slope) (src/kokoro/decoder.rs:540-577,
 *     src/kokoro/gpu_backend.rs:186-200); one pass here, same rounding
 *     sequence.
 *
 *   snake (f32 or f16): out = x + sin^2(alpha_c x) / (alpha_c + 1e-9), one alpha
 *     per channel of x [rows, T] (KokoroGpuBackend::snake,
 *     src/kokoro/gpu_backend.rs:51-52; snake_activation
 *     kernels/kokoro_kernels.py:24-55; snake_activation_tensor
 *     src/kokoro/decoder.rs:1471-1476).
 *
 * One lane per 16-byte chunk (4 f32 or 8 f16/bf16 elements), flat grid,
 * arithmetic in f32 and one rounding to the storage dtype. The _s variants
 * take one element per lane for unaligned pointers and ragged tails.
 */
#include "device_common.h"

template <int DT, int ACT>
NSR_DEV void act_vec(const nsr_ew_args& a) {
  constexpr int VEC = 16 / dt_size<DT>::value;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n / VEC) return;
  float v[VEC];
  unpack16<DT>(ld16((const char*)a.a + i * 16), v);
#pragma unroll
  for (int e = 0; e < VEC; ++e) v[e] = apply_act<ACT>(v[e]);
  st16((char*)a.out + i * 16, pack16<DT>(v));
}

template <int DT, int ACT>
NSR_DEV void act_scalar(const nsr_ew_args& a, int64_t first) {
  const int64_t i = first + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  store_scalar<DT>(a.out, i, apply_act<ACT>(load_scalar<DT>(a.a, i)));
}

template <int DT>
NSR_DEV void glu_vec(const nsr_ew_args& a) {
  constexpr int VEC = 16 / dt_size<DT>::value;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n / VEC) return;
  float x[VEC], g[VEC];
  unpack16<DT>(ld16((const char*)a.a + i * 16), x);
  unpack16<DT>(ld16((const char*)a.a + (a.n * dt_size<DT>::value) + i * 16), g);
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] = act_silu(g[e]) * x[e];
  st16((char*)a.out + i * 16, pack16<DT>(x));
}

template <int DT>
NSR_DEV void glu_scalar(const nsr_ew_args& a, int64_t first) {
  const int64_t i = first + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  const float x = load_scalar<DT>(a.a, i);
  const float g = load_scalar<DT>(a.a, a.n + i);
  store_scalar<DT>(a.out, i, act_silu(g) * x);
}

template <int DT>
NSR_DEV void add_vec(const nsr_ew_args& a) {
  constexpr int VEC = 16 / dt_size<DT>::value;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n / VEC) return;
  float x[VEC], r[VEC];
  unpack16<DT>(ld16((const char*)a.a + i * 16), x);
  unpack16<DT>(ld16((const char*)a.b + i * 16), r);
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] = x[e] + r[e];
  st16((char*)a.out + i * 16, pack16<DT>(x));
}

template <int DT>
NSR_DEV void add_scalar(const nsr_ew_args& a, int64_t first) {
  const int64_t i = first + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  store_scalar<DT>(a.out, i, load_scalar<DT>(a.a, i) + load_scalar<DT>(a.b, i));
}

/* Vector kernels cover n - n % VEC elements; the scalar kernels take `first`
 * (the first element they handle) so the host can launch them for the tail. */
#define NSR_EW_SET(DN, DT)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) nsrk_silu_##DN##_v(const nsr_ew_args a) { \
    act_vec<DT, ACT_SILU>(a);                                                               \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gelu_##DN##_v(const nsr_ew_args a) { \
    act_vec<DT, ACT_GELU>(a);                                                               \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                         \
      nsrk_silu_##DN##_s(const nsr_ew_args a, const int64_t first) {                        \
    act_scalar<DT, ACT_SILU>(a, first);                                                     \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                         \
      nsrk_gelu_##DN##_s(const nsr_ew_args a, const int64_t first) {                        \
    act_scalar<DT, ACT_GELU>(a, first);                                                     \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256) nsrk_glu_##DN##_v(const nsr_ew_args a) {  \
    glu_vec<DT>(a);                                                                         \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                         \
      nsrk_glu_##DN##_s(const nsr_ew_args a, const int64_t first) {                         \
    glu_scalar<DT>(a, first);                                                               \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256) nsrk_add_##DN##_v(const nsr_ew_args a) {  \
    add_vec<DT>(a);                                                                         \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                         \
      nsrk_add_##DN##_s(const nsr_ew_args a, const int64_t first) {                         \
    add_scalar<DT>(a, first);                                                               \
  }

NSR_EW_SET(f32, DT_F32)
NSR_EW_SET(f16, DT_F16)
NSR_EW_SET(bf16, DT_BF16)

/* ----------------------------------------------------------- combine -- */

NSR_DEV float combine_one(const nsr_combine_args& a, float x, float y, float z) {
  float v = x;
  if (a.b) v = v + y;
  if (a.c) v = v + z;
  if (a.flags & 1) v = v * a.scale;
  if (a.flags & 2) v = v > 0.f ? v : v * a.slope;
  return v;
}

/* one lane per 4 elements (16-byte aligned pointers) */
extern "C" __global__ void __launch_bounds__(256) nsrk_combine_f32_v(const nsr_combine_args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n / 4) return;
  const nsr_float4 x = ldf4(a.a + 4 * i);
  const nsr_float4 y = a.b ? ldf4(a.b + 4 * i) : x;
  const nsr_float4 z = a.c ? ldf4(a.c + 4 * i) : x;
  nsr_float4 o;
  o.x = combine_one(a, x.x, y.x, z.x);
  o.y = combine_one(a, x.y, y.y, z.y);
  o.z = combine_one(a, x.z, y.z, z.z);
  o.w = combine_one(a, x.w, y.w, z.w);
  stf4(a.out + 4 * i, o);
}

extern "C" __global__ void __launch_bounds__(256) nsrk_combine_f32_s(const nsr_combine_args a, const int64_t first) {
  const int64_t i = first + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n) return;
  a.out[i] = combine_one(a, a.a[i], a.b ? a.b[i] : 0.f, a.c ? a.c[i] : 0.f);
}

/* ------------------------------------------------------------- snake -- */

/* Workgroup = (row, 1024-element chunk of the row): the row's alpha and the
 * snake polynomial are set up once per workgroup; lanes take elements
 * t0 + 256 k (coalesced, any alignment). */
template <int DT>
NSR_DEV void snake_body(const nsr_snake_args& a) {
  const int64_t blk = blockIdx.x;
  const int64_t row = blk / a.chunks;
  const int64_t ch = blk - row * a.chunks;
  const int64_t c = row % a.C;
  const float alp = a.pdt == DT_F32 ? ((const float*)a.alpha)[c] : f16_bits_to_f32(((const uint16_t*)a.alpha)[c]);
  const snake_consts sc = make_snake_consts(alp);
  const int64_t base = row * a.T;
  const int64_t t0 = ch * 1024 + threadIdx.x;
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t t = t0 + 256 * k;
    v[k] = t < a.T ? load_scalar<DT>(a.x, base + t) : 0.f;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t t = t0 + 256 * k;
    if (t < a.T) store_scalar<DT>(a.out, base + t, snake_eval(v[k], sc));
  }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_snake_f32(const nsr_snake_args a) { snake_body<DT_F32>(a); }
extern "C" __global__ void __launch_bounds__(256) nsrk_snake_f16(const nsr_snake_args a) { snake_body<DT_F16>(a); }
