/*
 * nsr_oracle.c - CPU oracle for the fused layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, as a checker or as the
 * timed CPU baseline. The product (libnspeech_rocm.so) never calls it.
 *
 * Each function restates, in plain C and op for op, the CPU computation the
 * reference performs for one hot-path op (paths relative to the
 * dropbox/nspeech tree). The reference's CPU path is Rust on Candle, which is
 * not available here, so Candle's own op internals are restated from its
 * documented behaviour: every tensor op rounds its f32 result once, reductions
 * accumulate sequentially in f32, `t / n` and `t + c` on a tensor scale by the
 * f32 constant (affine). Parity of these restatements is pinned in tests
 * against library routines (torch f64 layer_norm / instance_norm / gelu /
 * silu, numpy complex rotation, numpy float16/bf16 conversion) and f64 closed
 * forms, and by invariants.
 *
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off -fopenmp). No FMA
 * contraction, no fast-math: every product and sum rounds as the Rust code's.
 * `nthreads` > 1 splits independent rows over OpenMP threads (same results).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------ f16 / bf16 ----- */

/* IEEE binary16 -> f32 (exact). half crate f16::to_f32 (Cargo.toml:88). */
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float v = (float)man * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* f32 -> bf16 round-to-nearest-even (half crate bf16::from_f32). */
static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* f64 -> bf16 RNE directly (half crate bf16::from_f64), used where Candle
 * evaluates a bf16 op in f64 (gelu_erf). Rounds to f32 with round-to-odd
 * (truncate toward zero, set the last bit when inexact), then to bf16 with
 * RNE: f32 keeps >= 2 more bits than bf16, so the two steps equal one RNE. */
static uint16_t f64_to_bf16(double d) {
  if (d != d) return 0x7fc0u;
  float f = (float)d;
  if ((double)f != d) {
    if (fabs((double)f) > fabs(d)) f = nextafterf(f, 0.0f);
    uint32_t u;
    memcpy(&u, &f, 4);
    u |= 1u;
    memcpy(&f, &u, 4);
  }
  return f32_to_bf16(f);
}

/* f32 -> IEEE binary16, round to nearest even (half crate f16::from_f32;
 * Triton's .to(tl.float16)); overflow to inf, NaN kept quiet. */
static uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (ax < 0x38800000u) {                                  /* |f| < 2^-14: subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign;           /* < 2^-25: rounds to 0 */
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;                       /* 14 - (e - 127) + 13 - 1 ... */
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

ORC_API void orc_f32_to_f16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}

ORC_API void orc_f16_to_f32(const uint16_t* h, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(h[i]);
}
ORC_API void orc_f32_to_bf16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(x[i]);
}
ORC_API void orc_bf16_to_f32(const uint16_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(x[i]);
}

/* ----------------------------------------------------------- Q8_0 ----- */

/* QTensor::dequantize for GGML Q8_0: a block is {f16 d; int8 qs[32]} and
 * y[32*b + j] = qs[j] * d (GGUF block_q8_0; producer
 * tools/quantize-moonshine/src/main.rs:69,121). Whole table, as
 * QEmbedding::forward does (src/parakeet/quantized_layers.rs:69). */
ORC_API void orc_q8_0_dequantize(const uint8_t* blocks, int64_t vocab, int64_t d, float* out) {
  const int64_t nb = d / 32;
  for (int64_t r = 0; r < vocab; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* bp = blocks + (r * nb + b) * 34;
      uint16_t hd;
      memcpy(&hd, bp, 2);
      const float dd = f16_to_f32(hd);
      for (int j = 0; j < 32; ++j) out[r * d + b * 32 + j] = (float)(int8_t)bp[2 + j] * dd;
    }
  }
}

/* index_select(ids, 0) of a dense [vocab, d] table
 * (src/parakeet/quantized_layers.rs:70). Returns the number of ids out of
 * range; their rows are zero-filled (Candle raises an error instead). */
ORC_API int64_t orc_index_select_rows(const float* table, int64_t vocab, int64_t d, const int64_t* ids,
                                      int64_t n, float* out) {
  int64_t bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t id = ids[i];
    if (id < 0 || id >= vocab) {
      ++bad;
      memset(out + i * d, 0, (size_t)d * sizeof(float));
    } else {
      memcpy(out + i * d, table + id * d, (size_t)d * sizeof(float));
    }
  }
  return bad;
}

/* ------------------------------------------------------ activations --- */

/* candle silu on f32: v / (1 + exp(-v)) (candle_nn::ops::silu,
 * src/moonshine/decoder.rs:409; Tensor::silu src/parakeet/fast_conformer.rs:207) */
static float silu_f32(float v) { return v / (1.0f + expf(-v)); }

/* candle gelu_erf on f32 evaluates in f64 and rounds once:
 * (erf(v / sqrt 2) + 1) * 0.5 * v (Tensor::gelu_erf, src/moonshine/encoder.rs:106) */
static double gelu_erf_f64(double v) { return (erf(v / sqrt(2.0)) + 1.0) * 0.5 * v; }
static float gelu_erf_f32(float v) { return (float)gelu_erf_f64((double)v); }

ORC_API void orc_silu_f32(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = silu_f32(x[i]);
}
ORC_API void orc_gelu_erf_f32(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = gelu_erf_f32(x[i]);
}

/* GLU of DecoderMLP::forward (src/moonshine/decoder.rs:406-409):
 * silu(gate).mul(x_part), fc1 = [x_part | gate]. */
ORC_API void orc_glu_silu_f32(const float* fc1, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = silu_f32(fc1[n + i]) * fc1[i];
}

/* FastAddOp::cpu_fwd (src/fast_ops.rs:32-34): dst[i] = a[i] + b[i]. */
ORC_API void orc_fast_add_f32(const float* a, const float* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* Q8_0 embedding as the reference computes it: dequantize the whole table,
 * index_select, then (act == 1) silu. `table_scratch` holds vocab * d f32. */
ORC_API int64_t orc_q8_0_embedding(const uint8_t* blocks, int64_t vocab, int64_t d, const int64_t* ids,
                                   int64_t n, int act, float* table_scratch, float* out) {
  orc_q8_0_dequantize(blocks, vocab, d, table_scratch);
  const int64_t bad = orc_index_select_rows(table_scratch, vocab, d, ids, n, out);
  if (act == 1) orc_silu_f32(out, out, n * d);
  if (act == 2) orc_gelu_erf_f32(out, out, n * d);
  return bad;
}

/* ------------------------------------------------------- LayerNorm ----- */

/* candle_nn::LayerNorm::forward on a contiguous f32 tensor with bias
 * (Parakeet conformer, src/parakeet/fast_conformer.rs:721-725,778-782) takes
 * candle_nn::ops::layer_norm, whose CPU kernel is one pass over the row:
 * sum and sum of squares in f32, var = sum2/n - mean^2,
 * y = (x - mean) * (1/sqrt(var + eps)) * w + b. (Candle internals recalled,
 * not available here; pinned against torch layer_norm in f64.) */
ORC_API void orc_layernorm_candle_f32(const float* x, const float* w, const float* b, float* y, int64_t rows,
                                      int64_t cols, float eps, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    float sum = 0.0f, sum2 = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const float v = xr[c];
      sum += v;
      sum2 += v * v;
    }
    const float mean = sum / (float)cols;
    const float var = sum2 / (float)cols - mean * mean;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t c = 0; c < cols; ++c) {
      const float wv = w ? w[c] : 1.0f;
      const float bv = b ? b[c] : 0.0f;
      yr[c] = (xr[c] - mean) * inv_std * wv + bv;
    }
  }
}

/* Explicit two-pass LayerNorm of the Moonshine encoder/decoder
 * (UnitOffsetLayerNorm::forward src/moonshine/encoder.rs:68-76,
 * LayerNorm::forward src/moonshine/decoder.rs:67-74), as Candle tensor ops:
 *   mean = sum_keepdim * f32(1/n); xc = x - mean; var = sum(xc*xc) * f32(1/n)
 *   std = sqrt(var + eps); normed = xc / std; out = normed * scale (+ beta)
 * scale = w + 1 when unit_offset (affine(1, 1) on the weight), w otherwise. */
ORC_API void orc_layernorm_twopass_f32(const float* x, const float* w, const float* b, float* y, int64_t rows,
                                       int64_t cols, float eps, int unit_offset, int nthreads) {
  const float inv_n = (float)(1.0 / (double)cols);
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    float sum = 0.0f;
    for (int64_t c = 0; c < cols; ++c) sum += xr[c];
    const float mean = sum * inv_n;
    float sq = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const float d = xr[c] - mean;
      sq += d * d;
    }
    const float var = sq * inv_n;
    const float std = sqrtf(var + eps);
    for (int64_t c = 0; c < cols; ++c) {
      const float normed = (xr[c] - mean) / std;
      float scale = w ? w[c] : 1.0f;
      if (unit_offset) scale = scale + 1.0f;
      float o = normed * scale;
      if (b) o = o + b[c];
      yr[c] = o;
    }
  }
}

/* bf16 chain for config 4a, as unfused Candle bf16 tensor ops would run it:
 *   h = x + res                (half crate bf16 add: f32 add, one rounding;
 *                               fast_add's loop src/fast_ops.rs:32-34)
 *   n = layer_norm(h, w, b)    (candle ops::layer_norm in f32 over the bf16
 *                               values, one rounding to bf16; w, b are bf16)
 *   y = gelu_erf(n)            (evaluated in f64, rounded to bf16)
 * w_bf16/b_bf16 are the bf16 weights. h_out may be NULL. */
ORC_API void orc_resadd_ln_gelu_bf16(const uint16_t* x, const uint16_t* res, const uint16_t* w_bf16,
                                     const uint16_t* b_bf16, uint16_t* h_out, uint16_t* y, int64_t rows,
                                     int64_t cols, float eps, int gelu, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * cols;
    const uint16_t* rr = res + r * cols;
    float sum = 0.0f, sum2 = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const uint16_t hb = f32_to_bf16(bf16_to_f32(xr[c]) + bf16_to_f32(rr[c]));
      if (h_out) h_out[r * cols + c] = hb;
      const float v = bf16_to_f32(hb);
      sum += v;
      sum2 += v * v;
    }
    const float mean = sum / (float)cols;
    const float var = sum2 / (float)cols - mean * mean;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t c = 0; c < cols; ++c) {
      const float v = bf16_to_f32(f32_to_bf16(bf16_to_f32(xr[c]) + bf16_to_f32(rr[c])));
      const float wv = bf16_to_f32(w_bf16[c]);
      const float bv = bf16_to_f32(b_bf16[c]);
      const uint16_t nb = f32_to_bf16((v - mean) * inv_std * wv + bv);
      y[r * cols + c] = gelu ? f64_to_bf16(gelu_erf_f64((double)bf16_to_f32(nb))) : nb;
    }
  }
}

/* --------------------------------------------------------- rotary ------ */

/* inv_freq[i] = 1 / theta^(2i/dim), f32 ops (src/moonshine/decoder.rs:90-92). */
static float inv_freq_f32(int i, int dim, float theta) {
  const float e = (2.0f * (float)i) / (float)dim;
  return 1.0f / powf(theta, e);
}

/* GPU RoPE table of src/moonshine/gpu_decoder.rs:326-340:
 * row p = [cos(p*f_0..f_{h-1}) | sin(p*f_0..f_{h-1})], f32. */
ORC_API void orc_rope_table_f32(float* table, int64_t max_pos, int rot, float theta) {
  const int half = rot / 2;
  for (int i = 0; i < half; ++i) {
    const float f = inv_freq_f32(i, rot, theta);
    for (int64_t p = 0; p < max_pos; ++p) {
      const float angle = (float)p * f;
      table[p * 2 * half + i] = cosf(angle);
      table[p * 2 * half + half + i] = sinf(angle);
    }
  }
}

/* RotaryEmbedding::forward + apply_rotary_pos_emb (src/moonshine/decoder.rs:
 * 100-111, 115-131, 133-183) for one tensor [B, H, T, Dh], positions
 * pos0 + t: angle = inv_freq * f32(pos) (one rounding), cos/sin in f32
 * (libm) computed once per position as the reference's cos/sin tensors,
 * out = x_rot * cos_interleaved + rotate_half_interleaved(x_rot) *
 * sin_interleaved (two rounded products, one rounded sum), cat pass-through.
 * `cs_scratch` holds 2 * T * rot/2 floats. */
ORC_API void orc_rotary_f32(const float* x, float* out, int64_t B, int64_t H, int64_t T, int64_t Dh, int rot,
                            float theta, int64_t pos0, float* cs_scratch, int nthreads) {
  const int half = rot / 2;
  float* cs = cs_scratch; /* [T][2][half]: cos then sin */
  for (int i = 0; i < half; ++i) {
    const float f = inv_freq_f32(i, rot, theta);
    for (int64_t t = 0; t < T; ++t) {
      const float angle = f * (float)(pos0 + t);
      cs[t * 2 * half + i] = cosf(angle);
      cs[t * 2 * half + half + i] = sinf(angle);
    }
  }
  const int64_t rows = B * H * T;
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t t = r % T;
    const float* ct = cs + t * 2 * half;
    const float* st = ct + half;
    const float* xr = x + r * Dh;
    float* orow = out + r * Dh;
    for (int i = 0; i < half; ++i) {
      const float c = ct[i], s = st[i];
      const float x0 = xr[2 * i], x1 = xr[2 * i + 1];
      const float p0 = x0 * c, q0 = (-x1) * s;
      const float p1 = x1 * c, q1 = x0 * s;
      orow[2 * i] = p0 + q0;
      orow[2 * i + 1] = p1 + q1;
    }
    for (int64_t dd = rot; dd < Dh; ++dd) orow[dd] = xr[dd];
  }
}

/* ------------------------------------------------- AdaIN1d + Snake ----- */

/* adain (src/kokoro/decoder.rs:1416-1428) then snake_activation_tensor
 * (:1471-1476) as Candle f32 tensor ops, per (b, c) row of x [B, C, T]:
 *   mean = sum * f32(1/T); diff = x - mean; var = sum(diff*diff) * f32(1/T)
 *   norm = diff / sqrt(var + eps); y = norm * (gamma + 1) + beta
 *   ax = y * alpha; s = sin(ax); sin_sq = s * s; inv_a = 1 / (alpha + 1e-9)
 *   out = y + sin_sq * inv_a
 * gamma/beta index b * bstride + c, alpha index c (f32 values; the GPU
 * backend's f16 parameters are widened exactly before the call). */
ORC_API void orc_adain_snake_f32(const float* x, const float* gamma, const float* beta, const float* alpha,
                                 float* out, int64_t B, int64_t C, int64_t T, int64_t gamma_bstride,
                                 int64_t beta_bstride, float eps, int nthreads) {
  const float inv_t = (float)(1.0 / (double)T);
  const int64_t rows = B * C;
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t bi = r / C, ci = r % C;
    const float* xr = x + r * T;
    float* orow = out + r * T;
    float sum = 0.0f;
    for (int64_t t = 0; t < T; ++t) sum += xr[t];
    const float mean = sum * inv_t;
    float sq = 0.0f;
    for (int64_t t = 0; t < T; ++t) {
      const float d = xr[t] - mean;
      sq += d * d;
    }
    const float var = sq * inv_t;
    const float std = sqrtf(var + eps);
    const float scale = gamma[bi * gamma_bstride + ci] + 1.0f;
    const float bt = beta[bi * beta_bstride + ci];
    const float a = alpha[ci];
    const float inv_a = 1.0f / (a + 1e-9f);
    for (int64_t t = 0; t < T; ++t) {
      const float norm = (xr[t] - mean) / std;
      const float y = norm * scale + bt;
      const float ax = y * a;
      const float s = sinf(ax);
      const float sin_sq = s * s;
      orow[t] = y + sin_sq * inv_a;
    }
  }
}

/* ------------------------------------------- decode-step RoPE + KV cache --- */

/* rope_qk_cache_fused (kernels/moonshine_kernels.py:1372-1454, dispatched by
 * enc_rope_qk_cache_fused src/triton_kernels.rs:975) followed by
 * kv_cache_append of v (:865-883, enc_kv_cache_append :993), one decode
 * position, f16 tensors:
 *   q [Hq, Dh], k [Hk, Dh] rotated in place on dims < rot (interleaved pairs,
 *   cos/sin = table[pos][i], table[pos][half + i]); each rotated value is
 *   f16(x0 * c - x1 * s) / f16(x1 * c + x0 * s) with f32 products;
 *   cache_k[h, pos, :] = rotated k row (pass-through dims copied);
 *   cache_v[h, pos, :] = v row (when v and cache_v are given).
 * Caches are [Hk, max_kv_len, Dh]. */
ORC_API void orc_rope_qk_cache_f16(uint16_t* q, uint16_t* k, const uint16_t* v, const float* table, int64_t Hq,
                                   int64_t Hk, int64_t Dh, int rot, int64_t pos, int64_t max_kv_len,
                                   uint16_t* cache_k, uint16_t* cache_v) {
  const int half = rot / 2;
  const float* cs = table + pos * 2 * half;
  for (int64_t pass = 0; pass < 2; ++pass) {
    uint16_t* x = pass == 0 ? q : k;
    const int64_t H = pass == 0 ? Hq : Hk;
    for (int64_t h = 0; h < H; ++h) {
      for (int i = 0; i < half; ++i) {
        const float c = cs[i], sn = cs[half + i];
        const float x0 = f16_to_f32(x[h * Dh + 2 * i]), x1 = f16_to_f32(x[h * Dh + 2 * i + 1]);
        const float p0 = x0 * c, q0 = x1 * sn, p1 = x1 * c, q1 = x0 * sn;
        x[h * Dh + 2 * i] = f32_to_f16(p0 - q0);
        x[h * Dh + 2 * i + 1] = f32_to_f16(p1 + q1);
      }
    }
  }
  for (int64_t h = 0; h < Hk; ++h) {
    memcpy(cache_k + (h * max_kv_len + pos) * Dh, k + h * Dh, (size_t)Dh * 2);
    if (v && cache_v) memcpy(cache_v + (h * max_kv_len + pos) * Dh, v + h * Dh, (size_t)Dh * 2);
  }
}

/* ------------------------------------------------------- Q8 GEMV (M = 1) --- */

/* gemv_q8 / gemv_q8_bias / gemv_q8_bias_glu / gemv_q8_resadd_ln
 * (kernels/moonshine_kernels.py:616-677, 1721-1819), repacked Q8 weights:
 * qs u32 [K, NW/4], the int8 weight of column c in byte c % 4 of word c / 4;
 * scales f16 [K/32, NW]. x f32 [K] (f16 inputs widened exactly). For every
 * column, in k order: acc += (x[k] * q[k, c]) * scale[k / 32, c], in f32.
 * mode 0: out[c] = acc[c] (+ bias[c] when bias != NULL), NW = N columns.
 * mode 1 (GLU, NW = 2N): out[c] = silu(acc[N + c] + bias[N + c]) * (acc[c] + bias[c]),
 *   silu(g) = g * sigmoid(g) in f32 (bias may be NULL).
 * Outputs are f32 before the kernels' final rounding to the output dtype. */
ORC_API void orc_gemv_q8_f32(const float* x, const uint32_t* qs, const uint16_t* scales, const float* bias,
                             float* out, int64_t K, int64_t N, int mode) {
  const int64_t NW = mode == 1 ? 2 * N : N;
  float* acc = mode == 1 ? (float*)malloc((size_t)NW * sizeof(float)) : out; /* mode 0 sums in place */
  for (int64_t c = 0; c < NW; ++c) acc[c] = 0.0f;
  for (int64_t k = 0; k < K; ++k) {
    const float xk = x[k];
    for (int64_t c = 0; c < NW; ++c) {
      const uint32_t w = qs[k * (NW / 4) + c / 4];
      const float q = (float)(int8_t)((w >> (8 * (c % 4))) & 0xffu);
      const float s = f16_to_f32(scales[(k / 32) * NW + c]);
      acc[c] += (xk * q) * s;
    }
  }
  if (mode == 0) {
    if (bias) for (int64_t c = 0; c < N; ++c) out[c] = acc[c] + bias[c];
  } else {
    for (int64_t c = 0; c < N; ++c) {
      const float xv = acc[c] + (bias ? bias[c] : 0.0f);
      const float g = acc[N + c] + (bias ? bias[N + c] : 0.0f);
      const float sg = g * (1.0f / (1.0f + expf(-g)));
      out[c] = sg * xv;
    }
    free(acc);
  }
}

/* gemv_q8_resadd_ln (kernels/moonshine_kernels.py:1775-1819): proj = f16(x @ W),
 * h = proj + residual (f32, written to out_f32), norm = f16(LN(h) * w) with
 * mean, centred variance over dim, eps; returns norm as f16 bits. */
ORC_API void orc_gemv_q8_resadd_ln(const float* x, const uint32_t* qs, const uint16_t* scales,
                                   const float* residual, const uint16_t* ln_w_f16, float* out_f32,
                                   uint16_t* norm_f16, int64_t K, int64_t dim, float eps) {
  float* acc = (float*)malloc((size_t)dim * sizeof(float));
  orc_gemv_q8_f32(x, qs, scales, NULL, acc, K, dim, 0);
  /* mode 0 without bias leaves the sums in acc */
  for (int64_t c = 0; c < dim; ++c) {
    const float proj = f16_to_f32(f32_to_f16(acc[c]));
    out_f32[c] = proj + residual[c];
  }
  float sum = 0.0f;
  for (int64_t c = 0; c < dim; ++c) sum += out_f32[c];
  const float mean = sum / (float)dim;
  float sq = 0.0f;
  for (int64_t c = 0; c < dim; ++c) {
    const float d = out_f32[c] - mean;
    sq += d * d;
  }
  const float inv_std = 1.0f / sqrtf(sq / (float)dim + eps);
  for (int64_t c = 0; c < dim; ++c)
    norm_f16[c] = f32_to_f16((out_f32[c] - mean) * inv_std * f16_to_f32(ln_w_f16[c]));
  free(acc);
}

/* ------------------------------------------------- Kokoro resblock conv --- */

/* conv1d_f32io (kernels/kokoro_kernels.py:773-816) over a batch: x f32
 * [B, C_in, T_in], w f16 [C_out, C_in, K], bias f16 [C_out] (or NULL),
 * out f32 [B, C_out, T_out]; per output acc = 0, then for ck in
 * 0 .. C_in*K-1 (c = ck / K, k = ck % K): t_in = t*stride - padding +
 * k*dilation, acc += x[c, t_in] * w[co, c, k] (x = 0 outside [0, T_in)),
 * then acc += bias[co]. f32 arithmetic in that order. */
ORC_API void orc_conv1d_f32io(const float* x, const uint16_t* w, const uint16_t* bias, float* out, int64_t B,
                              int64_t C_in, int64_t C_out, int64_t T_in, int64_t T_out, int64_t K, int64_t stride,
                              int64_t padding, int64_t dilation, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t co = 0; co < C_out; ++co) {
      const uint16_t* wr = w + co * C_in * K;
      float* orow = out + (b * C_out + co) * T_out;
      const float bv = bias ? f16_to_f32(bias[co]) : 0.0f;
      for (int64_t t = 0; t < T_out; ++t) {
        float acc = 0.0f;
        for (int64_t ck = 0; ck < C_in * K; ++ck) {
          const int64_t c = ck / K, k = ck % K;
          const int64_t ti = t * stride - padding + k * dilation;
          if (ti < 0 || ti >= T_in) continue;
          acc = acc + x[(b * C_in + c) * T_in + ti] * f16_to_f32(wr[ck]);
        }
        orow[t] = acc + bv;
      }
    }
}

/* ------------------------------------------------ decode attention ------- */

/* attention_decode_1d_masked (kernels/moonshine_kernels.py:1579-1625), one
 * query head at a time, f16 q / K / V widened exactly to f32:
 *   kv_head = q_head * n_kv_heads / n_q_heads;
 *   for each position j in order: s = (sum_d q[d] k_j[d]) * sm_scale (the sum
 *   over d in d order), m' = max(m, s), a = exp(m - m'), p = exp(s - m'),
 *   l = l a + p, acc = acc a + p v_j, m = m'  (m starts at -1e30, l = acc = 0);
 *   out = acc / l, here left in f32 (the kernel stores f16).
 * K/V element (h, j, d) at h * stride_kv_head + j * stride_kv_seq + d. */
ORC_API void orc_attention_decode_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, float* out,
                                      int64_t kv_len, int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads,
                                      float sm_scale, int64_t stride_kv_head, int64_t stride_kv_seq) {
  float* acc = (float*)malloc((size_t)head_dim * sizeof(float));
  for (int64_t qh = 0; qh < n_q_heads; ++qh) {
    const int64_t kvh = qh * n_kv_heads / n_q_heads;
    float m = -1e30f, l = 0.0f;
    for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0f;
    for (int64_t j = 0; j < kv_len; ++j) {
      const uint16_t* kr = k + kvh * stride_kv_head + j * stride_kv_seq;
      const uint16_t* vr = v + kvh * stride_kv_head + j * stride_kv_seq;
      float s = 0.0f;
      for (int64_t d = 0; d < head_dim; ++d) s += f16_to_f32(q[qh * head_dim + d]) * f16_to_f32(kr[d]);
      s = s * sm_scale;
      const float mn = s > m ? s : m;
      const float a = expf(m - mn), p = expf(s - mn);
      l = l * a + p;
      for (int64_t d = 0; d < head_dim; ++d) acc[d] = acc[d] * a + p * f16_to_f32(vr[d]);
      m = mn;
    }
    for (int64_t d = 0; d < head_dim; ++d) out[qh * head_dim + d] = acc[d] / l;
  }
  free(acc);
}

/* Kokoro generator tail, element-wise part. The reference's GPU chain after
 * the three resblocks of a stage (src/kokoro/decoder.rs:540-575; CPU
 * restatement :604-606) is elementwise_add_f32 twice
 * (kernels/kokoro_kernels.py:942-954), elementwise_scale_third_f32 (:958-969,
 * x * 0.3333333333333333 rounded to f32) and, after the last stage,
 * leaky_relu_f32 with slope 0.01 (the tl.where(x > 0, x, x * slope) form of
 * :109-122 and :600-605). Per element, with b / c / scale / lrelu optional:
 *   v = a; v = v + b; v = v + c; v = v * s; v = v > 0 ? v : v * slope. */
ORC_API void orc_combine_f32(const float* a, const float* b, const float* c, float* out, int64_t n, int scale,
                             float s, int lrelu, float slope) {
  for (int64_t i = 0; i < n; ++i) {
    float v = a[i];
    if (b) v = v + b[i];
    if (c) v = v + c[i];
    if (scale) v = v * s;
    if (lrelu) v = v > 0.0f ? v : v * slope;
    out[i] = v;
  }
}

/* Inverse STFT of conv_post's output, the reference's CPU istft
 * (src/kokoro/decoder.rs:1545-1632) fed as at :610-612 (magnitude =
 * exp(x[0 .. bins)), phase = sin(x[bins .. 2 bins))), batch 1:
 *   x [2 bins][n_frames] (bins = n_fft / 2 + 1);
 *   periodic Hann w[n] = 0.5 - 0.5 cos(2 pi n / n_fft) and the iDFT tables
 *   cos / sin(2 pi k n / n_fft), all from f32 angles (:1556-1571);
 *   frame[n] = (sum_k s_k (re_k cos_nk - im_k sin_nk)) / n_fft with
 *   re = m cos(p), im = m sin(p), s_k = 1 for k = 0 and bins - 1, else 2
 *   (:1585-1601); overlap-add of frame[n] * w[n] at f * hop + n, frames in
 *   order (:1604-1610); window_sum of w[n]^2 in frame order (:1576-1583);
 *   division where window_sum > 1e-8 (:1613-1618); trim n_fft / 2 at both
 *   ends (:1621-1628). out has (n_frames - 1) * hop samples. */
ORC_API void orc_istft_f32(const float* x, float* out, int64_t n_frames, int64_t n_fft, int64_t hop) {
  const int64_t bins = n_fft / 2 + 1, full = (n_frames - 1) * hop + n_fft, trim = n_fft / 2;
  const float PI = 3.14159265358979323846f;
  float* win = (float*)malloc((size_t)n_fft * sizeof(float));
  float* cb = (float*)malloc((size_t)(n_fft * bins) * sizeof(float));
  float* sb = (float*)malloc((size_t)(n_fft * bins) * sizeof(float));
  float* y = (float*)calloc((size_t)full, sizeof(float));
  float* ws = (float*)calloc((size_t)full, sizeof(float));
  float* fr = (float*)malloc((size_t)n_fft * sizeof(float));
  for (int64_t n = 0; n < n_fft; ++n) win[n] = 0.5f - 0.5f * cosf(2.0f * PI * (float)n / (float)n_fft);
  for (int64_t n = 0; n < n_fft; ++n)
    for (int64_t k = 0; k < bins; ++k) {
      const float ang = 2.0f * PI * (float)k * (float)n / (float)n_fft;
      cb[n * bins + k] = cosf(ang);
      sb[n * bins + k] = sinf(ang);
    }
  for (int64_t f = 0; f < n_frames; ++f)
    for (int64_t n = 0; n < n_fft; ++n) ws[f * hop + n] += win[n] * win[n];
  for (int64_t f = 0; f < n_frames; ++f) {
    for (int64_t n = 0; n < n_fft; ++n) {
      float v = 0.0f;
      for (int64_t k = 0; k < bins; ++k) {
        const float m = expf(x[k * n_frames + f]), p = sinf(x[(bins + k) * n_frames + f]);
        const float re = m * cosf(p), im = m * sinf(p);
        const float s = (k == 0 || k == bins - 1) ? 1.0f : 2.0f;
        v += s * (re * cb[n * bins + k] - im * sb[n * bins + k]);
      }
      fr[n] = v / (float)n_fft;
    }
    for (int64_t n = 0; n < n_fft; ++n) y[f * hop + n] += fr[n] * win[n];
  }
  for (int64_t i = 0; i < full; ++i)
    if (ws[i] > 1e-8f) y[i] /= ws[i];
  for (int64_t i = 0; i < full - 2 * trim; ++i) out[i] = y[i + trim];
  free(win);
  free(cb);
  free(sb);
  free(y);
  free(ws);
  free(fr);
}

/* Snake alone, snake_activation_tensor (src/kokoro/decoder.rs:1471-1476):
 * ax = x * alpha_c; out = x + sin(ax)^2 * (1 / (alpha_c + 1e-9)), f32 ops in
 * that order; x [rows][T], row r in channel r % C. */
ORC_API void orc_snake_f32(const float* x, const float* alpha, float* out, int64_t rows, int64_t C, int64_t T) {
  for (int64_t r = 0; r < rows; ++r) {
    const float a = alpha[r % C];
    const float inv_a = 1.0f / (a + 1e-9f);
    for (int64_t t = 0; t < T; ++t) {
      const float v = x[r * T + t];
      const float s = sinf(v * a);
      out[r * T + t] = v + (s * s) * inv_a;
    }
  }
}
