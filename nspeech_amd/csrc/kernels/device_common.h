/*
 * Device helpers shared by the gfx950 kernels: dtype conversion, 128-bit
 * vector access, wave64 DPP reductions, block reductions, activations and the
 * snake sin^2 evaluator. CDNA4 only (wave64).
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../nsr_kargs.h"

#define NSR_DEV __device__ __forceinline__

typedef float nsr_float4 __attribute__((ext_vector_type(4)));
typedef float nsr_float2 __attribute__((ext_vector_type(2)));
typedef __bf16 nsr_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t nsr_uint4 __attribute__((ext_vector_type(4)));
typedef uint32_t nsr_uint2 __attribute__((ext_vector_type(2)));

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
enum { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU = 2 };

/* ---------------------------------------------------------------- dtypes -- */

NSR_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

/* Two f32 -> packed bf16 (lo = a, hi = b), round to nearest even, NaN
 * quieted: one v_cvt_pk_bf16_f32. Same rounding as the `half` crate's
 * bf16::from_f32 used by Candle. */
NSR_DEV uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  const nsr_float2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, nsr_bf16x2));
}

NSR_DEV uint32_t f32_to_bf16_bits(float f) { return f32x2_to_bf16x2_bits(f, 0.0f) & 0xffffu; }

NSR_DEV float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

NSR_DEV uint32_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f; /* v_cvt_f16_f32, round to nearest even */
  return (uint32_t)__builtin_bit_cast(uint16_t, v);
}

template <int DT> NSR_DEV float load_scalar(const void* p, int64_t i) {
  if constexpr (DT == DT_F32) {
    return ((const float*)p)[i];
  } else if constexpr (DT == DT_F16) {
    return f16_bits_to_f32(((const uint16_t*)p)[i]);
  } else {
    return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  }
}

template <int DT> NSR_DEV void store_scalar(void* p, int64_t i, float v) {
  if constexpr (DT == DT_F32) {
    ((float*)p)[i] = v;
  } else if constexpr (DT == DT_F16) {
    ((uint16_t*)p)[i] = (uint16_t)f32_to_f16_bits(v);
  } else {
    ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
  }
}

template <int DT> struct dt_size { static constexpr int value = (DT == DT_F32) ? 4 : 2; };

/* Unpack a 16-byte chunk holding VEC = 16/size elements to floats. */
template <int DT> NSR_DEV void unpack16(const nsr_uint4 raw, float* v) {
  if constexpr (DT == DT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(raw[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t w = raw[i];
      if constexpr (DT == DT_BF16) {
        v[2 * i] = __uint_as_float(w << 16);
        v[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
      } else {
        v[2 * i] = f16_bits_to_f32(w & 0xffffu);
        v[2 * i + 1] = f16_bits_to_f32(w >> 16);
      }
    }
  }
}

/* Pack VEC floats into a 16-byte chunk of dtype DT (rounding as above). */
template <int DT> NSR_DEV nsr_uint4 pack16(const float* v) {
  nsr_uint4 r;
  if constexpr (DT == DT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __float_as_uint(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == DT_BF16) {
        r[i] = f32x2_to_bf16x2_bits(v[2 * i], v[2 * i + 1]);
      } else {
        r[i] = f32_to_f16_bits(v[2 * i]) | (f32_to_f16_bits(v[2 * i + 1]) << 16);
      }
    }
  }
  return r;
}

/* Round a float to dtype DT and back (value the tensor would hold). */
template <int DT> NSR_DEV float round_to(float v) {
  if constexpr (DT == DT_F32) {
    return v;
  } else if constexpr (DT == DT_BF16) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
  } else {
    return f16_bits_to_f32(f32_to_f16_bits(v));
  }
}

/* 128-bit global access. Data streamed through a kernel once is loaded and
 * stored non-temporally (it is not kept in L2 for reuse it will not get). */
NSR_DEV nsr_uint4 ld16(const void* p) { return __builtin_nontemporal_load((const nsr_uint4*)p); }
NSR_DEV void st16(void* p, nsr_uint4 v) { __builtin_nontemporal_store(v, (nsr_uint4*)p); }
NSR_DEV nsr_float4 ldf4(const float* p) { return __builtin_nontemporal_load((const nsr_float4*)p); }
NSR_DEV void stf4(float* p, nsr_float4 v) { __builtin_nontemporal_store(v, (nsr_float4*)p); }
/* cached 128-bit load, for small data many lanes re-read (gamma, beta) */
NSR_DEV nsr_uint4 ld16_cached(const void* p) { return *(const nsr_uint4*)p; }

/* ------------------------------------------------------- wave reductions -- */

/* DPP row/bank controls (GFX9 encoding). */
#define NSR_DPP_QUAD_1032 0xB1  /* quad_perm:[1,0,3,2] */
#define NSR_DPP_QUAD_2301 0x4E  /* quad_perm:[2,3,0,1] */
#define NSR_DPP_ROW_HALF_MIRROR 0x141
#define NSR_DPP_ROW_MIRROR 0x140
#define NSR_DPP_ROW_BCAST15 0x142
#define NSR_DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK>
NSR_DEV float dpp_add(float v) {
  /* lanes of rows outside ROW_MASK receive 0 (the `old` operand) */
  int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
  return v + __int_as_float(t);
}

/* Sum over the 64 lanes of the wave, returned uniformly to every lane.
 * Butterfly inside rows of 16 with quad_perm / mirror DPP, then row_bcast15 /
 * row_bcast31 carry the row sums into lane 63, which is broadcast. */
NSR_DEV float wave_sum(float v) {
  v = dpp_add<NSR_DPP_QUAD_1032, 0xF>(v);
  v = dpp_add<NSR_DPP_QUAD_2301, 0xF>(v);
  v = dpp_add<NSR_DPP_ROW_HALF_MIRROR, 0xF>(v);
  v = dpp_add<NSR_DPP_ROW_MIRROR, 0xF>(v);
  v = dpp_add<NSR_DPP_ROW_BCAST15, 0xA>(v);
  v = dpp_add<NSR_DPP_ROW_BCAST31, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* Sum over a workgroup of NWAVES waves; uniform result. `red` is LDS scratch
 * of NWAVES floats; the trailing barrier makes it reusable right away. */
template <int NWAVES>
NSR_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (NWAVES == 1) {
    return v;
  } else {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) s += red[w];
    __syncthreads();
    return s;
  }
}

/* Two sums over the workgroup at once (one LDS round trip); `red` holds
 * 2 * NWAVES floats. */
template <int NWAVES>
NSR_DEV void block_sum2(float& a, float& b, float* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  if constexpr (NWAVES > 1) {
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    if (lane == 0) {
      red[wid] = a;
      red[NWAVES + wid] = b;
    }
    __syncthreads();
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
      sa += red[w];
      sb += red[NWAVES + w];
    }
    __syncthreads();
    a = sa;
    b = sb;
  }
}

/* ------------------------------------------------------------ activations -- */

/* silu(v) = v / (1 + exp(-v)) (candle silu), as v * rcp(1 + 2^(-v log2 e))
 * with the hardware exp2 and reciprocal: branch-free, a few ulp. */
NSR_DEV float act_silu(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}

/* gelu_erf(v) = v * Phi(v), Phi(v) = 0.5 * (1 + erf(v / sqrt 2)) (candle
 * gelu_erf). Branch-free erfc from Abramowitz & Stegun, Handbook of
 * Mathematical Functions, formula 7.1.26: for z >= 0,
 *   erfc(z) = (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),
 *   t = 1 / (1 + p z),  |error| <= 1.5e-7,
 * with z = |v| / sqrt 2; Phi = 1 - erfc/2 for v >= 0 and erfc/2 below.
 * The coefficients below are the published a_k halved and p / sqrt 2. */
#define NSR_AS_P_SQRT2 0.23164189877f   /* 0.3275911 / sqrt(2) */
#define NSR_AS_HA1 0.127414796f         /* a1 / 2, a1 = 0.254829592 */
#define NSR_AS_HA2 -0.142248368f        /* a2 / 2, a2 = -0.284496736 */
#define NSR_AS_HA3 0.7107068705f        /* a3 / 2, a3 = 1.421413741 */
#define NSR_AS_HA4 -0.7265760135f       /* a4 / 2, a4 = -1.453152027 */
#define NSR_AS_HA5 0.5307027145f        /* a5 / 2, a5 = 1.061405429 */
NSR_DEV float act_gelu_erf(float v) {
  const float av = __builtin_fabsf(v);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(av, NSR_AS_P_SQRT2, 1.0f));
  float q = __builtin_fmaf(NSR_AS_HA5, t, NSR_AS_HA4);
  q = __builtin_fmaf(q, t, NSR_AS_HA3);
  q = __builtin_fmaf(q, t, NSR_AS_HA2);
  q = __builtin_fmaf(q, t, NSR_AS_HA1);
  /* exp(-v^2/2) = 2^(-v^2 log2(e) / 2) */
  const float e = __builtin_amdgcn_exp2f((av * -0.72134752044448170f) * av);
  const float h = (q * t) * e; /* erfc(|v|/sqrt 2) / 2 */
  const float phi = v >= 0.0f ? 1.0f - h : h;
  return v * phi;
}

template <int ACT> NSR_DEV float apply_act(float v) {
  if constexpr (ACT == ACT_SILU) {
    return act_silu(v);
  } else if constexpr (ACT == ACT_GELU) {
    return act_gelu_erf(v);
  } else {
    return v;
  }
}

/* ------------------------------------------------------------- snake sin^2 -- */

/* sin^2(t) = u * P(u), u = t^2, |t| <= pi/2. P fitted (weighted least squares
 * on Chebyshev nodes) to sin^2(sqrt(u))/u on [0, (pi/2)^2]; f32 Horner error
 * below 3e-7 relative. */
#define NSR_S2_C0 1.0f
#define NSR_S2_C1 -0.3333333432674408f
#define NSR_S2_C2 0.04444441944360733f
#define NSR_S2_C3 -0.0031745436135679483f
#define NSR_S2_C4 0.0001410240220138803f
#define NSR_S2_C5 -4.233750587445684e-06f
#define NSR_S2_C6 8.134502849088676e-08f

NSR_DEV float sin2_poly(float u) {
  float p = NSR_S2_C6;
  p = __builtin_fmaf(p, u, NSR_S2_C5);
  p = __builtin_fmaf(p, u, NSR_S2_C4);
  p = __builtin_fmaf(p, u, NSR_S2_C3);
  p = __builtin_fmaf(p, u, NSR_S2_C2);
  p = __builtin_fmaf(p, u, NSR_S2_C1);
  p = __builtin_fmaf(p, u, NSR_S2_C0);
  return p;
}

/* Per-row constants for snake(y) = y + sin^2(alpha*y) * inv_alpha evaluated
 * in y units: alpha*y = k*pi + alpha*r, k = rint(y*alpha/pi),
 * r = y - k*(pi/alpha) (two-term split), sin^2(alpha*y) = sin^2(alpha*r)
 * because sin^2 has period pi. */
struct snake_consts {
  float a_over_pi;   /* alpha / pi */
  float p_hi, p_lo;  /* pi / alpha = p_hi + p_lo (0, 0 when alpha == 0) */
  float a2;          /* alpha^2 */
  float k2;          /* alpha^2 * inv_alpha */
};

NSR_DEV snake_consts make_snake_consts(float alpha) {
  snake_consts s;
  const float inv_alpha = 1.0f / (alpha + 1e-9f); /* as decoder.rs:1474 */
  s.a_over_pi = (float)((double)alpha * 0.31830988618379067154);
  if (alpha != 0.0f) {
    const double pa = 3.14159265358979323846 / (double)alpha;
    s.p_hi = (float)pa;
    s.p_lo = (float)(pa - (double)s.p_hi);
  } else {
    s.p_hi = 0.f;
    s.p_lo = 0.f;
  }
  s.a2 = alpha * alpha;
  s.k2 = s.a2 * inv_alpha;
  return s;
}

NSR_DEV float snake_eval(float y, const snake_consts& s) {
  const float k = __builtin_rintf(y * s.a_over_pi);
  float r = __builtin_fmaf(-k, s.p_hi, y);
  r = __builtin_fmaf(-k, s.p_lo, r);
  const float v = r * r;
  const float p = sin2_poly(v * s.a2);
  return __builtin_fmaf(p, v * s.k2, y);
}
