/*
 * Device helpers shared by the gfx950 kernels: dtype conversion, 128-bit
 * vector access, wave64 DPP reductions, block reductions, activations and the
 * snake sin^2 evaluator. CDNA4 only (wave64).
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../nsr_kargs.h"

#define NSR_DEV __device__ __forceinline__

/* No fusing of a separate multiply and add into one fma in the enclosing
 * block (the compiler may do so by default). Kernels whose numerics need
 * every use of a rounded value to see the same rounding say so with this;
 * explicit __builtin_fmaf calls still fuse. */
#define NSR_NO_CONTRACT _Pragma("clang fp contract(off)")

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
        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
        const h2_t h = {(_Float16)v[2 * i], (_Float16)v[2 * i + 1]}; /* one v_cvt_pk_f16_f32, nearest even */
        r[i] = __builtin_bit_cast(uint32_t, h);
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
 * of NWAVES floats; the trailing barrier makes it reusable right away.
 * REUSE = false drops that barrier, for callers whose next write to `red`
 * comes after another block reduction's first barrier (two reductions on
 * separate buffers, alternating): every wave has read `red` by then. */
template <int NWAVES, bool REUSE = true>
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
    if constexpr (REUSE) __syncthreads();
    return s;
  }
}

/* Two sums over the workgroup at once (one LDS round trip); `red` holds
 * 2 * NWAVES floats. REUSE as in block_sum. */
template <int NWAVES, bool REUSE = true>
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
    if constexpr (REUSE) __syncthreads();
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

/* gelu_erf(v) = v Phi(v) for finite v, Phi in the logistic form
 *   Phi(v) = 1 / (1 + exp(-g(v))),  g(v) = logit Phi(v) = v G(v^2)
 * (the form of Bowling, Khasawneh, Kaewkuekool and Cho, "A logistic approximation to the cumulative normal
 * distribution", J. Industrial Engineering and Management 2(1), 2009, there with G linear in v^2). Here G is a
 * degree-6 polynomial in w = v^2 fitted by Lawson's iteratively reweighted least squares (minimax) to the
 * absolute error of Phi on |v| <= 6, and -log2(e) is folded into its coefficients, so
 *   gelu(v) = v * rcp(1 + 2^(v P(w))),  P = -log2(e) G:
 * 10 VALU operations and two transcendentals (A&S 7.1.26 above: 11 and two). Error of Phi 2.9e-8 on the fit.
 * Evaluated in f32 (this sequence, emulated with exact products) against v Phi(v) in float64 on a grid of
 * 2e6 points over [-12, 12] plus |v| from 1e-30 to 3.3e38: error <= 1.9e-7 max(|v Phi(v)|, 1), relative error
 * <= 1e-4 where |v Phi(v)| > 1e-3, no NaN (A&S 7.1.26 above in f32: 2.2e-7 and 1.7e-4). G stays positive
 * beyond the fitted range (its leading coefficient is positive), so for large |v| 2^(v P) -> 0 as v -> +inf
 * (result v) and -> inf as v -> -inf (rcp -> 0, result -0); v = -inf itself would give inf * 0 = NaN, hence
 * finite v. */
NSR_DEV float act_gelu_logistic(float v) {
  const float w = v * v;
  float p = __builtin_fmaf(-5.0672373e-09f, w, 3.8163131e-07f);
  p = __builtin_fmaf(p, w, -1.14398345e-05f);
  p = __builtin_fmaf(p, w, 0.00015957994f);
  p = __builtin_fmaf(p, w, 9.40492173e-05f);
  p = __builtin_fmaf(p, w, -0.104835123f);
  p = __builtin_fmaf(p, w, -2.30220938f);
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * p));
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

/* apply_act for finite v (GELU in the logistic form). */
template <int ACT> NSR_DEV float apply_act_finite(float v) {
  if constexpr (ACT == ACT_SILU) {
    return act_silu(v);
  } else if constexpr (ACT == ACT_GELU) {
    return act_gelu_logistic(v);
  } else {
    return v;
  }
}

/* ------------------------------------------------------------------ snake -- */

/* snake(t) = t + sin^2(alpha t) * (1 / (alpha + 1e-9)), the reference's form
 * (src/kokoro/decoder.rs:1471-1476), evaluated as:
 *   q = t * alpha/pi,  f = q - rint(q)  (exact: |f| <= 1/2, Sterbenz),
 *   sin^2(alpha t) = sin^2(pi f) = w Q(w),  w = f^2 in [0, 1/4],
 * sin^2 having period pi. Q is a degree-6 polynomial fitted to
 * sin^2(pi sqrt(w)) / w on [0, 1/4] by Lawson's iteratively reweighted least
 * squares (minimax) on Chebyshev nodes: relative error 5.4e-8 with the f32
 * coefficients below. The per-row factor 1/(alpha + 1e-9) is folded into the
 * coefficients, so one element costs 11 VALU operations:
 *   mul, rndne, sub, mul, 6 fma (Horner), fma (t + p*w).
 * Worst error over t in [-200, 200], alpha in {0, 1e-9, 1e-4, 0.5 .. 10, -0.7}:
 * 3.9e-7 of max(|out|, 1) in f32. */
#define NSR_SNAKE_Q0 9.869604110717773f
#define NSR_SNAKE_Q1 -32.469696044921875f
#define NSR_SNAKE_Q2 42.72837829589844f
#define NSR_SNAKE_Q3 -30.121654510498047f
#define NSR_SNAKE_Q4 13.205862045288086f
#define NSR_SNAKE_Q5 -3.910468578338623f
#define NSR_SNAKE_Q6 0.7385572195053101f

struct snake_consts {
  float a_pi; /* alpha / pi */
  float c[7]; /* Q coefficients times 1 / (alpha + 1e-9) */
};

NSR_DEV snake_consts make_snake_consts(float alpha) {
  snake_consts s;
  const float inv_a = 1.0f / (alpha + 1e-9f); /* recip(alpha + 1e-9), decoder.rs:1474 */
  s.a_pi = (float)((double)alpha * 0.31830988618379067154);
  s.c[0] = NSR_SNAKE_Q0 * inv_a;
  s.c[1] = NSR_SNAKE_Q1 * inv_a;
  s.c[2] = NSR_SNAKE_Q2 * inv_a;
  s.c[3] = NSR_SNAKE_Q3 * inv_a;
  s.c[4] = NSR_SNAKE_Q4 * inv_a;
  s.c[5] = NSR_SNAKE_Q5 * inv_a;
  s.c[6] = NSR_SNAKE_Q6 * inv_a;
  return s;
}

NSR_DEV float snake_eval(float t, const snake_consts& s) {
  const float q = t * s.a_pi;
  const float f = q - __builtin_rintf(q);
  const float w = f * f;
  float p = __builtin_fmaf(s.c[6], w, s.c[5]);
  p = __builtin_fmaf(p, w, s.c[4]);
  p = __builtin_fmaf(p, w, s.c[3]);
  p = __builtin_fmaf(p, w, s.c[2]);
  p = __builtin_fmaf(p, w, s.c[1]);
  p = __builtin_fmaf(p, w, s.c[0]);
  return __builtin_fmaf(p, w, t);
}

/* snake for kernels whose output is f16: Q of degree 4 (fitted the same way, relative error 1.0e-6), so one
 * element costs 9 VALU operations. Worst error over t in [-200, 200], alpha in {1e-9, 1e-4, 0.5 .. 10, -0.7}:
 * 2.2e-6 of max(|out|, 1) in f32, against an f16 rounding of up to 4.9e-4 of the value. */
#define NSR_SNAKE_H_Q0 9.86959457397461f
#define NSR_SNAKE_H_Q1 -32.46799087524414f
#define NSR_SNAKE_H_Q2 42.67864990234375f
#define NSR_SNAKE_H_Q3 -29.59571647644043f
#define NSR_SNAKE_H_Q4 10.860782623291016f

struct snake_consts_h {
  float a_pi;
  float c[5];
};

NSR_DEV snake_consts_h make_snake_consts_h(float alpha) {
  snake_consts_h s;
  const float inv_a = 1.0f / (alpha + 1e-9f);
  s.a_pi = (float)((double)alpha * 0.31830988618379067154);
  s.c[0] = NSR_SNAKE_H_Q0 * inv_a;
  s.c[1] = NSR_SNAKE_H_Q1 * inv_a;
  s.c[2] = NSR_SNAKE_H_Q2 * inv_a;
  s.c[3] = NSR_SNAKE_H_Q3 * inv_a;
  s.c[4] = NSR_SNAKE_H_Q4 * inv_a;
  return s;
}

NSR_DEV float snake_eval(float t, const snake_consts_h& s) {
  const float q = t * s.a_pi;
  const float f = q - __builtin_rintf(q);
  const float w = f * f;
  float p = __builtin_fmaf(s.c[4], w, s.c[3]);
  p = __builtin_fmaf(p, w, s.c[2]);
  p = __builtin_fmaf(p, w, s.c[1]);
  p = __builtin_fmaf(p, w, s.c[0]);
  return __builtin_fmaf(p, w, t);
}

/* ------------------------------------------------------ XCD tile order -- */

/* Workgroups are dealt round-robin to the 8 XCDs (workgroup b runs on XCD
 * b % 8). xcd_contiguous(b, n) gives workgroup b the tile that makes each
 * XCD take one contiguous run of the n tiles (XCD x the x-th run), so that
 * neighbouring tiles, which share cache lines at their edges, meet in one
 * XCD's L2. A bijection of [0, n) for a grid of n workgroups. */
NSR_DEV int xcd_contiguous(int b, int n) {
  const int per = (n + 7) >> 3, x = b & 7, i = b >> 3;
  const int full = n - 8 * (per - 1); /* XCDs that take `per` tiles */
  return (x < full ? x * per : full * per + (x - full) * (per - 1)) + i;
}

/* ------------------------------------------------------- buffer access -- */

/* Raw buffer resource over [base, base + bytes): loads past the end return
 * 0 and stores past the end are dropped by the hardware range check. */
typedef __amdgpu_buffer_rsrc_t nsr_rsrc;
#define NSR_RSRC_WORD3 0x00020000 /* gfx9 data format 32, raw (stride 0) */
#define NSR_AUX_NT 2              /* non-temporal (streamed) access */

NSR_DEV nsr_rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)bytes, NSR_RSRC_WORD3);
}

/* make_rsrc for a base and size that are wave-uniform but that the
 * compiler cannot prove so: readfirstlane keeps the descriptor in SGPRs
 * instead of wrapping every load that uses it in a readfirstlane loop. */
NSR_DEV nsr_rsrc make_rsrc_uniform(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return make_rsrc((const void*)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}

/* 16-byte load at voff + soff (soff wave-uniform, kept in an SGPR). */
NSR_DEV nsr_float4 buf_load4(nsr_rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, NSR_AUX_NT));
}

/* buf_load4 without the non-temporal bit (the line is cached as a normal load's) */
NSR_DEV nsr_float4 buf_load4c(nsr_rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

/* 16-byte store at voff + off with soffset 0. Stores carry their offset in
 * the VGPR address, never in soffset: the compiler exempts MUBUF stores with
 * an SGPR soffset from the wait state that a VALU write of the store's data
 * registers needs right after a >64-bit store, and on gfx950 such stores were
 * observed to write the overwritten values. */
NSR_DEV void buf_store4(nsr_rsrc r, uint32_t voff, uint32_t off, nsr_float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(nsr_uint4, v), r, voff + off, 0, NSR_AUX_NT);
}

/* s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt[3:0], vmcnt[5:4] at bit 14,
 * expcnt and lgkmcnt left at their maxima). */
#define NSR_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n)&15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8)))

/* Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E). */
template <int B, int E, typename F>
NSR_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}
