/*
 * Partial interleaved rotary embedding over q [B,Hq,T,Dh] and k [B,Hk,T,Dh].
 *
 * Reference semantics: RotaryEmbedding::{new,forward} and
 * apply_rotary_pos_emb (src/moonshine/decoder.rs:85-183):
 *   inv_freq[i] = 1 / theta^(2i/rot)              (f32, glibc powf)
 *   angle       = f32(pos) * inv_freq[i]          (one f32 multiply)
 *   out         = x*cos + rotate_half_interleaved(x)*sin  on dims < rot,
 *                 rotate_half maps the pair (x0, x1) to (-x1, x0);
 *   dims >= rot pass through (Tensor::cat of q_pass).
 * The GPU RoPE table of src/moonshine/gpu_decoder.rs:326-340 holds, per
 * position, cos[0..half) then sin[0..half) of the same f32 angles.
 *
 * One lane per float4 (two rotation pairs or four pass-through values), a
 * flat grid over q then k: fully coalesced 128-bit loads and stores, 8 B of
 * HBM traffic per element. With a table the cos/sin values are the
 * reference's own f32 values and the products are kept unfused
 * (fp contract off), giving the reference's rounding sequence exactly.
 * Without a table cos/sin are evaluated in-kernel (accurate sincosf) from
 * the same f32 angle. Measured on MI355X at config 1, each against the
 * same box's copy of the same bytes: a 2-D grid (q / k in blockIdx.y, a
 * lane's row and column from shifts, the first row's position from one
 * scalar remainder per workgroup) reached 82% of the copy's rate (table
 * path) against 86% for this flat grid with two 32-bit divisions per lane,
 * so the flat grid is kept.
 *
 * At these sizes the time is the chain of memory latencies, so every load
 * is issued before the first wait: the frequencies (or the table's cos/sin)
 * and x together, and on the sincos path the frequencies first, so that the
 * sincos runs while x is in flight. Reading q / k's pointers by the lane's
 * choice (a.src[which]) compiled to a vector load from the argument block
 * that the data load waited on; the pointers are taken as uniform copies and
 * selected per lane instead. With the frequency load behind the data load's
 * wait, the sincos path took 3.70 us at config 1 against 3.27-3.28 us now.
 */
#include "device_common.h"

/* a kernel-argument value as a wave-uniform copy (an SGPR) */
NSR_DEV uint32_t rope_uni32(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
NSR_DEV uint64_t rope_uni64(uint64_t v) {
  return ((uint64_t)rope_uni32((uint32_t)(v >> 32)) << 32) | rope_uni32((uint32_t)v);
}
/* 128-bit streaming access at an integer address, as global memory (a pointer rebuilt from an integer is
 * generic and would give flat instructions) */
typedef __attribute__((address_space(1))) nsr_float4 rope_gf4;
NSR_DEV nsr_float4 rope_ld(uint64_t addr) { return __builtin_nontemporal_load((const rope_gf4*)addr); }
/* q is loaded cached and k streamed: measured on MI355X at config 1 against both streamed (same box, two runs
 * each, 200 / 20 calls): sincos path 3.15-3.16 / 3.30-3.35 against 3.28 / 3.42-3.43 us, table path
 * 3.14-3.23 / 3.22-3.23 against 3.24-3.25 / 3.35-3.38 us. Two streams with one cached, as the fused
 * LayerNorm's x and residual. */
NSR_DEV nsr_float4 rope_ldc(uint64_t addr) { return *(const rope_gf4*)addr; }
NSR_DEV void rope_st(uint64_t addr, nsr_float4 v) { __builtin_nontemporal_store(v, (rope_gf4*)addr); }

template <bool TABLE>
NSR_DEV void rope_body(const nsr_rope_args& a) {
#pragma clang fp contract(off)
  const uint32_t f = blockIdx.x * 256u + threadIdx.x;
  /* q or k per lane, chosen between uniform copies of the two arguments: indexed by the lane's choice
   * (a.src[which]) they would be read from the argument block by a vector load that the data load waits on */
  const uint32_t nq = rope_uni32((uint32_t)a.n4[0]), nk = rope_uni32((uint32_t)a.n4[1]);
  const bool isk = f >= nq;
  const uint32_t g = isk ? f - nq : f;
  if (g >= (isk ? nk : nq)) return;
  const uint64_t sq = rope_uni64((uint64_t)a.src[0]), sk = rope_uni64((uint64_t)a.src[1]);
  const uint64_t dq = rope_uni64((uint64_t)a.dst[0]), dk = rope_uni64((uint64_t)a.dst[1]);
  const uint64_t src = isk ? sk : sq, dst = isk ? dk : dq;

  const uint32_t dh4 = (uint32_t)a.dh4;
  const uint32_t row = g / dh4;
  const uint32_t c4 = g - row * dh4;
  const bool rot = c4 < (uint32_t)a.rot4;
  /* pair index of (x.x, x.y); i0 + 1 for (x.z, x.w). Pass-through lanes read pair 0's parameters and
   * discard them, so every load is issued before the first wait (one memory latency, not two) */
  const int i0 = rot ? 2 * (int)c4 : 0;
  const uint32_t t = row % (uint32_t)a.T;
  const int64_t pos = a.pos0 + (int64_t)t;
  float c0 = 1.f, s0 = 0.f, c1 = 1.f, s1 = 0.f;
  nsr_float4 x;
  if (a.rot4 > 0) { /* uniform; with no rotated pairs the table may hold no columns */
    if constexpr (TABLE) {
      const float* tb = a.table + pos * (int64_t)(2 * a.half);
      const float2 cc = *(const float2*)(tb + i0);
      const float2 ss = *(const float2*)(tb + a.half + i0);
      x = isk ? rope_ld(src + (uint64_t)g * 16u) : rope_ldc(src + (uint64_t)g * 16u);
      c0 = cc.x; c1 = cc.y; s0 = ss.x; s1 = ss.y;
    } else {
      /* the frequencies are loaded first: the sincos waits only for them, while x is in flight */
      const float2 fr = *(const float2*)(a.inv_freq + i0);
      __builtin_amdgcn_sched_barrier(0);
      x = isk ? rope_ld(src + (uint64_t)g * 16u) : rope_ldc(src + (uint64_t)g * 16u);
      __builtin_amdgcn_sched_barrier(0);
      const float p = (float)pos;
      sincosf(p * fr.x, &s0, &c0);
      sincosf(p * fr.y, &s1, &c1);
    }
  } else {
    x = isk ? rope_ld(src + (uint64_t)g * 16u) : rope_ldc(src + (uint64_t)g * 16u);
  }
  /* x*cos + rotate_half(x)*sin with the products rounded separately */
  nsr_float4 o;
  o.x = x.x * c0 + (-x.y) * s0;
  o.y = x.y * c0 + x.x * s0;
  o.z = x.z * c1 + (-x.w) * s1;
  o.w = x.w * c1 + x.z * s1;
  rope_st(dst + (uint64_t)g * 16u, rot ? o : x);
}

extern "C" __global__ void __launch_bounds__(256) nsrk_rope_table_f32(const nsr_rope_args a) {
  rope_body<true>(a);
}

extern "C" __global__ void __launch_bounds__(256) nsrk_rope_compute_f32(const nsr_rope_args a) {
  rope_body<false>(a);
}

/* ------------------------------------------------- decode step: RoPE + cache -- */

/*
 * One decode position: q [Hq, Dh] and k [Hk, Dh] rotated in place on the
 * interleaved pairs < rotary_dim with the RoPE table row pos, the rotated k
 * row and the v row appended to the caches [Hk, max_kv_len, Dh] at pos.
 * Reference: rope_qk_cache_fused (kernels/moonshine_kernels.py:1372-1454,
 * enc_rope_qk_cache_fused src/triton_kernels.rs:975) and kv_cache_append
 * (:865-883, enc_kv_cache_append :993), which the reference's decoder
 * dispatches back to back (src/moonshine/gpu_decoder_metal.rs:144-156); here
 * one launch. One lane per element pair, four disjoint lane ranges (q pairs,
 * k pairs, k pass-through pairs, v pairs): no lane reads what another writes.
 * Each rotated value is the storage dtype of x0*c - x1*s / x1*c + x0*s with
 * the f32 products rounded separately.
 */
template <int DT>
NSR_DEV void load_pair(const void* p, int64_t e, float& a, float& b) {
  if constexpr (DT == DT_F32) {
    const float2 v = *((const float2*)p + (e >> 1));
    a = v.x;
    b = v.y;
  } else {
    const uint32_t w = *((const uint32_t*)p + (e >> 1));
    a = f16_bits_to_f32(w & 0xffffu);
    b = f16_bits_to_f32(w >> 16);
  }
}

template <int DT>
NSR_DEV void store_pair(void* p, int64_t e, float a, float b) {
  if constexpr (DT == DT_F32) {
    *((float2*)p + (e >> 1)) = make_float2(a, b);
  } else {
    *((uint32_t*)p + (e >> 1)) = f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
  }
}

template <int DT>
NSR_DEV void copy_pair(const void* src, int64_t es, void* dst, int64_t ed) {
  if constexpr (DT == DT_F32) {
    *((float2*)dst + (ed >> 1)) = *((const float2*)src + (es >> 1));
  } else {
    *((uint32_t*)dst + (ed >> 1)) = *((const uint32_t*)src + (es >> 1));
  }
}

/* p / d for 0 <= p < 2^22 and d >= 1: a float reciprocal estimate (off by at most one) and one correction
 * each way, instead of an integer division ahead of the loads the quotient addresses. */
NSR_DEV int div_small(int p, int d) {
  int q = (int)((float)p * __builtin_amdgcn_rcpf((float)d));
  q += (q + 1) * d <= p ? 1 : 0;
  q -= q * d > p ? 1 : 0;
  return q;
}

template <int DT>
NSR_DEV void rope_cache_body(const nsr_rope_cache_args& a) {
#pragma clang fp contract(off)
  int p = (int)(blockIdx.x * 256u + threadIdx.x);
  const int Dh = a.Dh, half = a.half;
  const float* cs = a.table + a.pos * (int64_t)(2 * half);
  if (p < a.nq + a.nk) {
    const bool isk = p >= a.nq;
    if (isk) p -= a.nq;
    const int h = div_small(p, half), i = p - h * half;
    void* x = isk ? a.k : a.q;
    const int64_t e = (int64_t)h * Dh + 2 * i;
    float x0, x1;
    load_pair<DT>(x, e, x0, x1);
    const float c = cs[i], s = cs[half + i];
    const float y0 = round_to<DT>(x0 * c - x1 * s);
    const float y1 = round_to<DT>(x1 * c + x0 * s);
    store_pair<DT>(x, e, y0, y1);
    if (isk) store_pair<DT>(a.cache_k, ((int64_t)h * a.max_kv_len + a.pos) * Dh + 2 * i, y0, y1);
    return;
  }
  p -= a.nq + a.nk;
  if (p < a.nkp) {
    const int npp = (Dh - 2 * half) / 2;
    const int h = div_small(p, npp), j = 2 * half + 2 * (p - h * npp);
    copy_pair<DT>(a.k, (int64_t)h * Dh + j, a.cache_k, ((int64_t)h * a.max_kv_len + a.pos) * Dh + j);
    return;
  }
  p -= a.nkp;
  if (p < a.nv) {
    const int nh = Dh / 2;
    const int h = div_small(p, nh), j = 2 * (p - h * nh);
    copy_pair<DT>(a.v, (int64_t)h * Dh + j, a.cache_v, ((int64_t)h * a.max_kv_len + a.pos) * Dh + j);
  }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_rope_cache_f16(const nsr_rope_cache_args a) {
  rope_cache_body<DT_F16>(a);
}

extern "C" __global__ void __launch_bounds__(256) nsrk_rope_cache_f32(const nsr_rope_cache_args a) {
  rope_cache_body<DT_F32>(a);
}
