/*
 * Fused AdaIN1d + Snake over x [B, C, T] f32.
 *
 * Reference semantics (src/kokoro/decoder.rs:1416-1428, :1471-1476):
 *   mean = mean_T(x); var = mean_T((x - mean)^2)          (biased)
 *   norm = (x - mean) / sqrt(var + 1e-5)
 *   y    = norm * (gamma + 1) + beta
 *   out  = y + sin(alpha * y)^2 * recip(alpha + 1e-9)
 * gamma/beta come per (batch, channel) from the style Linear (precomputed and
 * rounded to f16 for the GPU backend, decoder.rs:966-981), alpha per channel.
 *
 * Resident kernel (one workgroup per (b, c) row): the row is read from HBM
 * once into VGPRs (NV float4 per lane) and, for long rows, LDS (filled with
 * global_load_lds_dwordx4, no VGPR staging); mean and centred variance are
 * two passes over on-chip data; the apply pass writes out once. HBM traffic
 * is the algorithmic 8 bytes per element. sin^2 uses a period-pi reduction in
 * y units and a fitted polynomial (device_common.h), about 16 VALU ops per
 * element in total.
 *
 * Split path (rows longer than the on-chip budget, or unaligned pointers):
 * a stats kernel (single read, shifted sums) then an apply kernel (second
 * read): 12 bytes per element.
 */
#include "device_common.h"

NSR_DEV float adain_param(const void* p, int pdt, int64_t i) {
  return pdt == DT_F32 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

typedef __attribute__((address_space(3))) void lds_void;

/* Element-wise access to a partial chunk (row edge when not ALIGNED):
 * element idx of chunk space belongs to the row iff lo <= idx < hi. */
NSR_DEV nsr_float4 load_chunk_masked(const float* xb, int j, int lo, int64_t hi) {
  nsr_float4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t idx = 4 * (int64_t)j + e;
    if (idx >= lo && idx < hi) r[e] = xb[idx];
  }
  return r;
}

NSR_DEV nsr_float4 mask_chunk(nsr_float4 d, int j, int lo, int64_t hi) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t idx = 4 * (int64_t)j + e;
    if (idx < lo || idx >= hi) d[e] = 0.f;
  }
  return d;
}

NSR_DEV void store_chunk_masked(float* ob, int j, int lo, int64_t hi, nsr_float4 o) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t idx = 4 * (int64_t)j + e;
    if (idx >= lo && idx < hi) ob[idx] = o[e];
  }
}

NSR_DEV nsr_float4 adain_snake4(nsr_float4 d, float A, float bet, const snake_consts& sc) {
  nsr_float4 o;
  o.x = snake_eval(__builtin_fmaf(d.x, A, bet), sc);
  o.y = snake_eval(__builtin_fmaf(d.y, A, bet), sc);
  o.z = snake_eval(__builtin_fmaf(d.z, A, bet), sc);
  o.w = snake_eval(__builtin_fmaf(d.w, A, bet), sc);
  return o;
}

NSR_DEV float sumsq4(nsr_float4 d, float sq) {
  sq = __builtin_fmaf(d.x, d.x, sq);
  sq = __builtin_fmaf(d.y, d.y, sq);
  sq = __builtin_fmaf(d.z, d.z, sq);
  return __builtin_fmaf(d.w, d.w, sq);
}

/* ALIGNED: x and out 16-byte aligned and T % 4 == 0, so every row is a whole
 * number of float4 chunks j = 0..nch-1, chunk j held by lane j % BLOCK.
 * Otherwise chunks lie on the float4 grid of the tensor: the row's first and
 * last chunk are partial and held by lane 0 (element access, e0/e1), the
 * interior chunks 1..nch-2 are full and spread as j = 1 + tid + BLOCK*k.
 * All loads of the chunk array are branch-free (index clamped in bounds,
 * out-of-row slots zeroed by a select), which keeps the array in VGPRs. */
template <int BLOCK, int NV, bool ALIGNED>
NSR_DEV void adain_resident(const nsr_adain_args& a, int pdt) {
  constexpr int NW = BLOCK / 64;
  extern __shared__ nsr_float4 lds_x[];
  __shared__ float red[2 * NW];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t T = a.T;
  const int64_t bi = row / a.C;
  const int64_t ci = row - bi * a.C;

  const float gam = adain_param(a.gamma, pdt, bi * a.gamma_bstride + ci);
  const float bet = adain_param(a.beta, pdt, bi * a.beta_bstride + ci);
  const float alp = adain_param(a.alpha, pdt, ci);

  const int64_t s = row * T;
  const int64_t a0 = ALIGNED ? s : (s & ~(int64_t)3);
  const int lo = (int)(s - a0);        /* first row element in chunk space */
  const int64_t hi = (int64_t)lo + T;  /* one past the last */
  const int nch = (int)((hi + 3) >> 2);
  const int jlast = nch - 1;
  const float* xb = a.x + a0;
  float* ob = a.out + a0;
  const nsr_float4 zero4 = {0.f, 0.f, 0.f, 0.f};

  /* chunk held in slot k of this lane, and the last valid chunk index */
  const int jbase = ALIGNED ? tid : 1 + tid;
  const int jmax = ALIGNED ? jlast : nch - 2;

  int nl = 0;
  if constexpr (ALIGNED) {
    /* LDS part first: chunks tid + BLOCK*(NV+m), straight from HBM into LDS
     * (lane i of a wave lands at wave base + 16*i). */
    nl = a.lds_chunks;
#pragma unroll 1
    for (int m = 0; m < nl; ++m) {
      const int j = min(tid + BLOCK * (NV + m), jlast);
      __builtin_amdgcn_global_load_lds((const void*)(xb + 4 * (int64_t)j),
                                       (lds_void*)(lds_x + m * BLOCK + (tid & ~63)), 16, 0, 0);
    }
  }

  nsr_float4 v[NV];
  if (jmax >= jbase - tid) { /* at least one full chunk in the array (uniform) */
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = jbase + BLOCK * k;
      const nsr_float4 t = ldf4(xb + 4 * (int64_t)min(j, jmax));
      v[k] = j <= jmax ? t : zero4;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = zero4;
  }
  nsr_float4 e0 = zero4, e1 = zero4; /* partial edge chunks (unaligned, lane 0) */
  if constexpr (!ALIGNED) {
    if (tid == 0) {
      e0 = load_chunk_masked(xb, 0, lo, hi);
      if (jlast > 0) e1 = load_chunk_masked(xb, jlast, lo, hi);
    }
  }

  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) sum += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  if constexpr (!ALIGNED) sum += ((e0.x + e0.y) + (e0.z + e0.w)) + ((e1.x + e1.y) + (e1.z + e1.w));
  if constexpr (ALIGNED) {
    if (nl > 0) {
      /* each lane reads back only the LDS slots its own wave filled */
      __builtin_amdgcn_s_waitcnt(0);
#pragma unroll 1
      for (int m = 0; m < nl; ++m) {
        const int j = tid + BLOCK * (NV + m);
        const nsr_float4 t = lds_x[m * BLOCK + tid];
        sum += j < nch ? (t.x + t.y) + (t.z + t.w) : 0.f;
      }
    }
  }
  const float mean = block_sum<NW>(sum, red) * a.inv_t;

  /* Centred pass: d = x - mean, with sum(d^2) and sum(d). The second sum
   * corrects the f32 mean (corrected two-pass algorithm), which keeps rows
   * whose |mean| >> std accurate; the correction c is folded into the bias. */
  float sq = 0.f, sd = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = jbase + BLOCK * k;
    const nsr_float4 d = v[k] - mean;
    v[k] = j <= jmax ? d : zero4;
    sq = sumsq4(v[k], sq);
    sd += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  }
  if constexpr (!ALIGNED) {
    if (tid == 0) {
      e0 = mask_chunk(e0 - mean, 0, lo, hi);
      e1 = jlast > 0 ? mask_chunk(e1 - mean, jlast, lo, hi) : zero4;
    }
    sq = sumsq4(e0, sumsq4(e1, sq));
    sd += ((e0.x + e0.y) + (e0.z + e0.w)) + ((e1.x + e1.y) + (e1.z + e1.w));
  }
  if constexpr (ALIGNED) {
#pragma unroll 1
    for (int m = 0; m < nl; ++m) {
      const int j = tid + BLOCK * (NV + m);
      nsr_float4 d = lds_x[m * BLOCK + tid] - mean;
      d = j < nch ? d : zero4;
      sq = sumsq4(d, sq);
      sd += (d.x + d.y) + (d.z + d.w);
    }
  }
  block_sum2<NW>(sq, sd, red);
  const float c = sd * a.inv_t;
  const float var = fmaxf(__builtin_fmaf(-c, sd, sq) * a.inv_t, 0.0f);
  const float rstd = 1.0f / sqrtf(var + a.eps);
  const float A = (gam + 1.0f) * rstd;
  const float Bc = __builtin_fmaf(-c, A, bet); /* (d - c) * A + beta = d * A + Bc */
  const snake_consts sc = make_snake_consts(alp);

#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = jbase + BLOCK * k;
    const nsr_float4 o = adain_snake4(v[k], A, Bc, sc);
    if (j <= jmax) stf4(ob + 4 * (int64_t)j, o);
  }
  if constexpr (!ALIGNED) {
    if (tid == 0) {
      store_chunk_masked(ob, 0, lo, hi, adain_snake4(e0, A, Bc, sc));
      if (jlast > 0) store_chunk_masked(ob, jlast, lo, hi, adain_snake4(e1, A, Bc, sc));
    }
  }
  if constexpr (ALIGNED) {
#pragma unroll 1
    for (int m = 0; m < nl; ++m) {
      const int j = tid + BLOCK * (NV + m);
      const nsr_float4 o = adain_snake4(lds_x[m * BLOCK + tid] - mean, A, Bc, sc);
      if (j < nch) stf4(ob + 4 * (int64_t)j, o);
    }
  }
}

#define NSR_ADAIN_RES(BLOCK, NV)                                                  \
  extern "C" __global__ void __launch_bounds__(BLOCK)                            \
      nsrk_adain_res_b##BLOCK##_nv##NV##_a(const nsr_adain_args a, const int pdt) { \
    adain_resident<BLOCK, NV, true>(a, pdt);                                     \
  }                                                                              \
  extern "C" __global__ void __launch_bounds__(BLOCK)                            \
      nsrk_adain_res_b##BLOCK##_nv##NV##_u(const nsr_adain_args a, const int pdt) { \
    adain_resident<BLOCK, NV, false>(a, pdt);                                    \
  }

NSR_ADAIN_RES(256, 1)
NSR_ADAIN_RES(256, 2)
NSR_ADAIN_RES(256, 3)
NSR_ADAIN_RES(256, 4)
NSR_ADAIN_RES(256, 5)
NSR_ADAIN_RES(256, 6)
NSR_ADAIN_RES(256, 8)
NSR_ADAIN_RES(1024, 3)
NSR_ADAIN_RES(1024, 4)
NSR_ADAIN_RES(1024, 6)
NSR_ADAIN_RES(1024, 8)
NSR_ADAIN_RES(1024, 12)
NSR_ADAIN_RES(1024, 16)
NSR_ADAIN_RES(1024, 20)

/* ------------------------------------------------------------ split path -- */

/* Stats: one 1024-thread workgroup per row, single read. Sums are taken about
 * a shift K (the mean of the row's first up-to-1024 elements), which keeps
 * S2 - S1^2/n free of cancellation when |mean| >> std. Writes (mean, rstd). */
extern "C" __global__ void __launch_bounds__(1024) nsrk_adain_stats(const nsr_adain_args a) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t T = a.T;
  const float* xr = a.x + row * T;
  const int64_t nk = T < 1024 ? T : 1024;
  const float k0 = block_sum<16>(tid < nk ? xr[tid] : 0.f, red) / (float)nk;
  float s1 = 0.f, s2 = 0.f;
  for (int64_t i = tid; i < T; i += 1024) {
    const float d = xr[i] - k0;
    s1 += d;
    s2 = __builtin_fmaf(d, d, s2);
  }
  s1 = block_sum<16>(s1, red);
  s2 = block_sum<16>(s2, red);
  if (tid == 0) {
    const double n = (double)T;
    const double m1 = (double)s1 / n;
    double var = (double)s2 / n - m1 * m1;
    if (var < 0.0) var = 0.0;
    a.stats[2 * row] = (float)((double)k0 + m1);
    a.stats[2 * row + 1] = 1.0f / sqrtf((float)var + a.eps);
  }
}

/* Apply: grid (n_rows, ceil(T / 1024)); scalar element access. */
extern "C" __global__ void __launch_bounds__(256) nsrk_adain_apply(const nsr_adain_args a, const int pdt) {
  const int64_t row = blockIdx.x;
  const int64_t T = a.T;
  const int64_t bi = row / a.C;
  const int64_t ci = row - bi * a.C;
  const float mean = a.stats[2 * row];
  const float rstd = a.stats[2 * row + 1];
  const float gam = adain_param(a.gamma, pdt, bi * a.gamma_bstride + ci);
  const float bet = adain_param(a.beta, pdt, bi * a.beta_bstride + ci);
  const float alp = adain_param(a.alpha, pdt, ci);
  const float A = (gam + 1.0f) * rstd;
  const snake_consts sc = make_snake_consts(alp);
  const float* xr = a.x + row * T;
  float* orow = a.out + row * T;
  const int64_t base = (int64_t)blockIdx.y * 1024;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t i = base + e * 256 + threadIdx.x;
    if (i < T) orow[i] = snake_eval(__builtin_fmaf(xr[i] - mean, A, bet), sc);
  }
}
