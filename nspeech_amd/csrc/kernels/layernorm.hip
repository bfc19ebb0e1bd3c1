/*
 * LayerNorm family and fused residual-add + LayerNorm (+ activation).
 *
 * Reference semantics:
 *   candle_nn::LayerNorm (eps 1e-5, affine) as used by the Parakeet conformer
 *     (src/parakeet/fast_conformer.rs:721-725,778-782,793-811);
 *   UnitOffsetLayerNorm::forward src/moonshine/encoder.rs:68-76 (scale gamma+1);
 *   LayerNorm::forward src/moonshine/decoder.rs:67-74 (weight only);
 *   residual_add_layernorm_fused kernels/moonshine_kernels.py:955-991
 *     (h = proj + residual written out, LN(h) * w written out);
 *   the CPU chain fast_add (src/fast_ops.rs:16-36) -> LayerNorm -> gelu_erf.
 *
 * Design (gfx950): one wave64 per row, the row held in VGPRs as NC chunks of
 * 16 bytes per lane (128-bit coalesced loads), statistics in two passes over
 * the registers (mean, then centred sum of squares) with DPP wave reductions,
 * so x (and res) are read from HBM exactly once and y (and h) written once.
 * Four waves per 256-thread workgroup, no LDS and no block barriers; the grid
 * is capped and each wave walks rows with the grid's wave count as stride,
 * loading its next row while it reduces the current one.
 * Rows that are not 16-byte aligned or longer than 4096 columns take the
 * generic kernel at the bottom (one workgroup per row, scalar access).
 */
#include "device_common.h"

/* Chunk = VEC elements; 16 bytes of the narrowest tensor involved. */
template <int X, int R, int H, int Y>
struct ln_vec {
  static constexpr bool all32 = (X == DT_F32) && (R == DT_F32) && (H == DT_F32) && (Y == DT_F32);
  static constexpr int value = all32 ? 4 : 8;
};

/* VEC elements of dtype DT at base[elem]; NT: streamed (non-temporal) load,
 * otherwise a cached load (parameters every row re-reads). */
template <int DT, int VEC, bool NT = true>
NSR_DEV void load_vec(const void* base, int64_t elem, float* v) {
  constexpr int BYTES = VEC * dt_size<DT>::value;
  const char* p = (const char*)base + elem * dt_size<DT>::value;
  if constexpr (BYTES == 16) {
    unpack16<DT>(NT ? ld16(p) : ld16_cached(p), v);
  } else if constexpr (BYTES == 32) {
    unpack16<DT>(NT ? ld16(p) : ld16_cached(p), v);
    unpack16<DT>(NT ? ld16(p + 16) : ld16_cached(p + 16), v + 16 / dt_size<DT>::value);
  } else { /* 8 bytes: 4 x 16-bit */
    const nsr_uint2 r = *(const nsr_uint2*)p;
    nsr_uint4 r4 = {r[0], r[1], 0u, 0u};
    float t[8];
    unpack16<DT>(r4, t);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = t[i];
  }
}

template <int DT, int VEC>
NSR_DEV void store_vec(void* base, int64_t elem, const float* v) {
  constexpr int BYTES = VEC * dt_size<DT>::value;
  char* p = (char*)base + elem * dt_size<DT>::value;
  if constexpr (BYTES == 16) {
    st16(p, pack16<DT>(v));
  } else if constexpr (BYTES == 32) {
    st16(p, pack16<DT>(v));
    st16(p + 16, pack16<DT>(v + 16 / dt_size<DT>::value));
  } else {
    float t[8] = {v[0], v[1], v[2], v[3], 0.f, 0.f, 0.f, 0.f};
    const nsr_uint4 r4 = pack16<DT>(t);
    *(nsr_uint2*)p = nsr_uint2{r4[0], r4[1]};
  }
}

NSR_DEV float load_param(const void* p, int pdt, int64_t i) {
  return pdt == DT_F32 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

/* VEC gamma/beta values (f32 or f16, uniform branch); `fill` when p is NULL. */
template <int VEC>
NSR_DEV void load_param_vec(const void* p, int pdt, int col0, float* v, float fill) {
  if (!p) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = fill;
  } else if (pdt == DT_F32) {
    load_vec<DT_F32, VEC, false>(p, col0, v);
  } else {
    load_vec<DT_F16, VEC, false>(p, col0, v);
  }
}

/* Raw 16-byte words of one VEC-element chunk of dtype DT (1 or 2 words). */
template <int DT, int VEC> struct chunk_words { static constexpr int value = VEC * dt_size<DT>::value / 16; };

template <int DT, int VEC, bool CACHED = false>
NSR_DEV void load_raw(const void* base, int64_t elem, nsr_uint4* w) {
  const char* p = (const char*)base + elem * dt_size<DT>::value;
#pragma unroll
  for (int i = 0; i < chunk_words<DT, VEC>::value; ++i) w[i] = CACHED ? ld16_cached(p + 16 * i) : ld16(p + 16 * i);
}

template <int DT, int VEC>
NSR_DEV void unpack_raw(const nsr_uint4* w, float* v) {
#pragma unroll
  for (int i = 0; i < chunk_words<DT, VEC>::value; ++i) unpack16<DT>(w[i], v + i * (16 / dt_size<DT>::value));
}

/*
 * One wave64 per row, rows visited persistently: wave w of the grid takes
 * rows w, w + W, w + 2W, ... (W = waves in the grid), so gamma/beta are
 * loaded once per wave, and the next row's x (and res) chunks are loaded
 * while the current row is reduced and written. FUSED = false: h = x.
 * FUSED = true: h = round_H(x + res), stored (if a.h) as soon as it is
 * formed. PDT runtime, ACT compile time.
 */
template <int X, int R, int H, int Y, int NC, bool FUSED, int ACT, bool FULL = false>
NSR_DEV void ln_row_wave(const nsr_ln_args& a, int pdt) {
  constexpr int VEC = ln_vec<X, R, H, Y>::value;
  constexpr int XW = chunk_words<X, VEC>::value;
  constexpr int RW = FUSED ? chunk_words<R, VEC>::value : 1;
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.n_rows) return; /* whole wave leaves; no barriers below */
  /* FULL: n_cols == 64 * NC * VEC, every chunk guard below is true */
  const int nchunk = FULL ? 64 * NC : a.n_cols / VEC;

  /* gamma/beta do not depend on the row: when they fit in 64 more VGPRs
   * they are loaded once per wave, before the first row's loads */
  constexpr bool PREFETCH = NC * VEC <= 32;
  const float goff = a.unit_offset ? 1.0f : 0.0f; /* gamma + 1 (unit offset), added once per loaded gamma */
  float gpre[PREFETCH ? NC : 1][VEC], bpre[PREFETCH ? NC : 1][VEC];
  if constexpr (PREFETCH) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int j = lane + 64 * k;
      if (j < nchunk) {
        load_param_vec<VEC>(a.gamma, pdt, j * VEC, gpre[k], 1.0f);
        load_param_vec<VEC>(a.beta, pdt, j * VEC, bpre[k], 0.0f);
#pragma unroll
        for (int e = 0; e < VEC; ++e) gpre[k][e] += goff;
      }
    }
  }

  /* raw chunks of the row being worked on; refilled with the next row's
   * chunks while this one is reduced, when they fit in 32 VGPRs */
  constexpr bool PIPE = NC * (XW + (FUSED ? RW : 0)) * 4 <= 32;
  nsr_uint4 rx[NC][XW], rr[NC][RW];
  auto load_row = [&](int64_t r) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int j = lane + 64 * k;
      if (j < nchunk) {
        /* fused: x loaded cached and the residual streamed. Measured on MI355X at c4a ([24000, 1024] bf16,
         * GELU, 200 calls back to back, minimum / median of 5): 30.9-31.1 / 31.1-31.2 us against 33.3-33.4 /
         * 33.5 us with both streamed; the residual cached instead 31.2-31.3 us, both cached 32.8-32.9 us.
         * The same output bits. */
        load_raw<X, VEC, FUSED>(a.x, r * a.ld_x + (int64_t)j * VEC, rx[k]);
        if constexpr (FUSED) load_raw<R, VEC>(a.res, r * a.ld_x + (int64_t)j * VEC, rr[k]);
      }
    }
  };
  load_row(row);

  while (true) {
    const int64_t xrow = row * a.ld_x;
    const int64_t yrow = row * a.ld_y;
    const int64_t next = row + stride;
    const bool more = next < a.n_rows;

    float v[NC][VEC];
    float sum = 0.f, sum2 = 0.f;
    /* packed h words, stored once the next row's loads are issued */
    constexpr bool PACKED_H = FUSED && H != DT_F32 && chunk_words<H, VEC>::value == 1;
    /* bf16 h: sum and sum of squares straight from the packed words with v_dot2c_f32_bf16 (two products,
     * each exact in f32, added to the f32 accumulator): one instruction per pair for each sum instead of a
     * widening, an add and a centred fma per element, and the widening moves after the reductions */
    constexpr bool DOT_STATS = PACKED_H && H == DT_BF16;
    nsr_uint4 hsave[PACKED_H ? NC : 1];
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int j = lane + 64 * k;
      if (j < nchunk) {
        unpack_raw<X, VEC>(rx[k], v[k]);
        if constexpr (FUSED) {
          float r[VEC];
          unpack_raw<R, VEC>(rr[k], r);
          if constexpr (PACKED_H) {
            /* h = round_H(x + res) packed two at a time (one conversion per pair), stored as packed and
             * widened back from the packed words: the same values as rounding each element */
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[k][e] += r[e];
            hsave[k] = pack16<H>(v[k]);
            if constexpr (!DOT_STATS) unpack16<H>(hsave[k], v[k]);
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[k][e] = round_to<H>(v[k][e] + r[e]);
            if (a.h) store_vec<H, VEC>(a.h, xrow + (int64_t)j * VEC, v[k]);
          }
        }
        if constexpr (DOT_STATS) {
          const nsr_bf16x2 one = __builtin_bit_cast(nsr_bf16x2, 0x3f803f80u);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            /* a named copy: a bit_cast of the vector element itself reads element 0 with this compiler */
            const uint32_t w = hsave[k][i];
            const nsr_bf16x2 hw = __builtin_bit_cast(nsr_bf16x2, w);
            sum = __builtin_amdgcn_fdot2_f32_bf16(hw, one, sum, false);
            sum2 = __builtin_amdgcn_fdot2_f32_bf16(hw, hw, sum2, false);
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) sum += v[k][e];
        }
      }
    }
    if constexpr (PIPE) {
      if (more) load_row(next);
    }
    /* h after the next row's loads: measured on MI355X at [24000, 1024] bf16, 33.7 against 33.9-35.4 us over
     * 200 calls when each h chunk is stored as soon as it is formed */
    if constexpr (PACKED_H) {
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        const int j = lane + 64 * k;
        if (j < nchunk && a.h) st16((char*)a.h + (xrow + (int64_t)j * VEC) * dt_size<H>::value, hsave[k]);
      }
    }
    const float mean = wave_sum(sum) * a.inv_n;
    float var, shift; /* v[k][e] * rstd + shift * rstd = (h - mean) * rstd */
    if constexpr (DOT_STATS) {
      /* one pass, var = E[h^2] - mean^2: its rounding error relative to var is about (1 + mean^2 / var)
       * f32 ulps of the sums, so when mean^2 > var (a wave-uniform test) the row takes the centred two-pass
       * form over the registers instead */
      var = __builtin_fmaf(-mean, mean, wave_sum(sum2) * a.inv_n);
      shift = -mean;
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        const int j = lane + 64 * k;
        if (j < nchunk) unpack16<H>(hsave[k], v[k]);
      }
      if (mean * mean > var) {
        float sq = 0.f;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          const int j = lane + 64 * k;
          if (j < nchunk) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              v[k][e] -= mean;
              sq = __builtin_fmaf(v[k][e], v[k][e], sq);
            }
          }
        }
        var = wave_sum(sq) * a.inv_n;
        shift = 0.0f;
      }
      var = fmaxf(var, 0.0f);
    } else {
      /* centred pass; sum(d) corrects the f32 mean (corrected two-pass), which
       * keeps rows with |mean| >> std accurate. The correction changes the
       * variance by (mean rounding error)^2 / var, below f32 resolution unless
       * |mean| / std > 1e4: values held in f16 / bf16 (h, or x for a plain
       * LayerNorm) cannot have that spread, so those rows skip it. */
      constexpr bool CORR = H == DT_F32;
      float sq = 0.f, sd = 0.f;
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        const int j = lane + 64 * k;
        if (j < nchunk) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            v[k][e] -= mean;
            sq = __builtin_fmaf(v[k][e], v[k][e], sq);
            if constexpr (CORR) sd += v[k][e];
          }
        }
      }
      sq = wave_sum(sq);
      if constexpr (CORR) sd = wave_sum(sd);
      const float c = sd * a.inv_n;
      var = fmaxf(__builtin_fmaf(-c, sd, sq) * a.inv_n, 0.0f);
      shift = -c; /* (d - c) * rstd */
    }
    /* v_rsq_f32 (about 1 ulp) instead of a correctly rounded sqrt and divide, about 30 instructions per
     * row; var + eps > 0 is a normal number unless eps = 0 and the row is constant (then inf either way) */
    const float rstd = __builtin_amdgcn_rsqf(var + a.eps);
    const float crs = shift * rstd;

#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int j = lane + 64 * k;
      if (j < nchunk) {
        const int col0 = j * VEC;
        float g[VEC], b[VEC], o[VEC];
        if constexpr (PREFETCH) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            g[e] = gpre[k][e];
            b[e] = bpre[k][e];
          }
        } else {
          load_param_vec<VEC>(a.gamma, pdt, col0, g, 1.0f);
          load_param_vec<VEC>(a.beta, pdt, col0, b, 0.0f);
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] += goff;
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          /* a LayerNorm output is finite (finite parameters), so the activation's finite-input form applies */
          o[e] = apply_act_finite<ACT>(__builtin_fmaf(__builtin_fmaf(v[k][e], rstd, crs), g[e], b[e]));
        }
        store_vec<Y, VEC>(a.y, yrow + col0, o);
      }
    }
    if (!more) break;
    row = next;
    if constexpr (!PIPE) load_row(row);
  }
}

/* Kernel: PDT, ACT and FULL switch uniformly outside the row body. FULL
 * (n_cols == 64 * NC * VEC) drops the per-chunk column guards. */
template <int X, int R, int H, int Y, int NC, bool FUSED, bool FULL>
NSR_DEV void ln_wave_act(const nsr_ln_args& a, int pdt, int act) {
  if (act == ACT_GELU) {
    ln_row_wave<X, R, H, Y, NC, FUSED, ACT_GELU, FULL>(a, pdt);
  } else if (act == ACT_SILU) {
    ln_row_wave<X, R, H, Y, NC, FUSED, ACT_SILU, FULL>(a, pdt);
  } else {
    ln_row_wave<X, R, H, Y, NC, FUSED, ACT_NONE, FULL>(a, pdt);
  }
}

template <int X, int R, int H, int Y, int NC, bool FUSED>
NSR_DEV void ln_wave_entry(const nsr_ln_args& a, int pdt, int act, int full) {
  if (full) {
    ln_wave_act<X, R, H, Y, NC, FUSED, true>(a, pdt, act);
  } else {
    ln_wave_act<X, R, H, Y, NC, FUSED, false>(a, pdt, act);
  }
}

/* ---------------------------------------------------------------- generic -- */

/* One 256-thread workgroup per row, scalar loads, three passes over the row
 * (global memory): any n_cols, any alignment. The fused variant writes h in
 * the first pass and the later passes read h back from memory (or recompute
 * it when h is not stored). */
template <int X, int R, int H, int Y, bool FUSED>
NSR_DEV void ln_row_generic(const nsr_ln_args& a, int pdt, int act) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  if (row >= a.n_rows) return;
  const int n = a.n_cols;
  const int64_t xrow = row * a.ld_x;
  const int64_t yrow = row * a.ld_y;

  auto hval = [&](int c) -> float {
    float v = load_scalar<X>(a.x, xrow + c);
    if constexpr (FUSED) v = round_to<H>(v + load_scalar<R>(a.res, xrow + c));
    return v;
  };

  float s = 0.f;
  for (int c = threadIdx.x; c < n; c += 256) {
    const float v = hval(c);
    if constexpr (FUSED) {
      if (a.h) store_scalar<H>(a.h, xrow + c, v);
    }
    s += v;
  }
  const float mean = block_sum<4>(s, red) * a.inv_n;
  float q = 0.f, sd = 0.f;
  for (int c = threadIdx.x; c < n; c += 256) {
    const float d = hval(c) - mean;
    q = __builtin_fmaf(d, d, q);
    sd += d;
  }
  block_sum2<4>(q, sd, red);
  const float corr = sd * a.inv_n;
  const float var = fmaxf(__builtin_fmaf(-corr, sd, q) * a.inv_n, 0.0f);
  const float rstd = 1.0f / sqrtf(var + a.eps);
  for (int c = threadIdx.x; c < n; c += 256) {
    const float d = hval(c) - mean - corr;
    float g = a.gamma ? load_param(a.gamma, pdt, c) : 1.0f;
    if (a.unit_offset) g += 1.0f;
    const float b = a.beta ? load_param(a.beta, pdt, c) : 0.0f;
    float o = __builtin_fmaf(d * rstd, g, b);
    if (act == ACT_GELU) o = act_gelu_logistic(o); /* finite: a LayerNorm output */
    else if (act == ACT_SILU) o = act_silu(o);
    store_scalar<Y>(a.y, yrow + c, o);
  }
}

/* ------------------------------------------------------------ instances -- */
/* Kernel argument tail: pdt, act and full packed into one int
 * (pdt | act << 8 | full << 16). */

#define NSR_LN_WAVE(NAME, X, R, H, Y, NC, FUSED)                                \
  extern "C" __global__ void __launch_bounds__(256)                            \
      NAME(const nsr_ln_args a, const int mode) {                              \
    ln_wave_entry<X, R, H, Y, NC, FUSED>(a, mode & 0xff, (mode >> 8) & 0xff,    \
                                         mode >> 16);                          \
  }

#define NSR_LN_GENERIC(NAME, X, R, H, Y, FUSED)                                 \
  extern "C" __global__ void __launch_bounds__(256)                            \
      NAME(const nsr_ln_args a, const int mode) {                              \
    ln_row_generic<X, R, H, Y, FUSED>(a, mode & 0xff, (mode >> 8) & 0xff);      \
  }

/* Plain LayerNorm: x dtype -> y dtype, NC chunks per lane. */
#define NSR_LN_PLAIN_SET(XN, X, YN, Y)                                          \
  NSR_LN_WAVE(nsrk_ln_##XN##_##YN##_nc1, X, X, X, Y, 1, false)                   \
  NSR_LN_WAVE(nsrk_ln_##XN##_##YN##_nc2, X, X, X, Y, 2, false)                   \
  NSR_LN_WAVE(nsrk_ln_##XN##_##YN##_nc4, X, X, X, Y, 4, false)                   \
  NSR_LN_WAVE(nsrk_ln_##XN##_##YN##_nc8, X, X, X, Y, 8, false)                   \
  NSR_LN_GENERIC(nsrk_ln_##XN##_##YN##_generic, X, X, X, Y, false)

NSR_LN_PLAIN_SET(f32, DT_F32, f32, DT_F32)
NSR_LN_PLAIN_SET(f32, DT_F32, f16, DT_F16)
NSR_LN_PLAIN_SET(f32, DT_F32, bf16, DT_BF16)
NSR_LN_PLAIN_SET(f16, DT_F16, f32, DT_F32)
NSR_LN_PLAIN_SET(f16, DT_F16, f16, DT_F16)
NSR_LN_PLAIN_SET(f16, DT_F16, bf16, DT_BF16)
NSR_LN_PLAIN_SET(bf16, DT_BF16, f32, DT_F32)
NSR_LN_PLAIN_SET(bf16, DT_BF16, f16, DT_F16)
NSR_LN_PLAIN_SET(bf16, DT_BF16, bf16, DT_BF16)
/* f32 rows up to 4096 columns need 16 chunks of 4 per lane */
NSR_LN_WAVE(nsrk_ln_f32_f32_nc16, DT_F32, DT_F32, DT_F32, DT_F32, 16, false)

/* Fused residual add + LN profiles: x, res, h, y dtypes. */
#define NSR_RESLN_SET(PN, X, R, H, Y)                                           \
  NSR_LN_WAVE(nsrk_resln_##PN##_nc1, X, R, H, Y, 1, true)                        \
  NSR_LN_WAVE(nsrk_resln_##PN##_nc2, X, R, H, Y, 2, true)                        \
  NSR_LN_WAVE(nsrk_resln_##PN##_nc4, X, R, H, Y, 4, true)                        \
  NSR_LN_WAVE(nsrk_resln_##PN##_nc8, X, R, H, Y, 8, true)                        \
  NSR_LN_GENERIC(nsrk_resln_##PN##_generic, X, R, H, Y, true)

NSR_RESLN_SET(f32, DT_F32, DT_F32, DT_F32, DT_F32)
NSR_RESLN_SET(f16, DT_F16, DT_F16, DT_F16, DT_F16)
NSR_RESLN_SET(bf16, DT_BF16, DT_BF16, DT_BF16, DT_BF16)
/* moonshine decoder: f16 projection + f32 residual -> f32 residual, f16 norm */
NSR_RESLN_SET(f16f32, DT_F16, DT_F32, DT_F32, DT_F16)
NSR_LN_WAVE(nsrk_resln_f32_nc16, DT_F32, DT_F32, DT_F32, DT_F32, 16, true)
