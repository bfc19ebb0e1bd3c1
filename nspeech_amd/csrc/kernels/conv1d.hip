/*
 * Kokoro resblock conv1d on MFMA (kernels/kokoro_kernels.py:773-816,
 * src/kokoro/decoder.rs:1352-1380), optionally with the AdaIN1d + Snake of
 * its input fused into the load:
 *   out[b, co, t] = bias[co] (+ residual[b, co, t])
 *                   + sum_{ci, k} w[co, ci, k] * y[b, ci, t - padding + k * dilation]
 * with y = x (conv1d_f32io) or y = snake(AdaIN(x)) (the resblock's
 * adain -> snake -> conv), y = 0 outside [0, T_in). Stride 1.
 *
 * Implicit GEMM: M = C_out, N = t, reduction r = (k, ci) (ci fastest, so the
 * weights are packed once to [C_out][K][C_in] and an A fragment is 8
 * consecutive input channels, one 16-byte load). A workgroup (4 waves,
 * 2 x 2) owns 128 output channels x 64 output columns. Per chunk of 128
 * input channels it stages y for the 128 columns plus the (K-1)*dilation
 * halo in LDS, transposed to [t][ci] so a B fragment is one 16-byte LDS
 * read, then runs the K * 8 reduction steps of v_mfma_f32_32x32x16_f16.
 * Workgroups are persistent (about two per CU) and walk the tiles; each
 * loads the next tile's input into registers right after staging the
 * current one, so the load latency overlaps the current tile's MFMAs,
 * weight staging and stores. The tile is sized so that two workgroups fit
 * on a CU (<= 80 KB of LDS for (K - 1) * dilation <= 32).
 * The weights of one tap k ([128 co][128 ci], 34 KB) sit in LDS too, shared
 * by the two waves of each channel block; tap k+1's slice is loaded into
 * registers while tap k's MFMAs run.
 *
 * f32 accuracy from f16 MFMA: the weights are f16 (exact); each f32
 * activation is split as y = hi + lo, hi = f16(y), lo = f16(y - hi), and
 * both halves are multiplied (two MFMAs per step). hi*w and lo*w are exact
 * in f32 and y - hi - lo is below 2^-22 |y| for normal-range f16 values, so
 * the sums carry f32-level error with f32 accumulation.
 */
#include "device_common.h"

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) nsr_uint4 lds_u4;
typedef __attribute__((address_space(3))) nsr_float4 lds_f4;

typedef _Float16 nsr_h8 __attribute__((ext_vector_type(8)));
typedef float nsr_f32x16 __attribute__((ext_vector_type(16)));

#define CV_TT 64            /* output columns per workgroup */
#define CV_CO 128           /* output channels per workgroup */
#define CV_CI 128           /* input channels per LDS chunk */
#define CV_S (CV_CI + 8)    /* halfs per LDS row: 16-byte aligned, rows spread over banks */

NSR_DEV float conv_param(const void* p, int pdt, int64_t i) {
  return pdt == 0 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

typedef _Float16 cv_h2 __attribute__((ext_vector_type(2)));

/* Two f32 values split into packed f16 halves: hi = f16(y), lo = f16(y - hi), both rounded to nearest
 * even; y0 in the low 16 bits. Built as two-element vectors so each pair converts with one
 * v_cvt_pk_f16_f32 instead of two conversions and a shift-or. */
NSR_DEV void split_pair(float y0, float y1, uint32_t& hi, uint32_t& lo) {
  const cv_h2 h = {(_Float16)y0, (_Float16)y1};
  const cv_h2 l = {(_Float16)(y0 - (float)h[0]), (_Float16)(y1 - (float)h[1])};
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

/* The same split with hi widened back from the packed register (the empty asm hides where it came
 * from, so the compiler does not convert y to f16 a second time): two VALU operations fewer per pair,
 * one more live register; for the records pass, whose registers are not its limit. */
NSR_DEV void split_pair_packed(float y0, float y1, uint32_t& hi, uint32_t& lo) {
  const cv_h2 h = {(_Float16)y0, (_Float16)y1};
  uint32_t hb = __builtin_bit_cast(uint32_t, h);
  asm("" : "+v"(hb));
  const cv_h2 hh = __builtin_bit_cast(cv_h2, hb);
  const cv_h2 l = {(_Float16)(y0 - (float)hh[0]), (_Float16)(y1 - (float)hh[1])};
  hi = hb;
  lo = __builtin_bit_cast(uint32_t, l);
}

/* Value of lane (this lane ^ 1) / (this lane ^ 2) within its quad (DPP quad_perm). */
NSR_DEV float quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
NSR_DEV float quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
/* Value of lane j of this lane's quad (DPP quad_perm [j, j, j, j]; j a constant after unrolling). */
NSR_DEV float quad_bcast(float v, int j) {
  const int x = __builtin_bit_cast(int, v);
  switch (j) {
    case 0: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x00, 0xF, 0xF, false));
    case 1: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x55, 0xF, 0xF, false));
    case 2: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xAA, 0xF, 0xF, false));
    default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xFF, 0xF, 0xF, false));
  }
}

/* AdaIN + Snake coefficients of input row (b, ci): y = snake((x - mean) A + beta). */
struct cv_coef {
  float mean, A, bet;
  snake_consts sc;
};

NSR_DEV cv_coef cv_row_coef(const nsr_conv_args& a, int b, int ci) {
  cv_coef c;
  const int64_t row = (int64_t)b * a.C_in + ci;
  c.mean = a.stats[2 * row];
  const float rstd = a.stats[2 * row + 1];
  c.A = (conv_param(a.gamma, a.pdt, (int64_t)b * a.gamma_bstride + ci) + 1.0f) * rstd;
  c.bet = conv_param(a.beta, a.pdt, (int64_t)b * a.beta_bstride + ci);
  c.sc = make_snake_consts(conv_param(a.alpha, a.pdt, ci));
  return c;
}


template <bool FUSED, int NP>
NSR_DEV void conv_body(const nsr_conv_args& a) {
  extern __shared__ uint16_t cv_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wco = wave >> 1, wt = wave & 1; /* the wave's 64-channel and 32-column block */
  const int hl = lane >> 5, l32 = lane & 31;
  const int TL = CV_TT + (a.K - 1) * a.dilation; /* staged columns */
  uint16_t* yhi = cv_lds;
  uint16_t* ylo = cv_lds + TL * CV_S;
  uint16_t* wb = cv_lds + 2 * TL * CV_S; /* weight slice [CV_CO][CV_S] of one tap k */
  const int n_t = (a.T_out + CV_TT - 1) / CV_TT, n_co = (a.C_out + CV_CO - 1) / CV_CO;
  const int n_tiles = n_t * n_co * a.B, n_ch = (a.C_in + CV_CI - 1) / CV_CI;

  /* tile -> (batch, first output channel, first column); channel blocks
   * fastest, then columns, so neighbouring tiles read the same or adjacent
   * input columns */
  auto coords = [&](int tile, int& b, int& co0, int& t0) {
    const int r = tile / n_co;
    co0 = (tile - r * n_co) * CV_CO;
    b = r / n_t;
    t0 = (r - b * n_t) * CV_TT;
  };
  /* The workgroups of one XCD (blockIdx % 8) walk one contiguous eighth of
   * the tiles together, slot s = blockIdx / 8 taking its s-th, (s + S)-th,
   * ... tile: the tiles in flight on an XCD are neighbours, so the halo
   * columns one tile shares with the next are read from HBM once and hit
   * that XCD's L2 the second time. (Grids that are not a multiple of 8
   * workgroups walk the tiles in plain strided order.) */
  const bool xcd = (gridDim.x & 7) == 0;
  const int xid = xcd ? (int)(blockIdx.x & 7) : 0, S = xcd ? (int)(gridDim.x >> 3) : (int)gridDim.x;
  const int slot = xcd ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int t_lo = xcd ? (int)((int64_t)n_tiles * xid / 8) : 0;
  const int t_hi = xcd ? (int)((int64_t)n_tiles * (xid + 1) / 8) : n_tiles;

  /* x of one (tile, chunk), in registers: lane owns channel quad
   * q = wave + 4 (lane / 8) (4 channels) at staged columns j = lane % 8 + 8 i,
   * i < NP (8 NP >= TL). Indices are clamped into the row, so every load is
   * unconditional; 8 lanes cover 32 consecutive bytes of a row per load. */
  const int lq = wave + 4 * (lane >> 3), lj = lane & 7;
  float xv[NP][4];
  auto fetch = [&](int tile, int ch) {
    int b, co0, t0;
    coords(tile, b, co0, t0);
    const int c0 = ch * CV_CI, nq = min(CV_CI, a.C_in - c0) >> 2;
    if (lq >= nq) return;
    /* this (batch, chunk)'s rows through one buffer descriptor: 32-bit offsets */
    const nsr_rsrc xr = make_rsrc_uniform(a.x + ((int64_t)b * a.C_in + c0) * a.T_in, 4u * (uint32_t)(nq * 4) * (uint32_t)a.T_in);
    const uint32_t rowoff = (uint32_t)(4 * lq) * (uint32_t)a.T_in;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int tc = min(max(t0 - a.padding + lj + 8 * i, 0), a.T_in - 1);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        xv[i][r] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(xr, (rowoff + (uint32_t)(r * a.T_in) + (uint32_t)tc) * 4u, 0, 0));
    }
  };

  nsr_uint4 wr[8]; /* one tap's weight slice, 16-byte chunks id = tid + 256 i of [128 co][16 x 8 ci] */
  auto load_w = [&](int co0, int k, int c0, int cc) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = tid + 256 * i, co = id >> 4, c8 = id & 15;
      const bool ok = co0 + co < a.C_out && 8 * c8 < cc;
      wr[i] = ok ? *(const nsr_uint4*)(a.w + ((int64_t)(co0 + co) * a.K + k) * a.C_in + c0 + 8 * c8)
                 : nsr_uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store_w = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = tid + 256 * i, co = id >> 4, c8 = id & 15;
      *(nsr_uint4*)(wb + co * CV_S + 8 * c8) = wr[i];
    }
  };

  if (t_lo + slot >= t_hi) return;
  fetch(t_lo + slot, 0);
  for (int tile = t_lo + slot; tile < t_hi; tile += S) {
    int b, co0, t0;
    coords(tile, b, co0, t0);
    nsr_f32x16 acc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[m][i] = 0.f;
    for (int ch = 0; ch < n_ch; ++ch) {
      const int c0 = ch * CV_CI, cc = min(CV_CI, a.C_in - c0), nq = cc >> 2;
      load_w(co0, 0, c0, cc);
      __syncthreads(); /* the previous item's readers of y and the weight slice are done */

      /* stage y = x (or snake(AdaIN(x))) as f16 hi/lo, [t][ci]; a lane's four
       * rows are transformed one row at a time (one row's coefficients live) */
      if (lq < nq) {
        if constexpr (FUSED) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const cv_coef cf = cv_row_coef(a, b, c0 + 4 * lq + r);
#pragma unroll
            for (int i = 0; i < NP; ++i) xv[i][r] = snake_eval(__builtin_fmaf(xv[i][r] - cf.mean, cf.A, cf.bet), cf.sc);
          }
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          const int j = lj + 8 * i;
          if (j >= TL) continue;
          const int ti = t0 - a.padding + j;
          const bool in = ti >= 0 && ti < a.T_in;
          uint32_t hw[2], lw[2];
#pragma unroll
          for (int r = 0; r < 2; ++r) split_pair(in ? xv[i][2 * r] : 0.f, in ? xv[i][2 * r + 1] : 0.f, hw[r], lw[r]);
          *(nsr_uint2*)(yhi + j * CV_S + 4 * lq) = nsr_uint2{hw[0], hw[1]};
          *(nsr_uint2*)(ylo + j * CV_S + 4 * lq) = nsr_uint2{lw[0], lw[1]};
        }
      }
      /* next item's input: in flight during this item's MFMAs and stores */
      {
        int ntile = tile, nch = ch + 1;
        if (nch == n_ch) {
          nch = 0;
          ntile += S;
        }
        if (ntile < t_hi) fetch(ntile, nch);
      }
      store_w();
      __syncthreads();

      for (int k = 0; k < a.K; ++k) {
        if (k + 1 < a.K) load_w(co0, k + 1, c0, cc); /* in flight during this tap's MFMAs */
        const int yoff = (wt * 32 + l32 + k * a.dilation) * CV_S + 8 * hl;
        const int a0 = (wco * 64 + l32) * CV_S + 8 * hl;
        for (int g = 0; g < cc; g += 16) {
          nsr_h8 A[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) A[m] = *(const nsr_h8*)(wb + a0 + m * 32 * CV_S + g);
          const nsr_h8 Bh = *(const nsr_h8*)(yhi + yoff + g);
          const nsr_h8 Bl = *(const nsr_h8*)(ylo + yoff + g);
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m], Bh, acc[m], 0, 0, 0);
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m], Bl, acc[m], 0, 0, 0);
        }
        if (k + 1 < a.K) {
          __syncthreads(); /* every wave is done with tap k's slice */
          store_w();
          __syncthreads();
        }
      }
    }

    /* epilogue: the accumulators (lane: rows 8(i/4) + 4 hl + i%4 of column
     * l32 of each 32 x 32 tile) go through LDS (the y area, free once every
     * wave is past its MFMAs) so that each row segment is written with
     * 16-byte stores, 16 lanes per 64-column row */
    __syncthreads();
    float* ot = (float*)cv_lds; /* [CV_CO][CV_TT + 1] */
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        ot[(wco * 64 + m * 32 + 8 * (i >> 2) + 4 * hl + (i & 3)) * (CV_TT + 1) + wt * 32 + l32] = acc[m][i];
    __syncthreads();
    const bool vec = (a.pad_ & 1) != 0; /* T_out % 4 == 0 and 16-byte aligned out / residual */
#pragma unroll
    for (int it = 0; it < CV_CO / 16; ++it) {
      const int row = it * 16 + (tid >> 4), c4 = (tid & 15) * 4;
      const int co = co0 + row, t = t0 + c4;
      if (co >= a.C_out || t >= a.T_out) continue;
      const float bv = a.bias ? f16_bits_to_f32(a.bias[co]) : 0.f;
      const int64_t o = ((int64_t)b * a.C_out + co) * a.T_out + t;
      const float* src = ot + row * (CV_TT + 1) + c4;
      if (vec && t + 3 < a.T_out) {
        nsr_float4 v = {src[0] + bv, src[1] + bv, src[2] + bv, src[3] + bv};
        if (a.residual) v += *(const nsr_float4*)(a.residual + o);
        *(nsr_float4*)(a.out + o) = v;
      } else {
        for (int e = 0; e < 4 && t + e < a.T_out; ++e) {
          float v = src[e] + bv;
          if (a.residual) v += a.residual[o + e];
          a.out[o + e] = v;
        }
      }
    }
  }
}

/*
 * Resident-weight variant for C_in <= 128, C_out <= 128 and K <= 3 (the
 * resblock's kernel-size-3 convs) with 16-byte aligned rows (T_in % 4 ==
 * T_out % 4 == 0). The whole packed weight tensor, [K][128 co][128 ci] f16
 * zero-padded, is loaded into LDS once per workgroup and stays there
 * (<= 102 KB), next to one staged input tile. One 512-lane workgroup per
 * CU, persistent over the tiles, in two roles that overlap:
 *  - waves 0-3 (consumers) run the tile's MFMAs, 2 x 2 waves of 64 channels
 *    x 32 columns; a 4 x 4 transpose across each lane quad (DPP) turns the
 *    accumulators into four consecutive columns of one channel per lane, so
 *    that they go, + bias (+ residual, loaded before the MFMAs), straight to
 *    memory as 16-byte stores that fill whole 128-byte lines (cached stores:
 *    measured faster here than streaming ones);
 *  - waves 4-7 (producers) keep the input two tiles ahead: during tile n
 *    they issue the 16-byte loads of tile n + 2, transform tile n + 1
 *    (AdaIN + Snake when FUSED, then the f16 hi/lo split) into packed
 *    registers while the consumers multiply, and write it to the LDS tile
 *    once the consumers are done with tile n. A producer lane owns a 4
 *    channel x 4 column block per step: 8 lanes cover 128 contiguous bytes
 *    of a row, and the LDS writes of a wave fall on distinct bank pairs but
 *    for a factor of two.
 * Two barriers per tile. Each role's loads are unconditional (clamped
 * indices, buffer range checks) and in a fixed order, so the compiler's
 * in-order memory-counter waits are exact: a producer waits for tile n + 1
 * with tile n + 2 still in flight, and a consumer waits for its residual
 * alone.
 */
/* Row statistics of the stored output for the next AdaIN (STATS kernels):
 * after the quad transpose, lanes hl*32 + 4j + c4 (j = 0..7) hold columns
 * t .. t + 3 of one output row, 32 columns of it per wave. For each such
 * row block the wave writes (mean, M2) of its valid columns (their count
 * follows from T_out), two passes over the registers with sums across the
 * 8 lanes: DPP rotations by 4 and 8 within each 16-lane row, then a swizzle
 * that exchanges the two rows of the 32-lane half (no LDS traffic for the
 * first two steps). nsrk_conv_rowstats_merge combines a row's blocks. */
NSR_DEV float sum_lanes8(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  return v + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

/* All eight row blocks of a wave's tile at once (m = 0..1, q = 0..3: row
 * co_lane + 32 m + 8 q), so the eight cross-lane sums are in flight together
 * and the block's column count is divided out once. FULLB: all 32 columns
 * of the block lie before T_out, so no column is masked; the arithmetic is
 * the same either way (a masked column adds 0 to the sum and fma(0, 0, .)
 * to M2), so a block's statistics do not depend on the variant. */
template <bool FULLB>
NSR_DEV void emit_rows8_v(const nsr_float4 (&ov)[2][4], int t, int tb, int T_out, int l32, int co_lane, int C_out,
                          int64_t row0, int nblk, int blk, float* part) {
  const int nv = FULLB ? 4 : max(0, min(4, T_out - t));
  const float n = FULLB ? 32.f : (float)max(0, min(32, T_out - tb)); /* valid columns of the block */
  const float inv_n = FULLB ? 1.0f / 32.0f : 1.0f / fmaxf(n, 1.f);
  float mean[8], m2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) s += (FULLB || e < nv) ? ov[i >> 2][i & 3][e] : 0.f;
    mean[i] = s;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) mean[i] = sum_lanes8(mean[i]) * inv_n;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float qv = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = (FULLB || e < nv) ? ov[i >> 2][i & 3][e] - mean[i] : 0.f;
      qv = __builtin_fmaf(d, d, qv);
    }
    m2[i] = qv;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) m2[i] = sum_lanes8(m2[i]);
  if (l32 < 4 && (FULLB || n > 0.f)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int co = co_lane + 32 * (i >> 2) + 8 * (i & 3);
      if (co < C_out) *(nsr_float2*)(part + 2 * ((row0 + co) * nblk + blk)) = nsr_float2{mean[i], m2[i]};
    }
  }
}

NSR_DEV void emit_rows8(const nsr_float4 (&ov)[2][4], int t, int tb, int T_out, int l32, int co_lane, int C_out,
                        int64_t row0, int nblk, int blk, float* part) {
  if (tb + 32 <= T_out) /* wave-uniform */
    emit_rows8_v<true>(ov, t, tb, T_out, l32, co_lane, C_out, row0, nblk, blk, part);
  else
    emit_rows8_v<false>(ov, t, tb, T_out, l32, co_lane, C_out, row0, nblk, blk, part);
}

template <bool FUSED, bool RESID, int NU, bool STATS = false>
NSR_DEV void conv_rw_body(const nsr_conv_args& a) {
  extern __shared__ uint16_t cv_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool producer = __builtin_amdgcn_readfirstlane(wave) >= 4; /* wave-uniform role */
  const int TL = CV_TT + (a.K - 1) * a.dilation;
  uint16_t* wl = cv_lds; /* [K][CV_CO][CV_S] */
  uint16_t* yhi = cv_lds + a.K * CV_CO * CV_S;
  uint16_t* ylo = yhi + TL * CV_S;
  const int n_t = (a.T_out + CV_TT - 1) / CV_TT;
  const int n_tiles = n_t * a.B;
  const int nq = a.C_in >> 2;

  const bool xcd = (gridDim.x & 7) == 0;
  const int xid = xcd ? (int)(blockIdx.x & 7) : 0, S = xcd ? (int)(gridDim.x >> 3) : (int)gridDim.x;
  const int slot = xcd ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int t_lo = xcd ? (int)((int64_t)n_tiles * xid / 8) : 0;
  const int t_hi = xcd ? (int)((int64_t)n_tiles * (xid + 1) / 8) : n_tiles;
  if (t_lo + slot >= t_hi) return;
  const int first = t_lo + slot, cnt = (t_hi - first + S - 1) / S; /* tiles of this workgroup */
  auto tile_of = [&](int n) { return first + min(n, cnt - 1) * S; };

  /* weights, once: [C_out][K][C_in] -> [k][co][ci], zero outside the
   * tensor; all loads issued before the first LDS write (K <= 3: at most 12
   * 16-byte chunks per lane) */
  {
    constexpr int NW = 3 * CV_CO * 16 / 512;
    nsr_uint4 wv[NW];
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const int id = tid + 512 * u, c8 = id & 15, row = id >> 4;
      const int k = row / CV_CO, co = row - k * CV_CO;
      const bool ok = k < a.K && co < a.C_out && 8 * c8 < a.C_in;
      const int64_t src = ok ? ((int64_t)co * a.K + k) * a.C_in + 8 * c8 : 0;
      wv[u] = *(const nsr_uint4*)(a.w + src);
      if (!ok) wv[u] = nsr_uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const int id = tid + 512 * u, row = id >> 4;
      if (row < a.K * CV_CO) *(nsr_uint4*)(wl + row * CV_S + 8 * (id & 15)) = wv[u];
    }
  }

  if (producer) {
    /* lane: channel quad lq (channels 4 lq .. 4 lq + 3) x column quads
     * jq = lane % 8 + 8 u, u < NU, of the window that starts at the
     * 16-byte aligned column s0 = (t0 - padding) rounded down to 4 */
    const int lq = 8 * (wave - 4) + (lane >> 3), jl = lane & 7;
    const bool live = lq < nq;
    const uint32_t rowoff = (uint32_t)(4 * min(lq, nq - 1)) * (uint32_t)a.T_in; /* lanes past C_in: discarded */
    const int dsh = (-a.padding) & 3; /* (t0 - padding) - s0, the same for every tile (t0 % 64 == 0) */
    nsr_float4 ra[NU][4], rb[NU][4];  /* [u][channel r]: 4 columns */
    uint32_t pk[NU][4][4];            /* [u][column e]: hi channels 0-1, 2-3, lo channels 0-1, 2-3 */
    cv_coef cf[FUSED ? 4 : 1];
    int coef_b = -1;
    auto fetch = [&](int n, nsr_float4 (&xv)[NU][4]) {
      const int tile = tile_of(n);
      const int b = tile / n_t, t0 = (tile - b * n_t) * CV_TT;
      const int s0 = t0 - a.padding - dsh;
      const nsr_rsrc xr = make_rsrc_uniform(a.x + (int64_t)b * a.C_in * a.T_in, 4u * (uint32_t)a.C_in * (uint32_t)a.T_in);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        /* a quad before column 0 wraps to a huge offset (range-checked to 0)
         * or reads the previous row's tail; either way it is masked below */
        const uint32_t col = (uint32_t)(s0 + 4 * (jl + 8 * u));
#pragma unroll
        for (int r = 0; r < 4; ++r)
          xv[u][r] = __builtin_bit_cast(nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        xr, (rowoff + (uint32_t)(r * a.T_in) + col) * 4u, 0, 0));
      }
    };
    auto transform = [&](int n, nsr_float4 (&xv)[NU][4]) {
      const int tile = tile_of(n);
      const int b = tile / n_t, t0 = (tile - b * n_t) * CV_TT;
      const int s0 = t0 - a.padding - dsh;
      if constexpr (FUSED) {
        if (b != coef_b) {
#pragma unroll
          for (int r = 0; r < 4; ++r) cf[r] = cv_row_coef(a, b, min(4 * lq + r, a.C_in - 1));
          coef_b = b;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              xv[u][r][e] = snake_eval(__builtin_fmaf(xv[u][r][e] - cf[r].mean, cf[r].A, cf[r].bet), cf[r].sc);
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ti = s0 + 4 * (jl + 8 * u) + e;
          const bool in = live && ti >= 0 && ti < a.T_in;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float y0 = in ? xv[u][2 * h][e] : 0.f, y1 = in ? xv[u][2 * h + 1][e] : 0.f;
            split_pair(y0, y1, pk[u][e][h], pk[u][e][2 + h]);
          }
        }
    };
    auto write = [&]() {
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * (jl + 8 * u) + e - dsh; /* staged column */
          if (j >= 0 && j < TL) {
            *(nsr_uint2*)(yhi + j * CV_S + 4 * lq) = nsr_uint2{pk[u][e][0], pk[u][e][1]};
            *(nsr_uint2*)(ylo + j * CV_S + 4 * lq) = nsr_uint2{pk[u][e][2], pk[u][e][3]};
          }
        }
    };
    /* phase n (tile n being multiplied): x(n + 2) -> `refill`, x(n + 1) in `ready` */
    auto phase = [&](int n, nsr_float4 (&refill)[NU][4], nsr_float4 (&ready)[NU][4]) {
      fetch(n + 2, refill);
      transform(n + 1, ready);
      __syncthreads(); /* consumers are done with tile n's input */
      write();
      __syncthreads(); /* tile n + 1's input is staged */
    };
    fetch(0, ra);
    fetch(1, rb);
    transform(0, ra);
    write();
    __syncthreads(); /* weights and tile 0 staged */
    for (int n = 0; n < cnt; n += 2) {
      phase(n, ra, rb);
      phase(n + 1, rb, ra);
    }
  } else {
    const int wco = wave >> 1, wt = wave & 1;
    const int hl = lane >> 5, l32 = lane & 31, c4 = lane & 3;
    /* accumulator element (m, i): channel wco*64 + m*32 + 8*(i/4) + 4*hl + i%4,
     * column wt*32 + l32. After the quad transpose, group q = i/4 of lane
     * (hl, l32) holds channel wco*64 + m*32 + 8*q + 4*hl + l32%4 at columns
     * wt*32 + 4*(l32/4) .. + 3. */
    float bias[2][4] = {};
    if (a.bias) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int co = wco * 64 + m * 32 + 8 * q + 4 * hl + c4;
          const float v = f16_bits_to_f32(a.bias[min(co, a.C_out - 1)]);
          bias[m][q] = co < a.C_out ? v : 0.f;
        }
    }
    const uint32_t obytes = 4u * (uint32_t)a.C_out * (uint32_t)a.T_out;
    const int wbase = (wco * 64 + l32) * CV_S + 8 * hl;
    const int ybase = (wt * 32 + l32) * CV_S + 8 * hl;
    __syncthreads(); /* weights and tile 0 staged */
    const int cnt2 = (cnt + 1) & ~1; /* the producers' phase count */
    for (int n = 0; n < cnt2; ++n) {
      const int tile = tile_of(n);
      const int b = tile / n_t, t0 = (tile - b * n_t) * CV_TT;
      const int t = t0 + wt * 32 + 4 * (l32 >> 2); /* this lane's column quad after the transpose */
      /* per-batch output (and residual) range: channels past C_out fall outside it */
      nsr_float4 rv[RESID ? 2 : 1][RESID ? 4 : 1];
      if constexpr (RESID) {
        const nsr_rsrc rr = make_rsrc_uniform(a.residual + (int64_t)b * a.C_out * a.T_out, obytes);
        const uint32_t tc = (uint32_t)min(t, a.T_out - 4);
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t co = (uint32_t)(wco * 64 + m * 32 + 8 * q + 4 * hl + c4);
            rv[m][q] = __builtin_bit_cast(nsr_float4,
                                          __builtin_amdgcn_raw_buffer_load_b128(rr, (co * (uint32_t)a.T_out + tc) * 4u, 0, 0));
          }
      }
      nsr_f32x16 acc[2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] = 0.f;
      {
        /* operands of step s = (k, g) live in A[s & 1], B[s & 1]; step s + 1's
         * are read before step s's MFMAs are issued */
        nsr_h8 A[2][2], Bh[2], Bl[2];
        auto ld = [&](int buf, int k, int g) {
          const uint16_t* wk = wl + k * CV_CO * CV_S + wbase + g;
          A[buf][0] = *(const nsr_h8*)wk;
          A[buf][1] = *(const nsr_h8*)(wk + 32 * CV_S);
          const int yo = ybase + k * a.dilation * CV_S + g;
          Bh[buf] = *(const nsr_h8*)(yhi + yo);
          Bl[buf] = *(const nsr_h8*)(ylo + yo);
        };
        ld(0, 0, 0);
        for (int k = 0; k < a.K; ++k) {
          const int kn = min(k + 1, a.K - 1); /* the last tap reloads its own first step (unused) */
#pragma unroll
          for (int g = 0; g < CV_CI; g += 16) {
            const int cur = (g >> 4) & 1; /* CV_CI / 16 = 8 steps per tap: parity restarts each tap */
            if (g + 16 < CV_CI) {
              ld(cur ^ 1, k, g + 16);
            } else {
              ld(cur ^ 1, kn, 0);
            }
#pragma unroll
            for (int m = 0; m < 2; ++m)
              acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[cur][m], Bh[cur], acc[m], 0, 0, 0);
#pragma unroll
            for (int m = 0; m < 2; ++m)
              acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[cur][m], Bl[cur], acc[m], 0, 0, 0);
          }
          /* keep the order written above: step g + 1's four LDS reads, then
           * step g's four MFMAs (the scheduler would otherwise sink each read
           * to its use and expose the LDS latency) */
#pragma unroll
          for (int g = 0; g < CV_CI; g += 16) {
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); /* DS reads */
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0); /* MFMA */
          }
        }
      }
      __syncthreads(); /* done with this tile's input */
      if (n < cnt) {
        const nsr_rsrc orr = make_rsrc_uniform(a.out + (int64_t)b * a.C_out * a.T_out, obytes);
        nsr_float4 ov[STATS ? 2 : 1][STATS ? 4 : 1];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            /* 4 x 4 transpose across the quad: slot r of lane c goes to slot c
             * of lane r, in two exchanges (lane bit 0, then bit 1) */
            float v[4] = {acc[m][4 * q], acc[m][4 * q + 1], acc[m][4 * q + 2], acc[m][4 * q + 3]};
            float x1[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) x1[r] = quad_xor1(v[r ^ 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 1) ? x1[r] : v[r];
#pragma unroll
            for (int r = 0; r < 4; ++r) x1[r] = quad_xor2(v[r ^ 2]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 2) ? x1[r] : v[r];
            const uint32_t co = (uint32_t)(wco * 64 + m * 32 + 8 * q + 4 * hl + c4);
            nsr_float4 o = {v[0] + bias[m][q], v[1] + bias[m][q], v[2] + bias[m][q], v[3] + bias[m][q]};
            if constexpr (RESID) o += rv[m][q];
            if (t < a.T_out) /* T_out % 4 == 0: t < T_out covers t + 3 */
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(nsr_uint4, o), orr,
                                                     (co * (uint32_t)a.T_out + (uint32_t)t) * 4u, 0, 0);
            if constexpr (STATS) ov[m][q] = o;
          }
        if constexpr (STATS)
          emit_rows8(ov, t, t0 + wt * 32, a.T_out, l32, wco * 64 + 4 * hl + c4, a.C_out, (int64_t)b * a.C_out,
                     (a.T_out + 31) >> 5, (t0 + wt * 32) >> 5, a.row_part);
      }
      __syncthreads(); /* the next tile's input is staged */
    }
  }
}

#define NSR_CONV_RW1(NAME, FUSED, RESID, NP)                                                         \
  extern "C" __global__ void __launch_bounds__(512, 1) NAME(const nsr_conv_args a) {                 \
    conv_rw_body<FUSED, RESID, NP>(a);                                                              \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(512, 1) NAME##_st(const nsr_conv_args a) {            \
    conv_rw_body<FUSED, RESID, NP, true>(a);                                                        \
  }
/* NU = column quads per producer lane / 8: staged window (TL + 3 alignment
 * columns) of at most 96 (NU 3) or 128 (NU 4) columns */
#define NSR_CONV_RW(NU)                                                                              \
  NSR_CONV_RW1(nsrk_conv1d_rw_f16x2_nu##NU, false, false, NU)                                        \
  NSR_CONV_RW1(nsrk_conv1d_rw_res_f16x2_nu##NU, false, true, NU)                                     \
  NSR_CONV_RW1(nsrk_conv1d_rw_adain_snake_f16x2_nu##NU, true, false, NU)                             \
  NSR_CONV_RW1(nsrk_conv1d_rw_adain_snake_res_f16x2_nu##NU, true, true, NU)

NSR_CONV_RW(3)
NSR_CONV_RW(4)

/*
 * Streamed-weight producer/consumer variant: any K, C_in in chunks of 128,
 * C_out in blocks of 128, 16-byte aligned rows (T_in % 4 == T_out % 4 == 0)
 * and a staged window (TL + 3 alignment columns) of at most 128 columns.
 * One 512-lane workgroup per CU, persistent over the items (tile, input
 * chunk), tiles ordered channel block fastest:
 *  - waves 0-3 (consumers) multiply tap k from one LDS weight slot while
 *    tap k + 1's weights ([128 co][128 ci], 32 KB) travel through their
 *    registers into the other slot: one barrier per tap (the last tap of an
 *    item loads the next item's first). Each slice is read from L2 once per
 *    CU (loading A fragments per wave instead doubles the L1 traffic, which
 *    measured slower). After a tile's last
 *    chunk they store it as the resident-weight kernel does (quad transpose,
 *    16-byte stores, + bias, + residual loaded before the last chunk's MFMAs);
 *  - waves 4-7 (producers) keep the input two items ahead as in the
 *    resident-weight kernel and write the next item's staged tile once the
 *    consumers are past its last tap.
 * K + 1 barriers per item.
 */
template <bool FUSED, bool RESID, int NU, bool STATS = false>
NSR_DEV void conv_pc_body(const nsr_conv_args& a) {
  extern __shared__ uint16_t cv_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool producer = __builtin_amdgcn_readfirstlane(wave) >= 4; /* wave-uniform role */
  const int TL = CV_TT + (a.K - 1) * a.dilation;
  uint16_t* yhi = cv_lds;
  uint16_t* ylo = yhi + TL * CV_S;
  uint16_t* wsl = ylo + TL * CV_S; /* two weight slots [CV_CO][CV_S] */
  float* bias_l = (float*)(wsl + 2 * CV_CO * CV_S); /* [C_out] (0 without bias) */
  const int n_t = (a.T_out + CV_TT - 1) / CV_TT, n_co = (a.C_out + CV_CO - 1) / CV_CO;
  const int n_ch = (a.C_in + CV_CI - 1) / CV_CI;
  const int n_tiles = n_t * n_co * a.B;

  const bool xcd = (gridDim.x & 7) == 0;
  const int xid = xcd ? (int)(blockIdx.x & 7) : 0, S = xcd ? (int)(gridDim.x >> 3) : (int)gridDim.x;
  const int slot = xcd ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int t_lo = xcd ? (int)((int64_t)n_tiles * xid / 8) : 0;
  const int t_hi = xcd ? (int)((int64_t)n_tiles * (xid + 1) / 8) : n_tiles;
  if (t_lo + slot >= t_hi) return;
  const int first = t_lo + slot, cnt = (t_hi - first + S - 1) / S; /* tiles of this workgroup */
  const int items = cnt * n_ch, items2 = (items + 1) & ~1;       /* phases: even, the last ones repeat */
  /* item n -> tile (b, co0, t0) and input chunk c0 */
  auto item_of = [&](int n, int& b, int& co0, int& t0, int& c0) {
    const int nn = min(n, items - 1);
    const int tn = nn / n_ch, ch = nn - tn * n_ch;
    const int tile = first + tn * S;
    const int r = tile / n_co;
    co0 = (tile - r * n_co) * CV_CO;
    b = r / n_t;
    t0 = (r - b * n_t) * CV_TT;
    c0 = ch * CV_CI;
  };

  if (producer) {
    const int lq = 8 * (wave - 4) + (lane >> 3), jl = lane & 7;
    const int dsh = (-a.padding) & 3;
    nsr_float4 ra[NU][4], rb[NU][4];
    uint32_t pk[NU][4][4];
    cv_coef cf[FUSED ? 4 : 1];
    int coef_key = -1;
    auto fetch = [&](int n, nsr_float4 (&xv)[NU][4]) {
      int b, co0, t0, c0;
      item_of(n, b, co0, t0, c0);
      const int nq = min(CV_CI, a.C_in - c0) >> 2;
      const uint32_t rowoff = (uint32_t)(4 * min(lq, nq - 1)) * (uint32_t)a.T_in;
      const int s0 = t0 - a.padding - dsh;
      const nsr_rsrc xr = make_rsrc_uniform(a.x + ((int64_t)b * a.C_in + c0) * a.T_in, 4u * (uint32_t)(nq * 4) * (uint32_t)a.T_in);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const uint32_t col = (uint32_t)(s0 + 4 * (jl + 8 * u));
#pragma unroll
        for (int r = 0; r < 4; ++r)
          xv[u][r] = __builtin_bit_cast(nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        xr, (rowoff + (uint32_t)(r * a.T_in) + col) * 4u, 0, 0));
      }
    };
    auto transform = [&](int n, nsr_float4 (&xv)[NU][4]) {
      int b, co0, t0, c0;
      item_of(n, b, co0, t0, c0);
      const int nq = min(CV_CI, a.C_in - c0) >> 2;
      const bool live = lq < nq;
      const int s0 = t0 - a.padding - dsh;
      if constexpr (FUSED) {
        const int key = b * n_ch + (c0 / CV_CI);
        if (key != coef_key) {
#pragma unroll
          for (int r = 0; r < 4; ++r) cf[r] = cv_row_coef(a, b, c0 + min(4 * lq + r, 4 * nq - 1));
          coef_key = key;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              xv[u][r][e] = snake_eval(__builtin_fmaf(xv[u][r][e] - cf[r].mean, cf[r].A, cf[r].bet), cf[r].sc);
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ti = s0 + 4 * (jl + 8 * u) + e;
          const bool in = live && ti >= 0 && ti < a.T_in;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float y0 = in ? xv[u][2 * h][e] : 0.f, y1 = in ? xv[u][2 * h + 1][e] : 0.f;
            split_pair(y0, y1, pk[u][e][h], pk[u][e][2 + h]);
          }
        }
    };
    auto write = [&]() {
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * (jl + 8 * u) + e - dsh;
          if (j >= 0 && j < TL) {
            *(nsr_uint2*)(yhi + j * CV_S + 4 * lq) = nsr_uint2{pk[u][e][0], pk[u][e][1]};
            *(nsr_uint2*)(ylo + j * CV_S + 4 * lq) = nsr_uint2{pk[u][e][2], pk[u][e][3]};
          }
        }
    };
    auto phase = [&](int n, nsr_float4 (&refill)[NU][4], nsr_float4 (&ready)[NU][4]) {
      fetch(n + 2, refill);
      transform(n + 1, ready);
      for (int k = 0; k < a.K; ++k) __syncthreads(); /* the consumers' taps of item n */
      write();
      __syncthreads(); /* item n + 1's input is staged */
    };
    fetch(0, ra);
    fetch(1, rb);
    transform(0, ra);
    write();
    __syncthreads(); /* item 0's input, tap 0's weights and the bias staged */
    for (int n = 0; n < items2; n += 2) {
      phase(n, ra, rb);
      phase(n + 1, rb, ra);
    }
  } else {
    const int wco = wave >> 1, wt = wave & 1;
    const int hl = lane >> 5, l32 = lane & 31, c4 = lane & 3;
    const uint32_t obytes = 4u * (uint32_t)a.C_out * (uint32_t)a.T_out;
    /* weight slice (item n, tap k) -> registers: 16-byte chunks id = tid + 256 i of [128 co][16 x 8 ci] */
    nsr_uint4 wr[8];
    auto load_w = [&](int n, int k) {
      int b, co0, t0, c0;
      item_of(n, b, co0, t0, c0);
      const int cc = min(CV_CI, a.C_in - c0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int id = tid + 256 * i, co = id >> 4, c8 = id & 15;
        const bool ok = co0 + co < a.C_out && 8 * c8 < cc;
        const int64_t src = ok ? ((int64_t)(co0 + co) * a.K + k) * a.C_in + c0 + 8 * c8 : 0;
        wr[i] = *(const nsr_uint4*)(a.w + src);
        if (!ok) wr[i] = nsr_uint4{0u, 0u, 0u, 0u};
      }
    };
    auto store_w = [&](int sl) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int id = tid + 256 * i;
        *(nsr_uint4*)(wsl + sl * CV_CO * CV_S + (id >> 4) * CV_S + 8 * (id & 15)) = wr[i];
      }
    };
    for (int c = tid; c < a.C_out; c += 256) bias_l[c] = a.bias ? f16_bits_to_f32(a.bias[c]) : 0.f;
    load_w(0, 0);
    store_w(0);
    int ws = 0; /* slot of the tap about to be multiplied */
    __syncthreads(); /* item 0's input, tap 0's weights and the bias staged */
    const int wbase = (wco * 64 + l32) * CV_S + 8 * hl;
    const int ybase = (wt * 32 + l32) * CV_S + 8 * hl;
    nsr_f32x16 acc[2];
    for (int n = 0; n < items2; ++n) {
      int b, co0, t0, c0;
      item_of(n, b, co0, t0, c0);
      const bool last_chunk = c0 + CV_CI >= a.C_in;
      const int t = t0 + wt * 32 + 4 * (l32 >> 2);
      if (c0 == 0) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[m][i] = 0.f;
      }
      nsr_float4 rv[RESID ? 2 : 1][RESID ? 4 : 1];
      for (int k = 0; k < a.K; ++k) {
        if constexpr (RESID) {
          /* at the tile's last tap, ahead of the weight load, so the epilogue waits for it alone */
          if (k == a.K - 1 && last_chunk) {
            const nsr_rsrc rr = make_rsrc_uniform(a.residual + (int64_t)b * a.C_out * a.T_out, obytes);
            const uint32_t tc = (uint32_t)min(t, a.T_out - 4);
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const uint32_t co = (uint32_t)(co0 + wco * 64 + m * 32 + 8 * q + 4 * hl + c4);
                rv[m][q] = __builtin_bit_cast(
                    nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(rr, (co * (uint32_t)a.T_out + tc) * 4u, 0, 0));
              }
          }
        }
        /* next tap's weights (or the next item's first) into registers during this tap's MFMAs */
        if (k + 1 < a.K) {
          load_w(n, k + 1);
        } else {
          load_w(n + 1, 0);
        }
        const uint16_t* wk0 = wsl + ws * CV_CO * CV_S + wbase;
        const int yk = ybase + k * a.dilation * CV_S;
        nsr_h8 A[2][2], Bh[2], Bl[2];
        auto ld = [&](int buf, int g) {
          A[buf][0] = *(const nsr_h8*)(wk0 + g);
          A[buf][1] = *(const nsr_h8*)(wk0 + 32 * CV_S + g);
          Bh[buf] = *(const nsr_h8*)(yhi + yk + g);
          Bl[buf] = *(const nsr_h8*)(ylo + yk + g);
        };
        ld(0, 0);
#pragma unroll
        for (int g = 0; g < CV_CI; g += 16) {
          const int cur = (g >> 4) & 1;
          if (g + 16 < CV_CI) ld(cur ^ 1, g + 16);
#pragma unroll
          for (int m = 0; m < 2; ++m)
            acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[cur][m], Bh[cur], acc[m], 0, 0, 0);
#pragma unroll
          for (int m = 0; m < 2; ++m)
            acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[cur][m], Bl[cur], acc[m], 0, 0, 0);
        }
        /* order: steps 0 and 1's reads, step 0's MFMAs, then step g + 1's
         * reads before step g's MFMAs (the scheduler would otherwise sink each
         * read to its use and expose the LDS latency) */
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
#pragma unroll
        for (int g = 16; g < CV_CI - 16; g += 16) {
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        store_w(ws ^ 1); /* that slot's last readers (the previous tap) were past the previous barrier */
        ws ^= 1;
        __syncthreads(); /* tap k done everywhere; the next tap's weights staged */
      }
      if (last_chunk && n < items) {
        const nsr_rsrc orr = make_rsrc_uniform(a.out + (int64_t)b * a.C_out * a.T_out, obytes);
        nsr_float4 ov[STATS ? 2 : 1][STATS ? 4 : 1];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v[4] = {acc[m][4 * q], acc[m][4 * q + 1], acc[m][4 * q + 2], acc[m][4 * q + 3]};
            float x1[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) x1[r] = quad_xor1(v[r ^ 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 1) ? x1[r] : v[r];
#pragma unroll
            for (int r = 0; r < 4; ++r) x1[r] = quad_xor2(v[r ^ 2]);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 2) ? x1[r] : v[r];
            const int co = co0 + wco * 64 + m * 32 + 8 * q + 4 * hl + c4;
            const float bv = bias_l[min(co, a.C_out - 1)];
            nsr_float4 o = {v[0] + bv, v[1] + bv, v[2] + bv, v[3] + bv};
            if constexpr (RESID) o += rv[m][q];
            if (t < a.T_out)
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(nsr_uint4, o), orr,
                                                     ((uint32_t)co * (uint32_t)a.T_out + (uint32_t)t) * 4u, 0, 0);
            if constexpr (STATS) ov[m][q] = o;
          }
        if constexpr (STATS)
          emit_rows8(ov, t, t0 + wt * 32, a.T_out, l32, co0 + wco * 64 + 4 * hl + c4, a.C_out, (int64_t)b * a.C_out,
                     (a.T_out + 31) >> 5, (t0 + wt * 32) >> 5, a.row_part);
      }
      __syncthreads(); /* the next item's input is staged */
    }
  }
}

#define NSR_CONV_PC1(NAME, FUSED, RESID, NU)                                                         \
  extern "C" __global__ void __launch_bounds__(512, 1) NAME(const nsr_conv_args a) {                 \
    conv_pc_body<FUSED, RESID, NU>(a);                                                              \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(512, 1) NAME##_st(const nsr_conv_args a) {            \
    conv_pc_body<FUSED, RESID, NU, true>(a);                                                        \
  }
#define NSR_CONV_PC(NU)                                                                              \
  NSR_CONV_PC1(nsrk_conv1d_pc_f16x2_nu##NU, false, false, NU)                                        \
  NSR_CONV_PC1(nsrk_conv1d_pc_res_f16x2_nu##NU, false, true, NU)                                     \
  NSR_CONV_PC1(nsrk_conv1d_pc_adain_snake_f16x2_nu##NU, true, false, NU)                             \
  NSR_CONV_PC1(nsrk_conv1d_pc_adain_snake_res_f16x2_nu##NU, true, true, NU)

NSR_CONV_PC(3)
NSR_CONV_PC(4)

#define CV_TW 128           /* output columns per tile of the record kernel */

/* --------------------------------------------- conv on pre-split input records -- */

/* The MFMA kernel without per-element VALU work. On gfx950 a VALU
 * instruction issued on a SIMD delays that SIMD's MFMAs by several cycles
 * (measured: about 10 cycles of MFMA time per VALU instruction of another
 * wave), so the elementwise work of the resblock input (AdaIN + Snake, the
 * f16 hi / lo split, the transpose to [t][ci]) is done beforehand by
 * nsrk_conv_presplit, a bandwidth-bound pass, into records: for input column
 * tp - padding (tp = 0 .. T_out + (K - 1) dilation - 1) and each chunk of 128
 * input channels, 512 bytes = 16 chunks of 8 hi halves then 16 of 8 lo
 * halves (zeros outside the row and past C_in). The same pass writes the
 * weights in MFMA fragment order: for each block of 32 output channels cb,
 * tap k, channel chunk ch and step g, 1 KB = 64 lanes x 16 bytes, lane
 * (l32, hl) holding w[32 cb + l32][k][128 ch + 16 g + 8 hl .. + 7].
 *
 * Tiles are 128 output channels x 128 columns; each workgroup takes a
 * contiguous run of them (channel block fastest, then columns), so the next
 * tile's window of TL = 128 + (K - 1) dilation records shares all or
 * TL - 128 of its records with the current one. Records live in an LDS ring
 * of 256 slots of 528 bytes (record tp in slot tp & 255; the 16-byte pad puts
 * consecutive records in different bank groups, so 16 lanes reading one
 * chunk of 16 consecutive records do not conflict):
 *  - consumers (waves 0-3, 64 channels x 64 columns each as 2 x 2
 *    accumulators) read B fragments from the ring and hold their A
 *    fragments in registers, loaded one tap ahead straight from the fragment
 *    weights (one 1 KB load per fragment, L2-resident);
 *  - the record waves (4-7) load the next window's new records into
 *    registers at the start of an item and write each into its slot as soon
 *    as the record it replaces is dead: at once when the slot is free, after
 *    tap K - 2 when it holds a record that only earlier taps read, after the
 *    last tap otherwise (then one more barrier before the next item; never
 *    for consecutive tiles of one row with an even (K - 1) dilation).
 * Two barriers per item. LDS: 256 x 528 bytes. */
#define CV_RB 512           /* bytes per record */
#define CV_RS 528           /* bytes per record slot in LDS */
#define CV_RING 256         /* record slots in LDS */
#define CV_NRW 24           /* record rounds per transition: 24 x 8 records >= the largest window (192) */

struct cv_item {
  int b, co0, t0, ch;
};

/* The records of item n + 1 that item n's window lacks: [nb, ne) of (b, ch) of the next item. */
struct cv_trans {
  int nb, ne;
};

/* FULL32 (STATS only): T_out % 32 == 0, so every 32-column block is whole or
 * lies past T_out, and the statistics need no column masks (the masked form
 * and the dispatch between the two would not fit the kernel's registers). */
template <bool RESID, bool STATS = false, bool FULL32 = false>
NSR_DEV void conv_pr_body(const nsr_conv_args& a, const uint8_t* xs, const uint8_t* wf) {
  extern __shared__ __attribute__((aligned(16))) uint8_t cv_ring[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* wave-uniform: role and tile math in SALU */
  const int D = (a.K - 1) * a.dilation;
  const int TLe = CV_TW + D + (D & 1);             /* window length, rounded to even */
  const int Tp = a.T_out + D;                       /* records per (batch, channel chunk) */
  const int n_t = (a.T_out + CV_TW - 1) / CV_TW, n_co = (a.C_out + CV_CO - 1) / CV_CO;
  const int n_ch = (a.C_in + CV_CI - 1) / CV_CI;
  const int n_tiles = n_t * n_co * a.B;

  /* XCD-aware: XCD x (blocks x, x + 8, ...) takes an eighth of the tiles; each workgroup a contiguous run */
  const int G = (int)gridDim.x;
  const bool xcd = (G & 7) == 0;
  const int nx = xcd ? 8 : 1, xid = xcd ? (int)(blockIdx.x & 7) : 0;
  const int S = G / nx, slot = xcd ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int x_lo = (int)((int64_t)n_tiles * xid / nx), x_hi = (int)((int64_t)n_tiles * (xid + 1) / nx);
  const int first = x_lo + (int)((int64_t)(x_hi - x_lo) * slot / S);
  const int last = x_lo + (int)((int64_t)(x_hi - x_lo) * (slot + 1) / S);
  if (first >= last) return;
  const int items = (last - first) * n_ch;
  /* item n = tile first + n / n_ch, channel chunk n % n_ch; tiles run channel block fastest, then
   * columns, then batch. The first item is decoded once, the others by stepping (no divisions). */
  cv_item first_item;
  {
    const int r = first / n_co;
    first_item.ch = 0;
    first_item.co0 = (first - r * n_co) * CV_CO;
    first_item.b = r / n_t;
    first_item.t0 = (r - first_item.b * n_t) * CV_TW;
  }
  auto advance = [&](cv_item& it) {
    if (++it.ch < n_ch) return;
    it.ch = 0;
    it.co0 += CV_CO;
    if (it.co0 < n_co * CV_CO) return;
    it.co0 = 0;
    it.t0 += CV_TW;
    if (it.t0 < n_t * CV_TW) return;
    it.t0 = 0;
    ++it.b;
  };
  /* the records of window nx that window cu lacks: [nb, ne) (cu == nullptr: none present) */
  auto trans = [&](const cv_item* cu, const cv_item& nx_) {
    cv_trans tr;
    tr.nb = nx_.t0;
    tr.ne = nx_.t0 + TLe;
    if (cu && cu->b == nx_.b && cu->ch == nx_.ch && nx_.t0 >= cu->t0 && nx_.t0 < cu->t0 + TLe) tr.nb = cu->t0 + TLe;
    return tr;
  };
  /* slot phase of a new record: 0 = its slot is free during item n, 1 = freed by tap K - 2, 2 = freed by
   * the last tap (d = slot distance from the current window's start) */
  auto phase_of = [&](int d) { return d >= TLe ? 0 : (d < D ? 1 : 2); };
  /* Output staging: after item n's last tap its tile (row r = output channel co0 + r, 128 columns f32)
   * goes to LDS while the ring holds window n + 1 (start nt0): rows r < FS in the ring slots outside
   * that window, (nt0 + TLe + r) & 255, the other 128 - FS <= 56 rows after the ring. nt0 is a multiple
   * of 128 and TLe + FS <= 256, so those slots never wrap: slot ((nt0 + TLe) & 255) + r. */
  const int FS = (CV_RING - TLe) / 8 * 8;
  auto stage_ring = [&](int nt0, int r) {
    return (uint32_t)((nt0 + TLe) & (CV_RING - 1)) * CV_RS + (uint32_t)r * CV_RS;
  };
  auto stage_tail = [&](int r) { return (uint32_t)(CV_RING * CV_RS + (r - FS) * 512); };

  if (wave >= 4) {
    /* record waves: pairs of records per wave and round (lanes 0-31 record q, 32-63 record q + 1) */
    const int w4 = wave - 4;
    const uint32_t vl = (uint32_t)((lane >> 5) * CV_RS + (lane & 31) * 16);
    nsr_uint4 yr[CV_NRW];
    /* Per-lane addresses are computed only before the first item and between an item's last two
     * barriers, while the consumers run their epilogue: a VALU instruction issued while the consumer wave
     * on the same SIMD streams MFMAs waits for a gap in that stream (and delays it), so what runs during
     * the taps is memory and scalar instructions only. (The empty asm keeps the compiler from computing
     * the addresses again where they are used.) */
    auto pin = [](uint32_t& v) { asm volatile("" : "+v"(v)); };
    auto pin_u4 = [](lds_u4*& p) { asm volatile("" : "+v"(p)); };
    auto pin_f4 = [](lds_f4*& p) { asm volatile("" : "+v"(p)); };
    uint32_t vlo = (uint32_t)lane * 16u;
    pin(vlo);
    lds_u4* waddr[CV_NRW]; /* ring address of round r's pair in the coming transition */
    auto calc_waddr = [&](const cv_trans& tr) {
#pragma unroll
      for (int r = 0; r < CV_NRW; ++r) {
        waddr[r] = (lds_u4*)(cv_ring + (uint32_t)((tr.nb + 2 * (4 * r + w4)) & (CV_RING - 1)) * CV_RS + vl);
        pin_u4(waddr[r]);
      }
    };
    /* The staged tile of an item to global memory: pairs of rows (lanes 0-31 row 2 j, 32-63 row 2 j + 1,
     * 16 bytes per lane: 512 contiguous bytes per row). Wave w takes the pairs in the ring slots that it
     * will itself overwrite with records of the transition after the next item (pair j sits in slot
     * nt0 + TLe + 2 j, written by wave ((slot - nb2) / 2) & 3 of that transition), so no other wave
     * overwrites a row before it is read. */
    auto staged_jw = [&](int nt0, int nb2) { return (w4 - (((nt0 + TLe - nb2) & (CV_RING - 1)) >> 1)) & 3; };
    lds_f4* saddr[16];
    uint32_t svo = 0, sok = 0;
    auto calc_saddr = [&](const cv_item& im, int nt0, int jw) {
      const int quad = lane & 31, t = im.t0 + 4 * quad;
      svo = (uint32_t)(lane >> 5) * (uint32_t)a.T_out * 4u + (uint32_t)t * 4u;
      sok = t < a.T_out ? 1u : 0u;
      pin(svo);
      pin(sok);
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const int r0 = 2 * (jw + 4 * p);
        /* rows r0, r0 + 1: slot nt0 + TLe + r0 is even, so its neighbour does not wrap */
        saddr[p] = (lds_f4*)(cv_ring + (r0 < FS ? stage_ring(nt0, r0) + (uint32_t)(lane >> 5) * CV_RS
                                                : stage_tail(r0) + (uint32_t)(lane >> 5) * 512u) + 16u * (uint32_t)quad);
        pin_f4(saddr[p]);
      }
    };
    /* the staged rows of item m: read into registers before this wave's records overwrite their slots,
     * stored after the records are written, one 16-byte store per lane every `gap` sleep units, spread
     * over the taps so the consumers' A fragment loads do not queue behind a burst */
    nsr_float4 sv[16];
    auto read_staged = [&]() {
#pragma unroll
      for (int p = 0; p < 16; ++p) sv[p] = *saddr[p];
    };
    auto store_staged = [&](const cv_item& im, int jw, int gap) {
      const uint32_t obytes = 4u * (uint32_t)a.C_out * (uint32_t)a.T_out;
      const nsr_rsrc orr = make_rsrc_uniform(a.out + (int64_t)im.b * a.C_out * a.T_out, obytes);
      /* the residual (variants without statistics add it here), loaded 4 passes ahead */
      const nsr_rsrc rr = make_rsrc_uniform(RESID ? a.residual + (int64_t)im.b * a.C_out * a.T_out : a.out, obytes);
      nsr_float4 rq[RESID && !STATS ? 4 : 1];
      auto load_rq = [&](int p) {
        const int r0 = 2 * (jw + 4 * p);
        rq[p & 3] = __builtin_bit_cast(nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rr, svo, (uint32_t)(im.co0 + r0) * (uint32_t)a.T_out * 4u, 0));
      };
      if constexpr (RESID && !STATS) {
#pragma unroll
        for (int p = 0; p < 4; ++p) load_rq(p);
      }
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const int r0 = 2 * (jw + 4 * p);
        nsr_float4 v = sv[p];
        if constexpr (RESID && !STATS) {
          v += rq[p & 3];
          if (p + 4 < 16) load_rq(p + 4);
        }
        /* C_out is even on this path: both rows of a pair exist or neither */
        if (sok && im.co0 + r0 < a.C_out)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(nsr_uint4, v), orr, svo,
                                                 (uint32_t)(im.co0 + r0) * (uint32_t)a.T_out * 4u, 0);
        for (int z = 0; z < gap; ++z) __builtin_amdgcn_s_sleep(1);
      }
    };
    /* rolling items: ip = n - 1, ic = n, in = n + 1, in2 = n + 2 (valid below `items`); tc = the
     * transition n -> n + 1 */
    cv_item ip = first_item, ic = first_item, in = first_item, in2 = first_item;
    advance(in2);
    cv_trans tc = trans(nullptr, in);
    calc_waddr(tc);
    int jw_p = 0; /* staging pairs of item n - 1 */
    /* sleep units (64 cycles) between staged stores: 16 stores over about (K - 2) / 2 taps */
    const int gap = max(1, 3 * (a.K - 2) / 2);
    for (int n = -1; n < items; ++n) {
      const bool has_next = n + 1 < items;
      if (has_next) {
        const nsr_rsrc xr =
            make_rsrc_uniform(xs + ((int64_t)in.b * n_ch + in.ch) * Tp * CV_RB, (uint32_t)Tp * (uint32_t)CV_RB);
        /* 16 rounds always (128 new records for consecutive tiles; rounds past the new records re-read
         * the last pair), 8 more for a window that shares nothing with the current one */
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int q = min(tc.nb + 2 * (4 * r + w4), tc.ne - 2);
          yr[r] = __builtin_amdgcn_raw_buffer_load_b128(xr, vlo, (uint32_t)q * CV_RB, NSR_AUX_NT);
        }
        if (tc.ne - tc.nb > 128) {
#pragma unroll
          for (int r = 16; r < CV_NRW; ++r) {
            const int q = min(tc.nb + 2 * (4 * r + w4), tc.ne - 2);
            yr[r] = __builtin_amdgcn_raw_buffer_load_b128(xr, vlo, (uint32_t)q * CV_RB, NSR_AUX_NT);
          }
        }
      }
      const bool staged = n >= 1 && ip.ch == n_ch - 1;
      /* the rounds of each phase as bit masks, computed once per transition (scalar work here is shared
       * with the consumers' waves: one test per round and phase below) */
      uint32_t pm[3] = {0u, 0u, 0u};
      if (has_next) {
        const int dd = tc.nb + 2 * w4 - ic.t0;
#pragma unroll
        for (int r = 0; r < CV_NRW; ++r) {
          if (tc.nb + 2 * (4 * r + w4) < tc.ne) {
            const int d = (dd + 8 * r) & (CV_RING - 1); /* even; the pair's second record is d + 1 */
            const int p = n < 0 ? 0 : max(phase_of(d), phase_of((d + 1) & (CV_RING - 1)));
            pm[p] |= 1u << r;
          }
        }
        NSR_WAIT_VMCNT(0);
      }
      auto write_phase = [&](int ph) {
#pragma unroll
        for (int r = 0; r < CV_NRW; ++r)
          if ((pm[ph] >> r) & 1u) *waddr[r] = yr[r];
      };
      /* the staged rows are read once the records have arrived (not at the item's start, where their
       * LDS reads would meet the consumers' first tap), then this wave's records overwrite their slots */
      if (staged) read_staged();
      write_phase(0);
      if (staged) store_staged(ip, jw_p, gap);
      const bool has_next2 = n + 2 < items;
      const cv_trans tn = has_next2 ? trans(&in, in2) : tc;
      if (n < 0) {
        if (has_next2) calc_waddr(tn);
        __syncthreads(); /* item 0's window staged */
      } else {
        if (a.K > 1) __syncthreads(); /* taps 0 .. K - 2 of item n done */
        write_phase(1);
        __syncthreads(); /* item n done */
        write_phase(2);
        /* the consumers' epilogue: the next transition's and the staged tile's addresses */
        if (has_next2) calc_waddr(tn);
        if (ic.ch == n_ch - 1) {
          const int nt0 = has_next ? in.t0 : ic.t0;
          jw_p = staged_jw(nt0, has_next2 ? tn.nb : 0);
          calc_saddr(ic, nt0, jw_p);
        }
        __syncthreads(); /* item n + 1's window and item n's output staged */
      }
      ip = ic;
      ic = in;
      in = in2;
      advance(in2);
      tc = tn;
    }
    if (ip.ch == n_ch - 1) {
      read_staged();
      store_staged(ip, jw_p, 0);
    }
  } else {
    const int wco = wave >> 1, wt = wave & 1;
    const int hl = lane >> 5, l32 = lane & 31, c4 = lane & 3;
    const uint32_t obytes = 4u * (uint32_t)a.C_out * (uint32_t)a.T_out;
    const uint32_t kstride = (uint32_t)n_ch * 8192u, cbstride = (uint32_t)a.K * kstride;
    const nsr_rsrc wr = make_rsrc_uniform(wf, (uint32_t)n_co * 4u * cbstride);
    /* fragment weights of (item, tap) for this wave's 64 channels (m = 0: cb, m = 1: cb + 1) */
    auto a_base = [&](const cv_item& it, int k) {
      return (uint32_t)(it.co0 / 32 + 2 * wco) * cbstride + (uint32_t)k * kstride + (uint32_t)it.ch * 8192u;
    };
    nsr_h8 A[2][8];
    {
      const uint32_t ab = a_base(first_item, 0);
#pragma unroll
      for (int g = 0; g < 8; ++g)
#pragma unroll
        for (int m = 0; m < 2; ++m)
          A[m][g] = __builtin_bit_cast(nsr_h8, __builtin_amdgcn_raw_buffer_load_b128(
                                                    wr, (uint32_t)lane * 16u, ab + m * cbstride + g * 1024u, 0));
    }
    nsr_f32x16 acc[2][2];
    /* residual of column block tb (the statistics variants add it here; the others' record waves add it
     * when they store the tile) */
    nsr_float4 rv[RESID ? 2 : 1][RESID ? 2 : 1][RESID ? 4 : 1];
    auto load_resid = [&](const cv_item& it, int tb) {
      const nsr_rsrc rr = make_rsrc_uniform(a.residual + (int64_t)it.b * a.C_out * a.T_out, obytes);
      const uint32_t tc = (uint32_t)min(it.t0 + wt * 64 + tb * 32 + 4 * (l32 >> 2), a.T_out - 4);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t co = (uint32_t)(it.co0 + wco * 64 + m * 32 + 8 * q + 4 * hl + c4);
          rv[tb][m][q] = __builtin_bit_cast(
              nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(rr, (co * (uint32_t)a.T_out + tc) * 4u, 0, 0));
        }
    };
    uint32_t braw[2][4];
    int bias_co0 = -1;
    __syncthreads(); /* item 0's window staged */
    NSR_WAIT_VMCNT(0); /* tap 0 of every item starts with its A fragments in place (see the epilogue) */
    cv_item it = first_item, in = first_item;
    advance(in);
    for (int n = 0; n < items; ++n) {
      const bool last_chunk = it.ch == n_ch - 1;
      const bool has_next = n + 1 < items;
      const cv_item nxt = has_next ? in : it;
      if (it.ch == 0) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][tb][i] = 0.f;
      }
      if (last_chunk && it.co0 != bias_co0) {
        /* the bias of this lane's 8 output channels, raw halves loaded when the channel block changes
         * and converted in the epilogue (a conversion here would wait for every older memory operation) */
        const uint16_t* bsrc = a.bias ? a.bias : (const uint16_t*)a.w; /* any readable halves when there is no bias */
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) braw[m][q] = bsrc[min(it.co0 + wco * 64 + m * 32 + 8 * q + 4 * hl + c4, a.C_out - 1)];
        bias_co0 = it.co0;
      }
      const int j0 = it.t0 + 64 * wt + l32;
      /* one tap; tap 0 is issued on its own (peeled) so its waits for the A fragments loaded before the
       * previous item's epilogue count that epilogue's stores as younger operations, instead of sharing
       * the loop's waits and so waiting for the stores too */
      auto tap = [&](int k, auto reload) {
        /* B fragment (tb, step g): record j0 + 32 tb + k dilation, hi chunk 2 g + hl, lo 256 bytes further */
        const int j = j0 + k * a.dilation;
        uint32_t va[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) va[tb] = (uint32_t)((j + 32 * tb) & (CV_RING - 1)) * CV_RS + (uint32_t)hl * 16u;
        /* the A fragments of the next tap (or of the next item's tap 0; the last item's own tap 0 after
         * the last tap, a load never used) replace this tap's, step by step, unconditionally so the
         * tap is one basic block the schedule below can order */
        const uint32_t ab = k + 1 < a.K ? a_base(it, k + 1) : a_base(nxt, 0);
        nsr_h8 Bh[2][2], Bl[2][2];
        auto ld = [&](int buf, int g) {
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            Bh[buf][tb] = *(const nsr_h8*)(cv_ring + va[tb] + 32 * g);
            Bl[buf][tb] = *(const nsr_h8*)(cv_ring + va[tb] + 256 + 32 * g);
          }
        };
        ld(0, 0);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const int cur = g & 1;
          if (g + 1 < 8) ld(cur ^ 1, g + 1);
#pragma unroll
          for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
              acc[m][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m][g], Bh[cur][tb], acc[m][tb], 0, 0, 0);
#pragma unroll
          for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
              acc[m][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m][g], Bl[cur][tb], acc[m][tb], 0, 0, 0);
          if constexpr (decltype(reload)::value) {
#pragma unroll
            for (int m = 0; m < 2; ++m)
              A[m][g] = __builtin_bit_cast(nsr_h8, __builtin_amdgcn_raw_buffer_load_b128(
                                                        wr, (uint32_t)lane * 16u, ab + m * cbstride + g * 1024u, 0));
          }
        }
        /* order: step 0's reads, then per step: the next step's reads, its 8 MFMAs, its 2 A reloads */
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int g = 0; g < 7; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
        if (k == a.K - 2) __syncthreads(); /* taps 0 .. K - 2 done: their records may be replaced */
      };
      /* with a residual and statistics the last tap does not reload: the epilogue's registers would not
       * hold the next item's A fragments as well, which are loaded after it instead */
      constexpr bool last_reload = !(RESID && STATS);
      tap(0, std::true_type{});
      for (int k = 1; k < a.K - 1; ++k) tap(k, std::true_type{});
      if (a.K > 1) tap(a.K - 1, std::bool_constant<last_reload>{});
      __syncthreads(); /* item n done */
      /* the next tap's A fragments (loaded during the last tap) have arrived by now: waiting for them
       * here keeps tap 0 of the next item free of waits */
      NSR_WAIT_VMCNT(0);
      if (last_chunk) {
        float bv[2][4];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) bv[m][q] = a.bias ? f16_bits_to_f32((uint16_t)braw[m][q]) : 0.f;
        /* row r of the staged tile: in the ring (row groups of 8 lie wholly in the ring or after it) */
        auto stage_row = [&](int R0, int r) { return R0 < FS ? stage_ring(nxt.t0, r) : stage_tail(r); };
        if constexpr (!STATS) {
          /* accumulator element i of lane (hl, l32) is channel 8 (i / 4) + 4 hl + i % 4 of its 32-channel
           * block at column l32: dword writes, 32 consecutive columns per half-wave, no cross-lane moves;
           * bv[m][q] holds channel 8 q + 4 hl + c4, so the bias of element i is in quad lane i % 4. A group
           * of 8 rows lies wholly in the ring (stride CV_RS) or after it (stride 512): its base and stride
           * are wave-uniform, so a row's address is one add from the group's. */
          const int wcu = __builtin_amdgcn_readfirstlane(wco);
          const uint32_t lcol = (uint32_t)(64 * wt + l32) * 4u;
#pragma unroll
          for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int R0 = 64 * wcu + 32 * m + 8 * g4;
              const bool ring = R0 < FS;
              const uint32_t rs = ring ? (uint32_t)CV_RS : 512u;
              uint32_t la = stage_row(R0, R0) + (uint32_t)(4 * hl) * rs + lcol;
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                const int i = 4 * g4 + c;
                const float bi = quad_bcast(bv[m][g4], c);
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) *(float*)(cv_ring + la + 128u * tb) = acc[m][tb][i] + bi;
                la += rs;
              }
            }
        } else {
          /* row statistics: the quad transpose gives each lane 4 consecutive columns */
          if constexpr (RESID) {
            load_resid(it, 0);
            load_resid(it, 1);
          }
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) {
            const int tl = wt * 64 + tb * 32 + 4 * (l32 >> 2), t = it.t0 + tl;
            nsr_float4 ov[2][4];
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float v[4] = {acc[m][tb][4 * q], acc[m][tb][4 * q + 1], acc[m][tb][4 * q + 2], acc[m][tb][4 * q + 3]};
                float x1[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) x1[r] = quad_xor1(v[r ^ 1]);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 1) ? x1[r] : v[r];
#pragma unroll
                for (int r = 0; r < 4; ++r) x1[r] = quad_xor2(v[r ^ 2]);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = ((r ^ c4) & 2) ? x1[r] : v[r];
                const float bb = bv[m][q];
                nsr_float4 o = {v[0] + bb, v[1] + bb, v[2] + bb, v[3] + bb};
                if constexpr (RESID) o += rv[tb][m][q];
                const int R0 = 64 * wco + 32 * m + 8 * q;
                *(nsr_float4*)(cv_ring + stage_row(R0, R0 + 4 * hl + c4) + (uint32_t)tl * 4u) = o;
                ov[m][q] = o;
              }
            const int tbk = it.t0 + wt * 64 + tb * 32;
            if constexpr (FULL32) {
              if (tbk < a.T_out)
                emit_rows8_v<true>(ov, t, tbk, a.T_out, l32, it.co0 + wco * 64 + 4 * hl + c4, a.C_out,
                                   (int64_t)it.b * a.C_out, (a.T_out + 31) >> 5, tbk >> 5, a.row_part);
            } else {
              emit_rows8_v<false>(ov, t, tbk, a.T_out, l32, it.co0 + wco * 64 + 4 * hl + c4, a.C_out,
                                  (int64_t)it.b * a.C_out, (a.T_out + 31) >> 5, tbk >> 5, a.row_part);
            }
          }
        }
      }
      if constexpr (!last_reload) {
        const uint32_t ab = a_base(nxt, 0);
#pragma unroll
        for (int g = 0; g < 8; ++g)
#pragma unroll
          for (int m = 0; m < 2; ++m)
            A[m][g] = __builtin_bit_cast(nsr_h8, __builtin_amdgcn_raw_buffer_load_b128(
                                                      wr, (uint32_t)lane * 16u, ab + m * cbstride + g * 1024u, 0));
      }
      __syncthreads(); /* item n + 1's window and item n's output staged */
      it = in;
      advance(in);
    }
    NSR_WAIT_VMCNT(0); /* the last tap's unused reloads */
  }
}

#define NSR_CONV_PR1(NAME, RESID)                                                                    \
  extern "C" __global__ void __launch_bounds__(512, 1)                                              \
      NAME(const nsr_conv_args a, const uint8_t* xs, const uint8_t* wf) {                           \
    conv_pr_body<RESID>(a, xs, wf);                                                                 \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(512, 1)                                              \
      NAME##_st(const nsr_conv_args a, const uint8_t* xs, const uint8_t* wf) {                      \
    conv_pr_body<RESID, true>(a, xs, wf);                                                           \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(512, 1)                                              \
      NAME##_st32(const nsr_conv_args a, const uint8_t* xs, const uint8_t* wf) {                    \
    conv_pr_body<RESID, true, true>(a, xs, wf);                                                     \
  }
NSR_CONV_PR1(nsrk_conv1d_pr_f16x2, false)
NSR_CONV_PR1(nsrk_conv1d_pr_res_f16x2, true)

/* Records and fragment weights for nsrk_conv1d_pr*. Record tp (tp = 0 ..
 * T_in + 2 padding - 1, input column tp - padding) of channel chunk ch holds
 * y = x (or snake(AdaIN(x)) in the fused form, with the row statistics in
 * a.stats) of channels 128 ch .. 128 ch + 127 split as hi = f16(y),
 * lo = f16(y - hi): 16 chunks of 8 hi halves, then 16 of 8 lo halves; zeros
 * outside [0, T_in) and past C_in. One 256-lane workgroup per 64 input
 * columns 64 j .. 64 j + 63 of one (batch, chunk), j from -ceil(padding / 64)
 * so the blocks before column 0 cover the leading padding records; blocks
 * are aligned to the input rows (not to the padded columns), so a row's 64
 * columns are two whole 128-byte lines when rows start on 16 bytes. Each
 * lane loads 8 channels x 4 columns (one 16-byte load per channel, 64
 * consecutive columns per row across 16 lanes), transforms and packs them
 * into its chunks of 4 records in LDS, then the block's records (64 j +
 * padding onwards, those in [0, T_in + 2 padding)) are stored contiguously:
 * records are 512 bytes, so the stores stay aligned. Bandwidth-bound: x read once, the
 * records written once (4 bytes per element each way). The workgroups after
 * the records' write the fragment weights, 16 bytes per lane. Blocks are
 * mapped XCD-contiguously (XCD x takes the x-th eighth of the logical
 * blocks), so neighbouring blocks, which share the cache lines at their
 * column boundary, run on one L2. */
template <bool FUSED>
NSR_DEV void conv_presplit(const nsr_conv_args& a, uint8_t* xs, uint8_t* wf) {
  __shared__ __attribute__((aligned(16))) uint8_t rec[64 * CV_RS];
  __shared__ __attribute__((aligned(16))) float coef[FUSED ? CV_CI * 12 : 4];
  const int tid = threadIdx.x, rg = tid >> 4, cq = tid & 15;
  const int Tp = a.T_in + 2 * a.padding;
  const int jlo = (a.padding + 63) / 64; /* blocks before input column 0 */
  const int nblk = (a.T_in + a.padding + 63) / 64 + jlo, n_ch = (a.C_in + CV_CI - 1) / CV_CI;
  const int G = (int)gridDim.x;
  const int lb = (G & 7) == 0 ? (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int nrb = a.B * n_ch * nblk;
  if (lb >= nrb) {
    /* fragment weights: 16 bytes per lane */
    const int n_co = (a.C_out + CV_CO - 1) / CV_CO;
    const int64_t f = (int64_t)(lb - nrb) * 256 + tid; /* 16-byte unit */
    const int64_t nf = (int64_t)n_co * 4 * a.K * n_ch * 512;
    if (f >= nf) return;
    const int ln = (int)(f & 63);
    int64_t grp = f >> 6;
    const int g = (int)(grp & 7);
    grp >>= 3;
    const int ch = (int)(grp % n_ch);
    grp /= n_ch;
    const int k = (int)(grp % a.K);
    const int cb = (int)(grp / a.K);
    const int co = 32 * cb + (ln & 31), ci0 = CV_CI * ch + 16 * g + 8 * (ln >> 5);
    uint32_t hv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t lo16 = 0, hi16 = 0;
      if (co < a.C_out) {
        const uint16_t* wrow = a.w + ((int64_t)co * a.K + k) * a.C_in;
        if (ci0 + 2 * e < a.C_in) lo16 = wrow[ci0 + 2 * e];
        if (ci0 + 2 * e + 1 < a.C_in) hi16 = wrow[ci0 + 2 * e + 1];
      }
      hv[e] = lo16 | (hi16 << 16);
    }
    *(nsr_uint4*)(wf + f * 16) = nsr_uint4{hv[0], hv[1], hv[2], hv[3]};
    return;
  }
  const int bc = lb / nblk; /* b * n_ch + ch */
  const int j64 = (lb - bc * nblk - jlo) * 64; /* the block's first input column */
  const int b = bc / n_ch, ch = bc - b * n_ch;
  const int c0 = ch * CV_CI + 8 * rg; /* this lane's 8 channels */
  const int ti0 = j64 + 4 * cq;      /* its 4 input columns ti0 .. ti0 + 3 */
  /* the whole block inside the row and the channel chunk full: nothing to zero (wave-uniform) */
  const bool full = j64 >= 0 && j64 + 63 < a.T_in && (ch + 1) * CV_CI <= a.C_in;
  const nsr_rsrc xr = make_rsrc_uniform(a.x + (int64_t)b * a.C_in * a.T_in, 4u * (uint32_t)a.C_in * (uint32_t)a.T_in);
  /* Interior lanes: one 16-byte load per channel (4-byte aligned offsets). Lanes whose 4 columns cross
   * either end of the row load each column on its own at a clamped column, so no load leaves the
   * batch's buffer; those columns, and channels past C_in, are zeroed below. */
  float y[8][4];
  if (ti0 >= 0 && ti0 + 3 < a.T_in) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = min(c0 + i, a.C_in - 1);
      const nsr_float4 v = __builtin_bit_cast(
          nsr_float4, __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)((int64_t)c * a.T_in + ti0) * 4u, 0, NSR_AUX_NT));
#pragma unroll
      for (int e = 0; e < 4; ++e) y[i][e] = v[e];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = min(c0 + i, a.C_in - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ti = min(max(ti0 + e, 0), a.T_in - 1);
        y[i][e] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)((int64_t)c * a.T_in + ti) * 4u, 0, NSR_AUX_NT));
      }
    }
  }
  if constexpr (FUSED) {
    /* the AdaIN + Snake coefficients of the 128 channels, once per workgroup (lane c: channel 128 ch + c),
     * then each lane reads its 8 channels' from LDS */
    if (tid < CV_CI) {
      const cv_coef cf = cv_row_coef(a, b, min(ch * CV_CI + tid, a.C_in - 1));
      *(nsr_float4*)(coef + 12 * tid) = nsr_float4{cf.mean, cf.A, cf.bet, cf.sc.a_pi};
      *(nsr_float4*)(coef + 12 * tid + 4) = nsr_float4{cf.sc.c[0], cf.sc.c[1], cf.sc.c[2], cf.sc.c[3]};
      *(nsr_float4*)(coef + 12 * tid + 8) = nsr_float4{cf.sc.c[4], cf.sc.c[5], cf.sc.c[6], 0.f};
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool crow = c0 + i < a.C_in;
    if constexpr (FUSED) {
      const float* cp = coef + 12 * (8 * rg + i);
      const nsr_float4 q0 = *(const nsr_float4*)cp, q1 = *(const nsr_float4*)(cp + 4), q2 = *(const nsr_float4*)(cp + 8);
      cv_coef cf;
      cf.mean = q0[0];
      cf.A = q0[1];
      cf.bet = q0[2];
      cf.sc.a_pi = q0[3];
      cf.sc.c[0] = q1[0];
      cf.sc.c[1] = q1[1];
      cf.sc.c[2] = q1[2];
      cf.sc.c[3] = q1[3];
      cf.sc.c[4] = q2[0];
      cf.sc.c[5] = q2[1];
      cf.sc.c[6] = q2[2];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[i][e] = snake_eval(__builtin_fmaf(y[i][e] - cf.mean, cf.A, cf.bet), cf.sc);
      __builtin_amdgcn_sched_barrier(0); /* one channel's coefficients live at a time */
    }
    if (!full) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ti = ti0 + e;
        y[i][e] = (crow && ti >= 0 && ti < a.T_in) ? y[i][e] : 0.f;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) split_pair_packed(y[2 * h][e], y[2 * h + 1][e], hi[h], lo[h]);
    /* record 4 cq + e sits in LDS slot 16 e + cq: the 16 lanes of one chunk (cq = 0 .. 15) write 16
     * consecutive slots, which the 528-byte stride puts in 16 different bank groups */
    const int sl = 16 * e + cq;
    *(nsr_uint4*)(rec + sl * CV_RS + 16 * rg) = nsr_uint4{hi[0], hi[1], hi[2], hi[3]};
    *(nsr_uint4*)(rec + sl * CV_RS + 256 + 16 * rg) = nsr_uint4{lo[0], lo[1], lo[2], lo[3]};
  }
  __syncthreads();
  /* record r of the block is tp = j64 + padding + r; the buffer covers the block's records inside
   * [0, Tp), so stores of the others (negative or past-the-end offsets) are dropped by its range check */
  const int tq = j64 + a.padding, tlo = max(tq, 0), thi = min(tq + 64, Tp);
  const nsr_rsrc orr = make_rsrc_uniform(xs + ((int64_t)bc * Tp + tlo) * CV_RB, (uint32_t)((thi - tlo) * CV_RB));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = tid + 256 * i; /* 16-byte chunk: slot id >> 5, chunk id & 31 */
    const int sl = id >> 5, r = 4 * (sl & 15) + (sl >> 4); /* the slot's record */
    __builtin_amdgcn_raw_buffer_store_b128(*(const nsr_uint4*)(rec + sl * CV_RS + 16 * (id & 31)), orr,
                                           (uint32_t)((r + tq - tlo) * CV_RB + 16 * (id & 31)), 0, NSR_AUX_NT);
  }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_conv_presplit(const nsr_conv_args a, uint8_t* xs, uint8_t* wf) {
  conv_presplit<false>(a, xs, wf);
}
extern "C" __global__ void __launch_bounds__(256)
    nsrk_conv_presplit_adain_snake(const nsr_conv_args a, uint8_t* xs, uint8_t* wf) {
  conv_presplit<true>(a, xs, wf);
}




/* NP = ceil(TL / 8) staged columns per lane: TL <= 72, 96, 128 */
/* OCC, OCCF: workgroups per CU the register budget of the plain and the
 * fused kernel is sized for (NP 9 plain: two, which the LDS of short halos
 * allows; the others one: the fused NP 9 kernel needs more than 256
 * registers per lane) */
#define NSR_CONV(NP, OCC, OCCF)                                                                          \
  extern "C" __global__ void __launch_bounds__(256, OCC) nsrk_conv1d_f16x2_np##NP(const nsr_conv_args a) { \
    conv_body<false, NP>(a);                                                                            \
  }                                                                                                     \
  extern "C" __global__ void __launch_bounds__(256, OCCF)                                               \
      nsrk_conv1d_adain_snake_f16x2_np##NP(const nsr_conv_args a) {                                     \
    conv_body<true, NP>(a);                                                                             \
  }

NSR_CONV(9, 2, 1)
NSR_CONV(12, 1, 1)
NSR_CONV(16, 1, 1)

/* [C_out][C_in][K] -> [C_out][K][C_in], one thread per weight. */
extern "C" __global__ void __launch_bounds__(256) nsrk_conv1d_pack(const nsr_conv_pack_args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = a.C_out * a.C_in * a.K;
  if (i >= n) return;
  const int64_t co = i / (a.C_in * a.K);
  const int64_t r = i - co * a.C_in * a.K;
  const int64_t ci = r / a.K, k = r - ci * a.K;
  a.wp[(co * a.K + k) * a.C_in + ci] = a.w[i];
}

/* Merge a row's (mean, M2) blocks (Chan, Golub and LeVeque's pairwise
 * update: n = na + nb, d = mb - ma, mean = ma + d nb / n,
 * M2 = M2a + M2b + d^2 na nb / n; block i holds min(32, T_out - 32 i)
 * columns) into the row's mean and 1 / sqrt(M2 / n + eps), the statistics
 * the fused AdaIN+Snake conv reads. One workgroup per row; each lane merges
 * blocks i = tid + 256 k in order (eight loads in flight at a time), then a
 * fixed tree over the lanes: the result does not depend on timing. */
NSR_DEV void chan_merge(float& n, float& mean, float& m2, float nb, float mb, float m2b) {
  const float nn = n + nb;
  if (nb > 0.f) {
    const float d = mb - mean;
    const float f = nb / nn;
    mean = __builtin_fmaf(d, f, mean);
    m2 = m2 + m2b + d * d * n * f;
    n = nn;
  }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_conv_rowstats_merge(const nsr_rowstats_args a) {
  __shared__ float sn[256], sm[256], sq[256];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const nsr_float2* pr = (const nsr_float2*)a.part + row * a.nblk;
  float n = 0.f, mean = 0.f, m2 = 0.f;
  for (int i0 = 0; i0 < a.nblk; i0 += 8 * 256) {
    nsr_float2 p[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + tid + 256 * u;
      p[u] = pr[min(i, a.nblk - 1)];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + tid + 256 * u;
      const float nb = i < a.nblk ? (float)min(32, a.T_out - 32 * i) : 0.f;
      chan_merge(n, mean, m2, nb, p[u].x, p[u].y);
    }
  }
  sn[tid] = n;
  sm[tid] = mean;
  sq[tid] = m2;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) {
      float n0 = sn[tid], m0 = sm[tid], q0 = sq[tid];
      chan_merge(n0, m0, q0, sn[tid + w], sm[tid + w], sq[tid + w]);
      sn[tid] = n0;
      sm[tid] = m0;
      sq[tid] = q0;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const float var = fmaxf(sq[0] / fmaxf(sn[0], 1.f), 0.f);
    a.stats[2 * row] = sm[0];
    a.stats[2 * row + 1] = 1.0f / sqrtf(var + a.eps);
  }
}
