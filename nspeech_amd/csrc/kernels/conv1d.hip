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
 * The tile is sized so that two workgroups fit on a CU (<= 80 KB of LDS for
 * (K - 1) * dilation <= 32): one stages its input while the other
 * multiplies.
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

typedef _Float16 nsr_h8 __attribute__((ext_vector_type(8)));
typedef float nsr_f32x16 __attribute__((ext_vector_type(16)));

#define CV_TT 64            /* output columns per workgroup */
#define CV_CO 128           /* output channels per workgroup */
#define CV_CI 128           /* input channels per LDS chunk */
#define CV_S (CV_CI + 8)    /* halfs per LDS row: 16-byte aligned, rows spread over banks */

NSR_DEV float conv_param(const void* p, int pdt, int64_t i) {
  return pdt == 0 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

NSR_DEV uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

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

/* Halo'd tile columns are staged 64 at a time (one per lane); at most
 * CV_JT x 64 columns: (K - 1) * dilation <= CV_JT * 64 - CV_TT. */
#define CV_JT 2

template <bool FUSED>
NSR_DEV void conv_body(const nsr_conv_args& a) {
  extern __shared__ uint16_t cv_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wco = wave >> 1, wt = wave & 1; /* the wave's 64-channel and 32-column block */
  const int t0 = blockIdx.x * CV_TT, co0 = blockIdx.y * CV_CO, b = blockIdx.z;
  const int TL = CV_TT + (a.K - 1) * a.dilation; /* staged columns */
  uint16_t* yhi = cv_lds;
  uint16_t* ylo = cv_lds + TL * CV_S;
  uint16_t* wb = cv_lds + 2 * TL * CV_S; /* weight slice [CV_CO][CV_S] of one tap k */
  const int hl = lane >> 5, l32 = lane & 31;

  nsr_f32x16 acc[2];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[m][i] = 0.f;

  /* weight slice staging: thread owns 16-byte chunks id = tid + 256 i of the
   * [128 co][16 chunks of 8 ci] slice */
  nsr_uint4 wr[8];
  auto load_w = [&](int k, int c0, int cc) {
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

  /* the staged columns of this lane: index clamped into the row (loads are
   * unconditional), value masked to zero outside it */
  int tcl[CV_JT];
  bool tin[CV_JT], jin[CV_JT];
#pragma unroll
  for (int jt = 0; jt < CV_JT; ++jt) {
    const int j = jt * 64 + lane, ti = t0 - a.padding + j;
    jin[jt] = j < TL;
    tin[jt] = ti >= 0 && ti < a.T_in;
    tcl[jt] = min(max(ti, 0), a.T_in - 1);
  }

  for (int c0 = 0; c0 < a.C_in; c0 += CV_CI) {
    const int cc = min(CV_CI, a.C_in - c0);
    load_w(0, c0, cc);
    __syncthreads(); /* the previous chunk's readers are done */

    /* stage y[c0 .. c0+cc) x [t0 - padding, t0 - padding + TL) as f16 hi/lo,
     * [t][ci]: wave w takes channel quads w, w + 4, ... (at most CV_CI / 16
     * of them); lanes run along t; every load of the chunk is issued before
     * the first value is used */
    {
      constexpr int QB = FUSED ? 2 : 4; /* quads per load batch (16 or 32 floats per lane in flight) */
      const float* xb = a.x + ((int64_t)b * a.C_in + c0) * a.T_in;
      const int nq = cc >> 2;
      for (int q0 = wave; q0 < nq; q0 += 4 * QB) {
        float v[QB][4][CV_JT];
#pragma unroll
        for (int i = 0; i < QB; ++i) {
          const int q = q0 + 4 * i;
          if (q < nq) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int jt = 0; jt < CV_JT; ++jt) v[i][r][jt] = xb[(int64_t)(4 * q + r) * a.T_in + tcl[jt]];
          }
        }
#pragma unroll
        for (int i = 0; i < QB; ++i) {
          const int q = q0 + 4 * i;
          if (q >= nq) break;
          cv_coef cf[4];
          if constexpr (FUSED) {
#pragma unroll
            for (int r = 0; r < 4; ++r) cf[r] = cv_row_coef(a, b, c0 + 4 * q + r);
          }
#pragma unroll
          for (int jt = 0; jt < CV_JT; ++jt) {
            if (!jin[jt]) continue;
            const int j = jt * 64 + lane;
            uint32_t hw[2], lw[2];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float y = v[i][r][jt];
              if constexpr (FUSED) y = snake_eval(__builtin_fmaf(y - cf[r].mean, cf[r].A, cf[r].bet), cf[r].sc);
              y = tin[jt] ? y : 0.f;
              const _Float16 hi = (_Float16)y;
              const _Float16 lo = (_Float16)(y - (float)hi);
              const uint32_t hb = h_bits(hi), lb = h_bits(lo);
              if (r & 1) {
                hw[r >> 1] |= hb << 16;
                lw[r >> 1] |= lb << 16;
              } else {
                hw[r >> 1] = hb;
                lw[r >> 1] = lb;
              }
            }
            *(nsr_uint2*)(yhi + j * CV_S + 4 * q) = nsr_uint2{hw[0], hw[1]};
            *(nsr_uint2*)(ylo + j * CV_S + 4 * q) = nsr_uint2{lw[0], lw[1]};
          }
        }
      }
    }
    store_w();
    __syncthreads();

    for (int k = 0; k < a.K; ++k) {
      if (k + 1 < a.K) load_w(k + 1, c0, cc); /* in flight during this tap's MFMAs */
      const int yoff = (wt * 32 + l32 + k * a.dilation) * CV_S + 8 * hl;
      const int a0 = (wco * 64 + l32) * CV_S + 8 * hl;
      /* two reduction steps per iteration: all LDS reads first */
      for (int g = 0; g < cc; g += 32) {
        const bool two = g + 16 < cc;
        nsr_h8 A[2][2], Bh[2], Bl[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int gg = g + 16 * s2;
          if (s2 == 1 && !two) break;
#pragma unroll
          for (int m = 0; m < 2; ++m) A[s2][m] = *(const nsr_h8*)(wb + a0 + m * 32 * CV_S + gg);
          Bh[s2] = *(const nsr_h8*)(yhi + yoff + gg);
          Bl[s2] = *(const nsr_h8*)(ylo + yoff + gg);
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          if (s2 == 1 && !two) break;
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[s2][m], Bh[s2], acc[m], 0, 0, 0);
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[s2][m], Bl[s2], acc[m], 0, 0, 0);
        }
      }
      if (k + 1 < a.K) {
        __syncthreads(); /* every wave is done with tap k's slice */
        store_w();
        __syncthreads();
      }
    }
  }

  /* epilogue: lane holds rows 8(i/4) + 4 hl + i%4 of column l32 of each 32 x 32 tile */
  const int t = t0 + wt * 32 + l32;
  if (t < a.T_out) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wco * 64 + m * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (co >= a.C_out) continue;
        const int64_t o = ((int64_t)b * a.C_out + co) * a.T_out + t;
        float v = acc[m][i];
        if (a.bias) v += f16_bits_to_f32(a.bias[co]);
        if (a.residual) v += a.residual[o];
        a.out[o] = v;
      }
  }
}

extern "C" __global__ void __launch_bounds__(256, 2) nsrk_conv1d_f16x2(const nsr_conv_args a) { conv_body<false>(a); }

extern "C" __global__ void __launch_bounds__(256, 2) nsrk_conv1d_adain_snake_f16x2(const nsr_conv_args a) {
  conv_body<true>(a);
}

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
