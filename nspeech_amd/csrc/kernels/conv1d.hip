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
 * 2 x 2) owns 128 output channels x 128 output columns. Per chunk of 128
 * input channels it stages y for the 128 columns plus the (K-1)*dilation
 * halo in LDS, transposed to [t][ci] so a B fragment is one 16-byte LDS
 * read, then runs the K * 8 reduction steps of v_mfma_f32_32x32x16_f16.
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

#define CV_TT 128           /* output columns per workgroup */
#define CV_CO 128           /* output channels per workgroup */
#define CV_CI 128           /* input channels per LDS chunk */
#define CV_S (CV_CI + 8)    /* halfs per LDS row: 16-byte aligned, rows spread over banks */
#define CV_NCOEF 12         /* floats per input channel: mean, A, beta, snake consts */

NSR_DEV float conv_param(const void* p, int pdt, int64_t i) {
  return pdt == 0 ? ((const float*)p)[i] : f16_bits_to_f32(((const uint16_t*)p)[i]);
}

NSR_DEV uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

template <bool FUSED>
NSR_DEV void conv_body(const nsr_conv_args& a) {
  extern __shared__ uint16_t cv_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wco = wave >> 1, wt = wave & 1; /* the wave's 64-channel and 64-column block */
  const int t0 = blockIdx.x * CV_TT, co0 = blockIdx.y * CV_CO, b = blockIdx.z;
  const int TL = CV_TT + (a.K - 1) * a.dilation; /* staged columns */
  uint16_t* yhi = cv_lds;
  uint16_t* ylo = cv_lds + TL * CV_S;
  float* coef = (float*)(cv_lds + 2 * TL * CV_S);

  nsr_f32x16 acc[2][2];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[m][n][i] = 0.f;

  const int hl = lane >> 5, l32 = lane & 31;
  int co_l[2];
  bool co_ok[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    co_l[m] = co0 + wco * 64 + m * 32 + l32;
    co_ok[m] = co_l[m] < a.C_out;
  }
  const nsr_h8 hzero = {};

  for (int c0 = 0; c0 < a.C_in; c0 += CV_CI) {
    const int cc = min(CV_CI, a.C_in - c0);
    __syncthreads(); /* the previous chunk's readers are done */
    if constexpr (FUSED) {
      if (tid < cc) {
        const int64_t row = (int64_t)b * a.C_in + c0 + tid;
        const int ci = c0 + tid;
        const float mean = a.stats[2 * row], rstd = a.stats[2 * row + 1];
        const float gam = conv_param(a.gamma, a.pdt, (int64_t)b * a.gamma_bstride + ci);
        const float bet = conv_param(a.beta, a.pdt, (int64_t)b * a.beta_bstride + ci);
        const snake_consts sc = make_snake_consts(conv_param(a.alpha, a.pdt, ci));
        float* cf = coef + tid * CV_NCOEF;
        cf[0] = mean;
        cf[1] = (gam + 1.0f) * rstd;
        cf[2] = bet;
        cf[3] = sc.a_pi;
#pragma unroll
        for (int q = 0; q < 7; ++q) cf[4 + q] = sc.c[q];
      }
      __syncthreads();
    }
    /* stage y[c0 .. c0+cc) x [t0 - padding, t0 - padding + TL) as f16 hi/lo, [t][ci] */
    const float* xb = a.x + ((int64_t)b * a.C_in + c0) * a.T_in;
    for (int e = tid; e < cc * TL; e += 256) {
      const int ci = e / TL, j = e - ci * TL;
      const int ti = t0 - a.padding + j;
      float v = 0.f;
      if (ti >= 0 && ti < a.T_in) {
        v = xb[(int64_t)ci * a.T_in + ti];
        if constexpr (FUSED) {
          const float* cf = coef + ci * CV_NCOEF;
          snake_consts sc;
          sc.a_pi = cf[3];
#pragma unroll
          for (int q = 0; q < 7; ++q) sc.c[q] = cf[4 + q];
          v = snake_eval(__builtin_fmaf(v - cf[0], cf[1], cf[2]), sc);
        }
      }
      const _Float16 hi = (_Float16)v;
      const _Float16 lo = (_Float16)(v - (float)hi);
      yhi[j * CV_S + ci] = h_bits(hi);
      ylo[j * CV_S + ci] = h_bits(lo);
    }
    __syncthreads();

    for (int k = 0; k < a.K; ++k) {
      const uint16_t* wk[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) wk[m] = a.w + ((int64_t)co_l[m] * a.K + k) * a.C_in + c0 + 8 * hl;
      const int jb = wt * 64 + l32 + k * a.dilation;
      for (int g = 0; g < cc; g += 16) {
        nsr_h8 A[2], Bh[2], Bl[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) A[m] = co_ok[m] ? *(const nsr_h8*)(wk[m] + g) : hzero;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int off = (jb + n * 32) * CV_S + g + 8 * hl;
          Bh[n] = *(const nsr_h8*)(yhi + off);
          Bl[n] = *(const nsr_h8*)(ylo + off);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int n = 0; n < 2; ++n) {
            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m], Bh[n], acc[m][n], 0, 0, 0);
            acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[m], Bl[n], acc[m][n], 0, 0, 0);
          }
      }
    }
  }

  /* epilogue: lane holds rows 8(i/4) + 4 hl + i%4 of column l32 of each 32 x 32 tile */
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int t = t0 + wt * 64 + n * 32 + l32;
      if (t >= a.T_out) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int co = co0 + wco * 64 + m * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (co >= a.C_out) continue;
        const int64_t o = ((int64_t)b * a.C_out + co) * a.T_out + t;
        float v = acc[m][n][i];
        if (a.bias) v += f16_bits_to_f32(a.bias[co]);
        if (a.residual) v += a.residual[o];
        a.out[o] = v;
      }
    }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_conv1d_f16x2(const nsr_conv_args a) { conv_body<false>(a); }

extern "C" __global__ void __launch_bounds__(256) nsrk_conv1d_adain_snake_f16x2(const nsr_conv_args a) {
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
