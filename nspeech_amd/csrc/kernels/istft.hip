/*
 * Inverse STFT of the Kokoro generator's conv_post output.
 *
 * Reference semantics: istft_fused (kernels/kokoro_kernels.py:1097-1183,
 * KokoroGpuBackend::istft_gpu src/kokoro/gpu_backend.rs:220-225, Metal impl
 * src/kokoro/gpu_decoder.rs:1062-1075) and the CPU path it replaces
 * (src/kokoro/decoder.rs:606-612 and istft :1546-1632): x [2 bins, n_frames]
 * f32 (bins = n_fft / 2 + 1) holds log-magnitudes then raw phases;
 *   mag_k = exp(x[k]), ph_k = sin(x[bins + k]),
 *   frame_f[n] = (1 / n_fft) sum_k s_k mag_k (cos(ph_k) cos(2 pi k n / n_fft)
 *                                           - sin(ph_k) sin(2 pi k n / n_fft)),
 *   s_k = 1 for the DC and Nyquist bins, 2 otherwise;
 *   y[p] = sum_f w[p - f hop] frame_f[p - f hop] / sum_f w[p - f hop]^2
 *   (periodic Hann w, frames in order; 0 where the window sum <= 1e-8),
 * returned without the n_fft / 2 samples of centre padding on each side:
 * out[i] = y[i + n_fft / 2], out_len = (n_frames - 1) hop.
 *
 * Design (gfx950): the reference evaluates, for every output sample, the
 * spectrum of each frame that overlaps it (n_fft / hop frames x bins exp /
 * sin / cos each). Here one lane computes one frame: its bins' magnitude and
 * phase once, then the n_fft windowed samples, into LDS; then each output
 * sample sums its frames (in frame order) and divides by the window sum. A
 * workgroup owns a run of frames and the samples that only those frames
 * reach; neighbouring workgroups recompute n_fft / hop - 1 boundary frames.
 * The frame phase bounds the kernel (VALU, not HBM), so it is cut down:
 *  - cos / sin of the phase, whose argument sin(raw) lies in [-1, 1], are
 *    Taylor polynomials to degree 14 / 13 (truncation below 1.2e-11, i.e.
 *    rounding-limited in f32) instead of range-reduced library calls;
 *  - the factor 2 of the inner bins is folded into re / im (exact);
 *  - the real iDFT is evaluated through its symmetry: with
 *    C_n = sum_k re_k cos(2 pi k n / N) and S_n = sum_k im_k sin(...),
 *    sample n is C_n - S_n and sample N - n is C_n + S_n, so only
 *    n = 0 .. N / 2 are summed. The basis uses the angle of (k n mod N),
 *    exact to f32 rounding; the reference's f32 angles of up to 2 pi k n / N
 *    (about 60 rad) carry up to ~2e-6 of angle rounding, well inside the
 *    1e-5 f32 parity bar.
 */
#include "device_common.h"

/* cos and sin of |x| <= 1 by Horner on the Taylor series (terms to x^14 and
 * x^13; the first dropped terms are below 1.2e-11 and 7.7e-13). */
NSR_DEV void sincos_unit(float x, float& s, float& c) {
  const float x2 = x * x;
  float ps = -1.0f / 6227020800.0f;                /* -1/13! */
  ps = fmaf(ps, x2, 1.0f / 39916800.0f);           /* 1/11! */
  ps = fmaf(ps, x2, -1.0f / 362880.0f);            /* -1/9! */
  ps = fmaf(ps, x2, 1.0f / 5040.0f);               /* 1/7! */
  ps = fmaf(ps, x2, -1.0f / 120.0f);               /* -1/5! */
  ps = fmaf(ps, x2, 1.0f / 6.0f);                  /* 1/3! */
  s = fmaf(-x * x2, ps, x);                        /* x - x^3 (1/3! - ...) */
  float pc = 1.0f / 87178291200.0f;                /* 1/14! */
  pc = fmaf(pc, x2, -1.0f / 479001600.0f);         /* -1/12! */
  pc = fmaf(pc, x2, 1.0f / 3628800.0f);            /* 1/10! */
  pc = fmaf(pc, x2, -1.0f / 40320.0f);             /* -1/8! */
  pc = fmaf(pc, x2, 1.0f / 720.0f);                /* 1/6! */
  pc = fmaf(pc, x2, -1.0f / 24.0f);                /* -1/4! */
  pc = fmaf(pc, x2, 0.5f);                         /* 1/2! */
  c = fmaf(-x2, pc, 1.0f);                         /* 1 - x^2 (1/2! - ...) */
}

/* N = n_fft at compile time (the bins' spectra stay in registers) */
template <int N>
NSR_DEV void istft_body(const nsr_istft_args& a) {
  constexpr int bins = N / 2 + 1, H = N / 2;
  __shared__ float cosb[(H + 1) * bins]; /* [n = 0 .. N / 2][k] */
  __shared__ float sinb[(H + 1) * bins];
  __shared__ float win[N];
  extern __shared__ float frames[]; /* [frames_per_group][n_fft] windowed frame samples */
  const int tid = threadIdx.x;
  const int hop = a.hop, R = N / hop, trim = N / 2;
  const float PI = 3.14159265358979323846f;
  for (int i = tid; i < (H + 1) * bins; i += 256) {
    const int n = i / bins, k = i - n * bins;
    const float ang = 2.0f * PI * (float)((k * n) % N) / (float)N;
    cosb[i] = cosf(ang);
    sinb[i] = sinf(ang);
  }
  /* periodic Hann, the reference's f32 formula (decoder.rs:1558-1560) */
  for (int n = tid; n < N; n += 256) win[n] = 0.5f - 0.5f * cosf(2.0f * PI * (float)n / (float)N);
  __syncthreads();

  /* frames [F0, F0 + FG) computed here; the samples owned are the untrimmed
   * positions all of whose frames lie in that range (the first and last
   * groups also own the positions the edges of the signal leave) */
  const int FG = a.frames_per_group, step = FG - (R - 1);
  const int64_t F0 = (int64_t)blockIdx.x * step;
  const int nloc = (int)min((int64_t)FG, a.n_frames - F0); /* frames of this group */
  if (tid < nloc) {
    const int64_t f = F0 + tid;
    /* all 2 bins loads first, so that one memory latency covers them */
    float lm[bins], rp[bins];
#pragma unroll
    for (int k = 0; k < bins; ++k) {
      lm[k] = a.x[(int64_t)k * a.n_frames + f];
      rp[k] = a.x[(int64_t)(bins + k) * a.n_frames + f];
    }
    float re[bins], im[bins];
#pragma unroll
    for (int k = 0; k < bins; ++k) {
      const float m = (k == 0 || k == bins - 1) ? expf(lm[k]) : 2.0f * expf(lm[k]);
      float sn, cs;
      sincos_unit(sinf(rp[k]), sn, cs);
      re[k] = m * cs;
      im[k] = m * sn;
    }
#pragma unroll
    for (int n = 0; n <= H; ++n) {
      float c = 0.f, sm = 0.f;
#pragma unroll
      for (int k = 0; k < bins; ++k) {
        c = fmaf(re[k], cosb[n * bins + k], c);
        sm = fmaf(im[k], sinb[n * bins + k], sm);
      }
      frames[tid * N + n] = ((c - sm) / (float)N) * win[n];
      if (n > 0 && n < H) frames[tid * N + (N - n)] = ((c + sm) / (float)N) * win[N - n];
    }
  }
  __syncthreads();

  /* owned untrimmed positions base + [q_lo, q_hi), base = F0 * hop (the first
   * sample of frame F0); frame F0 + g covers q in [g hop, g hop + N) */
  const int64_t base = F0 * hop;
  const int q_lo = blockIdx.x == 0 ? 0 : (R - 1) * hop;
  const int q_hi = F0 + FG >= a.n_frames ? (nloc - 1) * hop + N : FG * hop;
  for (int q = q_lo + tid; q < q_hi; q += 256) {
    const int64_t i = base + q - trim; /* output index */
    if (i < 0 || i >= a.out_len) continue;
    const int g_first = q - N + 1 <= 0 ? 0 : (q - N + hop) / hop; /* ceil((q - N + 1) / hop) */
    const int g_last = min(q / hop, nloc - 1);
    float acc = 0.f, ws = 0.f;
    for (int g = g_first; g <= g_last; ++g) {
      const int n = q - g * hop;
      acc += frames[g * N + n];
      ws += win[n] * win[n];
    }
    a.out[i] = ws > 1e-8f ? acc / ws : 0.f;
  }
}

#define NSR_ISTFT(N)                                                                             \
  extern "C" __global__ void __launch_bounds__(256) nsrk_istft_f32_n##N(const nsr_istft_args a) { \
    istft_body<N>(a);                                                                           \
  }

NSR_ISTFT(16)
NSR_ISTFT(20)
NSR_ISTFT(32)
