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
 * sin / cos each). Here each frame's spectrum is computed once, then its
 * n_fft windowed samples, into LDS; then each output sample sums its frames
 * (in frame order) and divides by the window sum. A workgroup owns a run of
 * 64 frames and the samples that only those frames reach; neighbouring
 * workgroups recompute n_fft / hop - 1 boundary frames.
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

/* sin(x): Cody-Waite reduction x = j pi/2 + r (pi/2 split in three f32
 * parts, j = rint(2x/pi), exact products by FMA), then Taylor polynomials of
 * sin and cos on |r| <= pi/4 (to r^9 and r^10; first dropped terms below
 * 2e-9 and 1.2e-10) and the quadrant j mod 4. Accurate to a few f32 ulps for
 * |x| <= 65536; larger arguments take the library sinf. */
NSR_DEV float sin_cw(float x) {
  const float j = __builtin_rintf(x * 0.636619772367581343f);
  float r = fmaf(j, -1.57079637050628662109375f, x);
  r = fmaf(j, 4.37113882867379289e-08f, r);
  r = fmaf(j, 1.71512451e-15f, r);
  const float r2 = r * r;
  float ps = 1.0f / 362880.0f;
  ps = fmaf(ps, r2, -1.0f / 5040.0f);
  ps = fmaf(ps, r2, 1.0f / 120.0f);
  ps = fmaf(ps, r2, -1.0f / 6.0f);
  const float sn = fmaf(r * r2, ps, r);
  float pc = -1.0f / 3628800.0f;
  pc = fmaf(pc, r2, 1.0f / 40320.0f);
  pc = fmaf(pc, r2, -1.0f / 720.0f);
  pc = fmaf(pc, r2, 1.0f / 24.0f);
  pc = fmaf(pc, r2, -0.5f);
  const float cs = fmaf(r2, pc, 1.0f);
  const int q = (int)j & 3;
  float v = (q & 1) ? cs : sn;
  v = (q & 2) ? -v : v;
  return __builtin_fabsf(x) <= 65536.0f ? v : sinf(x);
}

/* N = n_fft at compile time. A workgroup of 256 lanes owns NSR_ISTFT_FG
 * frames and works in three phases, each spread over all lanes so that
 * every lane carries a few items (and many waves hide each other's latency):
 *  A. spectrum: item (bin k, frame) -> re, im into LDS [k][frame];
 *  B. iDFT: item (sample pair n / N - n, frame) -> windowed samples into LDS
 *     [frame][n] (row stride N + 1: conflict-free column writes);
 *  C. overlap-add: item (output sample) -> sum of its frames / window sum. */
#define NSR_ISTFT_FG 64
template <int N>
NSR_DEV void istft_body(const nsr_istft_args& a) {
  constexpr int bins = N / 2 + 1, H = N / 2, FG = NSR_ISTFT_FG, NS = N + 1;
  constexpr int IA = (bins * FG + 255) / 256;    /* phase A items per lane */
  constexpr int IB = ((H + 1) * FG + 255) / 256; /* phase B items per lane */
  __shared__ float cosm[N], sinm[N]; /* cos / sin(2 pi m / N), m = 0 .. N - 1 */
  __shared__ float win[N], winn[N]; /* the window, and the window / N (the iDFT's scale folded in) */
  __shared__ float sre[bins * FG], sim[bins * FG]; /* [k][frame] */
  __shared__ float frames[FG * NS];                /* [frame][n], windowed */
  const int tid = threadIdx.x;
  const int hop = a.hop, R = N / hop, trim = N / 2;
  const float PI = 3.14159265358979323846f;

  /* groups of 64 frames overlap by R - 1 and do not start on a cache line: neighbouring groups run on one XCD
   * (xcd_contiguous), so the lines they share come from HBM once */
  const int grp = xcd_contiguous((int)blockIdx.x, (int)gridDim.x);
  const int step = FG - (R - 1);
  const int64_t F0 = (int64_t)grp * step;
  const int nloc = (int)min((int64_t)FG, a.n_frames - F0); /* frames of this group */

  /* phase A loads first (one memory latency for all), then the tables */
  /* 32-bit element offsets (the host keeps 2 bins n_frames below 2^31) */
  const int nfr = (int)a.n_frames, f0 = (int)F0;
  float lm[IA], rp[IA];
#pragma unroll
  for (int it = 0; it < IA; ++it) {
    const int i = tid + 256 * it;
    const int k = i / FG, fl = i % FG;
    const bool ok = i < bins * FG && fl < nloc;
    const int off = (ok ? k : 0) * nfr + f0 + (ok ? fl : 0);
    lm[it] = a.x[off];
    rp[it] = a.x[off + bins * nfr];
  }
  /* the iDFT basis cos / sin(2 pi k n / N) takes N values, at m = k n mod N;
   * the periodic Hann window is the reference's f32 formula (decoder.rs:
   * 1558-1560), 0.5 - 0.5 cos(2 pi n / N), from the same cosines */
  if (tid < N) {
    const float ang = 2.0f * PI * (float)tid / (float)N;
    const float c = cosf(ang);
    cosm[tid] = c;
    sinm[tid] = sinf(ang);
    win[tid] = 0.5f - 0.5f * c;
    winn[tid] = (0.5f - 0.5f * c) / (float)N;
  }
#pragma unroll
  for (int it = 0; it < IA; ++it) {
    const int i = tid + 256 * it;
    if (i < bins * FG) {
      const int k = i / FG;
      const float e = expf(lm[it]);
      const float m = (k == 0 || k == bins - 1) ? e : 2.0f * e; /* one-sided: inner bins twice */
      float sn, cs;
      sincos_unit(sin_cw(rp[it]), sn, cs);
      sre[i] = m * cs;
      sim[i] = m * sn;
    }
  }
  __syncthreads();

#pragma unroll
  for (int it = 0; it < IB; ++it) {
    const int i = tid + 256 * it;
    const int n = __builtin_amdgcn_readfirstlane(i / FG), fl = i % FG; /* n: uniform over a wave (FG = 64) */
    if (i < (H + 1) * FG && fl < nloc) {
      float c = 0.f, sm = 0.f;
#pragma unroll
      for (int k = 0; k < bins; ++k) {
        const int m = (k * n) % N; /* wave-uniform */
        c = fmaf(sre[k * FG + fl], cosm[m], c);
        sm = fmaf(sim[k * FG + fl], sinm[m], sm);
      }
      /* (c -/+ sm) / N * w[n] as one multiply by w[n] / N (no division per item) */
      frames[fl * NS + n] = (c - sm) * winn[n];
      if (n > 0 && n < H) frames[fl * NS + (N - n)] = (c + sm) * winn[N - n];
    }
  }
  __syncthreads();

  /* owned untrimmed positions base + [q_lo, q_hi), base = F0 * hop (the first
   * sample of frame F0); frame F0 + g covers q in [g hop, g hop + N); the
   * first and last groups also own the positions the signal's edges leave */
  const int64_t base = F0 * hop;
  const float inv_hop = 1.0f / (float)hop;
  const int q_lo = grp == 0 ? 0 : (R - 1) * hop;
  const int q_hi = F0 + FG >= a.n_frames ? (nloc - 1) * hop + N : FG * hop;
  for (int q = q_lo + tid; q < q_hi; q += 256) {
    const int64_t i = base + q - trim; /* output index */
    if (i < 0 || i >= a.out_len) continue;
    /* q / hop by a float reciprocal, exact after one correction (q < 2^16) */
    int qd = (int)((float)q * inv_hop);
    qd += (qd + 1) * hop <= q ? 1 : 0;
    qd -= qd * hop > q ? 1 : 0;
    const int g_last = min(qd, nloc - 1);
    const int g_first = max(0, qd - (R - 1)); /* frames qd - R + 1 .. qd cover q */
    float acc = 0.f, ws = 0.f;
    for (int g = g_first; g <= g_last; ++g) {
      const int n = q - g * hop;
      acc += frames[g * NS + n];
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
