/*
 * Q8 GEMV at M = 1 (decoder projections) over the repacked Q8 layout:
 * qs u32 [K, NW/4] (the int8 weight of column c in byte c % 4 of word c / 4),
 * scales f16 [K/32, NW]. Forms (kernels/moonshine_kernels.py):
 *   mode 0  out = x @ W (+ bias)                       gemv_q8 / gemv_q8_bias :616-677
 *   mode 1  out = silu(x @ Wg + bg) * (x @ Wx + bx)    gemv_q8_bias_glu :1721-1772
 *           (W [K, 2N]: x half in columns [0, N), gate half in [N, 2N))
 *   mode 2  h = f16(x @ W) + residual (written f32), out = LN(h) * w
 *                                                      gemv_q8_resadd_ln :1775-1819
 *
 * Design (gfx950, memory-bound on the weights): split-K over a 2-D grid so
 * that even a 640 x 2560 projection spreads over ~200-400 workgroups. A
 * workgroup (256 threads = 16 column lanes x 16 row lanes) covers a tile of
 * 256 weight columns (16 per lane, one 16-byte word of qs per row) and a
 * chunk of K. Per 32-row Q8 block a lane reads its 16 scales and 2 rows
 * and applies the scale once to the two-row sum. The 16 row lanes are
 * reduced through LDS in a fixed order. With one K chunk the epilogue follows directly; otherwise
 * each workgroup stores its f32 partial sums, and the last workgroup of a
 * tile to finish (a device-scope atomic count; no workgroup ever waits on
 * another) adds the partials in chunk order, applies the epilogue and resets
 * the count for the next call. Results do not depend on arrival order.
 */
#include "device_common.h"

enum { GEMV_PLAIN = 0, GEMV_GLU = 1, GEMV_RESLN = 2 };

template <int XDT>
NSR_DEV float gemv_x(const void* x, int64_t k) {
  return load_scalar<XDT>(x, k);
}

/* One 32-row block for this lane's 16 columns: rows 2*kl and 2*kl + 1 of
 * the block, summed in f32, times the block scale, added to acc. */
template <int XDT>
NSR_DEV void gemv_block(const nsr_gemv_args& a, int64_t b, int kl, int64_t w0, float* acc) {
  const int64_t r0 = b * 32 + 2 * kl;
  const int64_t nw4 = a.NW >> 2;
  const nsr_uint4 q0 = ld16(a.qs + r0 * nw4 + w0);
  const nsr_uint4 q1 = ld16(a.qs + (r0 + 1) * nw4 + w0);
  const nsr_uint4 s01 = ld16_cached(a.scales + b * a.NW + 4 * w0);
  const nsr_uint4 s23 = ld16_cached(a.scales + b * a.NW + 4 * w0 + 8);
  const float x0 = gemv_x<XDT>(a.x, r0), x1 = gemv_x<XDT>(a.x, r0 + 1);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    /* signed byte j % 4 of word j / 4 -> f32: one v_cvt_f32_i32 with a
     * sign-extended byte select. (Written as an int8_t cast: the same value
     * through __builtin_amdgcn_sbfe is folded by this compiler into an
     * unsigned convert of the sign-extended byte, wrong for negatives.) */
    const int sh = 8 * (j & 3);
    const float v0 = (float)(int)(int8_t)(q0[j >> 2] >> sh);
    const float v1 = (float)(int)(int8_t)(q1[j >> 2] >> sh);
    const float blk = __builtin_fmaf(x1, v1, x0 * v0);
    const uint32_t sw = j < 8 ? s01[j >> 1] : s23[(j - 8) >> 1];
    const float sc = f16_bits_to_f32((j & 1) ? (sw >> 16) : (sw & 0xffffu));
    acc[j] = __builtin_fmaf(blk, sc, acc[j]);
  }
}

/* Device-scope "am I the last of `total` arrivals on counter c": every
 * thread's prior global writes are released before the count, and the last
 * arrival acquires all of them. The last arrival resets the counter. */
NSR_DEV bool gemv_arrive_last(uint32_t* c, uint32_t total, uint32_t* flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(c, 1u);
    *flag = prev == total - 1u ? 1u : 0u;
    if (prev == total - 1u) atomicExch(c, 0u);
  }
  __syncthreads();
  const bool last = *flag != 0u;
  if (last) __threadfence();
  return last;
}

template <int XDT, int ODT, int MODE>
NSR_DEV void gemv_q8_body(const nsr_gemv_args& a) {
  __shared__ float red[16][257];
  __shared__ float fin[256];
  __shared__ float redl[8];
  __shared__ uint32_t flag;
  const int tid = threadIdx.x;
  const int cl = tid & 15, kl = tid >> 4;
  const int t = blockIdx.x, s = blockIdx.y;

  /* this lane's first weight column; GLU tiles pair 128 x-half columns with
   * the matching 128 gate-half columns */
  int64_t c0;
  bool cvalid;
  if constexpr (MODE == GEMV_GLU) {
    const int64_t oc = (int64_t)t * 128 + 16 * (cl & 7);
    c0 = oc + (cl >= 8 ? a.N : 0);
    cvalid = oc < a.N;
  } else {
    c0 = (int64_t)t * 256 + 16 * cl;
    cvalid = c0 < a.NW;
  }

  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  if (cvalid) {
    const int64_t bpc = a.kc >> 5;
    const int64_t b0 = (int64_t)s * bpc;
    const int64_t b1 = min(b0 + bpc, (int64_t)(a.K >> 5));
    for (int64_t b = b0; b < b1; ++b) gemv_block<XDT>(a, b, kl, c0 >> 2, acc);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) red[kl][16 * cl + j] = acc[j];
  __syncthreads();
  /* thread tid owns tile column tid: the 16 row lanes summed in order */
  float v = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) v += red[r][tid];

  int64_t col; /* weight column of tile column tid */
  bool valid;
  if constexpr (MODE == GEMV_GLU) {
    const int64_t oc = (int64_t)t * 128 + (tid & 127);
    col = oc + (tid >= 128 ? a.N : 0);
    valid = oc < a.N;
  } else {
    col = (int64_t)t * 256 + tid;
    valid = col < a.NW;
  }

  if (a.S > 1) {
    /* split K: the last chunk of this tile to arrive adds all chunks' partial
     * sums in chunk order */
    if (valid) a.partial[(int64_t)s * a.NW + col] = v;
    if (!gemv_arrive_last(a.counters + t, (uint32_t)a.S, &flag)) return;
    if (valid) {
      v = 0.f;
      for (int i = 0; i < a.S; ++i) v += a.partial[(int64_t)i * a.NW + col];
    }
  }

  if constexpr (MODE == GEMV_PLAIN) {
    if (valid) store_scalar<ODT>(a.out, col, a.bias ? v + a.bias[col] : v);
  } else if constexpr (MODE == GEMV_GLU) {
    fin[tid] = valid ? (a.bias ? v + a.bias[col] : v) : 0.f;
    __syncthreads();
    if (tid < 128 && valid) {
      const float g = fin[tid + 128];
      const float sg = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
      store_scalar<ODT>(a.out, col, sg * fin[tid]);
    }
  } else {
    /* h = f16(projection) + residual for this tile's columns; the last tile
     * to finish normalises all N columns */
    if (valid) a.out_f32[col] = round_to<DT_F16>(v) + a.residual[col];
    if (gridDim.x > 1) {
      if (!gemv_arrive_last(a.counters + gridDim.x, gridDim.x, &flag)) return;
    } else {
      __syncthreads();
    }
    float sum = 0.f;
    for (int64_t c = tid; c < a.N; c += 256) sum += a.out_f32[c];
    const float mean = block_sum<4>(sum, redl) / (float)a.N;
    float sq = 0.f;
    for (int64_t c = tid; c < a.N; c += 256) {
      const float d = a.out_f32[c] - mean;
      sq = __builtin_fmaf(d, d, sq);
    }
    const float var = block_sum<4>(sq, redl) / (float)a.N;
    const float rstd = 1.0f / sqrtf(var + a.eps);
    for (int64_t c = tid; c < a.N; c += 256) {
      const float w = a.ln_w_f16 ? f16_bits_to_f32(((const uint16_t*)a.ln_w)[c]) : ((const float*)a.ln_w)[c];
      store_scalar<ODT>(a.out, c, (a.out_f32[c] - mean) * rstd * w);
    }
  }
}

#define NSR_GEMV(XN, XDT, ON, ODT)                                                              \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8_##XN##_##ON(const nsr_gemv_args a) { \
    gemv_q8_body<XDT, ODT, GEMV_PLAIN>(a);                                                     \
  }                                                                                             \
  extern "C" __global__ void __launch_bounds__(256)                                             \
      nsrk_gemv_q8_glu_##XN##_##ON(const nsr_gemv_args a) {                                     \
    gemv_q8_body<XDT, ODT, GEMV_GLU>(a);                                                       \
  }                                                                                             \
  extern "C" __global__ void __launch_bounds__(256)                                             \
      nsrk_gemv_q8_resln_##XN##_##ON(const nsr_gemv_args a) {                                   \
    gemv_q8_body<XDT, ODT, GEMV_RESLN>(a);                                                     \
  }

NSR_GEMV(f16, DT_F16, f16, DT_F16)
NSR_GEMV(f16, DT_F16, f32, DT_F32)
NSR_GEMV(f32, DT_F32, f16, DT_F16)
NSR_GEMV(f32, DT_F32, f32, DT_F32)
