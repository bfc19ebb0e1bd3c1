/*
 * Q8 GEMV at M = 1 (decoder projections), three forms
 * (kernels/moonshine_kernels.py):
 *   plain  out = x @ W (+ bias)                       gemv_q8 / gemv_q8_bias :616-677
 *   glu    out = silu(x @ Wg + bg) * (x @ Wx + bx)    gemv_q8_bias_glu :1721-1772
 *          (W [K, 2N]: x half in columns [0, N), gate half in [N, 2N))
 *   h      h = f16(x @ W) + residual (f32)            first half of gemv_q8_resadd_ln
 *          :1775-1819; the LayerNorm of h is a second launch (the row
 *          LayerNorm kernels), since it needs every column of h
 * over two weight layouts:
 *
 * - the reference's repacked Q8: qs u32 [K, NW/4] (the int8 weight of column
 *   c in byte c % 4 of word c / 4), scales f16 [K/32, NW]. A workgroup owns 8
 *   weight columns (plain, h) or 8 x-half + 8 gate-half columns (glu) over
 *   all of K; its 256 lanes take row pairs (2 rows of one 32-row block, so
 *   one scale per column) and are reduced through LDS in a fixed order. Each
 *   row contributes only 8 bytes per workgroup, so the 16 tiles of one
 *   128-byte line of qs words (128 columns) share every line they read, and
 *   they meet in an L2 only when they run on one XCD (workgroups are dealt
 *   round-robin to the 8 XCDs). Two tile maps:
 *   - line groups: XCD x takes the 16-tile groups x, x + 8, ..., so every
 *     line comes from HBM once (grid: 16 workgroups per group on each XCD,
 *     those past the last tile exit at once);
 *   - contiguous runs: XCD x takes the x-th run of ceil(n / 8) tiles, which
 *     balances the XCDs when the groups do not divide evenly, at the cost of
 *     reading the lines of a group split between two XCDs twice.
 *   The host takes line groups unless that leaves an XCD with more tiles
 *   than both the balanced share and its 32 CUs.
 *
 * - t4 tiles (nsr_q8_pack_t4): tile t holds 4 weight columns for all K rows
 *   contiguously, [K][4] int8, with its scales [K/32][4] f16. A workgroup
 *   reads its tile as consecutive 16-byte chunks (4 rows x 4 columns per
 *   lane), so every wave load is one contiguous 1 KB span: the weight
 *   stream runs at the coalesced-read rate. GLU tiles hold x-half columns
 *   2t, 2t+1 and gate-half columns 2t, 2t+1.
 *
 * No workgroup depends on another (no split-K, no scratch, no atomics);
 * every column's sum is formed in a fixed order, so results are
 * reproducible run to run.
 */
#include "device_common.h"

enum { GEMV_PLAIN = 0, GEMV_GLU = 1, GEMV_H = 2 };

/* Line groups: workgroup b, the (b / 8)-th on XCD b % 8, takes the next tile
 * of that XCD's groups x, x + 8, x + 16, ...; -1 past the last tile. */
NSR_DEV int line_group_tile(int b, int n) {
  const int x = b & 7, i = b >> 3;
  const int t = 16 * (x + 8 * (i >> 4)) + (i & 15);
  return t < n ? t : -1;
}

NSR_DEV float silu_f(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

NSR_DEV float s8(uint32_t w, int byte) { return (float)(int)(int8_t)(w >> (8 * byte)); }

/* ------------------------------------------------ reference layout -- */

template <int XDT, int ODT, int MODE>
NSR_DEV void gemv_ref(const nsr_gemv_args& a) {
  /* columns per workgroup: 8 (plain, h) or 8 x-half + 8 gate-half (glu) */
  constexpr int NC = MODE == GEMV_GLU ? 16 : 8;
  __shared__ float red[256][NC + 1];
  __shared__ float red2[256];
  __shared__ float fin[NC];
  const int tid = threadIdx.x;
  const int t = a.line_groups ? line_group_tile(blockIdx.x, a.n_tiles) : xcd_contiguous(blockIdx.x, a.n_tiles);
  if (t < 0) return; /* the whole workgroup: no barrier is reached */
  const int64_t nw4 = a.NW >> 2;
  /* first word (per row) of each 8-column group */
  const int64_t g0 = 2 * (int64_t)t;
  const int64_t g1 = (a.N >> 2) + 2 * (int64_t)t; /* gate half (glu only) */

  /* the epilogue's bias or residual for column tid < NC, loaded ahead of the weights (after the reduction it
   * would add one more memory latency to the chain) */
  const int64_t ecol = 4 * ((tid < 8) ? g0 : g1) + (tid & 7);
  float pre = 0.f;
  if (tid < NC) {
    if constexpr (MODE == GEMV_H) {
      pre = a.residual[ecol];
    } else {
      if (a.bias) pre = a.bias[ecol];
    }
  }
  float acc[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) acc[j] = 0.f;
  const int npairs = a.K >> 1;
  for (int p = tid; p < npairs; p += 256) {
    const int64_t r0 = 2 * (int64_t)p, b = p >> 4;
    const uint32_t* q0 = a.qs + r0 * nw4;
    const uint32_t* q1 = q0 + nw4;
    uint32_t w0[NC / 4], w1[NC / 4], sw[NC / 2];
#pragma unroll
    for (int h = 0; h < NC / 8; ++h) {
      const int64_t g = h ? g1 : g0;
      const nsr_uint2 a0 = *(const nsr_uint2*)(q0 + g), a1 = *(const nsr_uint2*)(q1 + g);
      w0[2 * h] = a0.x;
      w0[2 * h + 1] = a0.y;
      w1[2 * h] = a1.x;
      w1[2 * h + 1] = a1.y;
      const nsr_uint4 s4 = ld16_cached(a.scales + b * a.NW + 4 * g);
      sw[4 * h] = s4.x;
      sw[4 * h + 1] = s4.y;
      sw[4 * h + 2] = s4.z;
      sw[4 * h + 3] = s4.w;
    }
    const float x0 = load_scalar<XDT>(a.x, r0), x1 = load_scalar<XDT>(a.x, r0 + 1);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const float blk = __builtin_fmaf(x1, s8(w1[j >> 2], j & 3), x0 * s8(w0[j >> 2], j & 3));
      const float sc = f16_bits_to_f32((j & 1) ? (sw[j >> 1] >> 16) : (sw[j >> 1] & 0xffffu));
      acc[j] = __builtin_fmaf(blk, sc, acc[j]);
    }
  }
  /* fixed-order reduction over the 256 lanes: 256/NC strided groups, then NC partials each */
  constexpr int G = 256 / NC;
#pragma unroll
  for (int j = 0; j < NC; ++j) red[tid][j] = acc[j];
  __syncthreads();
  {
    const int col = tid % NC, g = tid / NC;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < NC; ++k) v += red[g + G * k][col];
    red2[tid] = v;
  }
  __syncthreads();
  if (tid < NC) {
    float v = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) v += red2[NC * g + tid];
    const int64_t col = ecol;
    if constexpr (MODE == GEMV_PLAIN) {
      store_scalar<ODT>(a.out, col, a.bias ? v + pre : v);
    } else if constexpr (MODE == GEMV_H) {
      a.out_f32[col] = round_to<DT_F16>(v) + pre;
    } else {
      fin[tid] = a.bias ? v + pre : v;
    }
  }
  if constexpr (MODE == GEMV_GLU) {
    __syncthreads();
    if (tid < 8) store_scalar<ODT>(a.out, 4 * g0 + tid, silu_f(fin[8 + tid]) * fin[tid]);
  }
}

/* ------------------------------------------------------- t4 tiles -- */

template <int XDT, int ODT, int MODE, int BLOCK>
NSR_DEV void gemv_t4(const nsr_gemv_args& a) {
  constexpr int NWV = BLOCK / 64;
  __shared__ float red[NWV][4];
  const int tid = threadIdx.x;
  const int t = blockIdx.x;
  const nsr_uint4* tile = (const nsr_uint4*)a.qs + (int64_t)t * (a.K >> 2);
  const nsr_uint2* tsc = (const nsr_uint2*)a.scales + (int64_t)t * (a.K >> 5);
  const int nchunk = a.K >> 2;
  /* the epilogue's bias or residual, loaded ahead of the tile: after the reduction it would add one more
   * memory latency to the chain */
  float pre0 = 0.f, pre1 = 0.f;
  if constexpr (MODE == GEMV_PLAIN) {
    if (tid < 4 && a.bias) pre0 = a.bias[4 * (int64_t)t + tid];
  } else if constexpr (MODE == GEMV_H) {
    if (tid < 4) pre0 = a.residual[4 * (int64_t)t + tid];
  } else {
    if (tid < 2 && a.bias) {
      pre0 = a.bias[2 * (int64_t)t + tid];
      pre1 = a.bias[a.N + 2 * (int64_t)t + tid];
    }
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = tid; j < nchunk; j += BLOCK) {
    const nsr_uint4 q = ld16(tile + j); /* rows 4j .. 4j+3, 4 columns each */
    const nsr_uint2 sw = tsc[j >> 3];
    float xs[4];
    if constexpr (XDT == DT_F16) {
      const nsr_uint2 xw = *((const nsr_uint2*)a.x + j);
      xs[0] = f16_bits_to_f32(xw.x & 0xffffu);
      xs[1] = f16_bits_to_f32(xw.x >> 16);
      xs[2] = f16_bits_to_f32(xw.y & 0xffffu);
      xs[3] = f16_bits_to_f32(xw.y >> 16);
    } else {
      const nsr_float4 xv = *((const nsr_float4*)a.x + j);
      xs[0] = xv.x;
      xs[1] = xv.y;
      xs[2] = xv.z;
      xs[3] = xv.w;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float blk = xs[0] * s8(q[0], c);
#pragma unroll
      for (int i = 1; i < 4; ++i) blk = __builtin_fmaf(xs[i], s8(q[i], c), blk);
      const float sc = f16_bits_to_f32((c & 1) ? (sw[c >> 1] >> 16) : (sw[c >> 1] & 0xffffu));
      acc[c] = __builtin_fmaf(blk, sc, acc[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float w = wave_sum(acc[c]);
    if ((tid & 63) == 0) red[tid >> 6][c] = w;
  }
  __syncthreads();
  if (tid < 4) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) v += red[w][tid];
    if constexpr (MODE == GEMV_PLAIN) {
      const int64_t col = 4 * (int64_t)t + tid;
      store_scalar<ODT>(a.out, col, a.bias ? v + pre0 : v);
    } else if constexpr (MODE == GEMV_H) {
      const int64_t col = 4 * (int64_t)t + tid;
      a.out_f32[col] = round_to<DT_F16>(v) + pre0;
    } else {
      red[0][tid] = v; /* every wave's partials were read above */
    }
  }
  if constexpr (MODE == GEMV_GLU) {
    __syncthreads();
    if (tid < 2) {
      const int64_t col = 2 * (int64_t)t + tid;
      const float xv = red[0][tid] + pre0; /* pre0, pre1 = 0 without a bias */
      const float gv = red[0][2 + tid] + pre1;
      store_scalar<ODT>(a.out, col, silu_f(gv) * xv);
    }
  }
}

/* t4 packing: one thread per (tile, row) word, then one per (tile, block)
 * scale quad. Source column of tile t, slot c: 4t + c (plain); 2t + c for
 * c < 2 and N + 2t + c - 2 otherwise (GLU). */
NSR_DEV int64_t t4_src_col(int64_t t, int c, int N) {
  if (N == 0) return 4 * t + c;
  return c < 2 ? 2 * t + c : (int64_t)N + 2 * t + (c - 2);
}

extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8t4_pack(const nsr_q8_pack_args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t tiles = a.NW >> 2;
  const int64_t nq = tiles * a.K;
  if (i < nq) {
    const int64_t t = i / a.K, r = i - t * a.K;
    const uint8_t* row = a.qs + r * a.NW;
    uint32_t w = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) w |= (uint32_t)row[t4_src_col(t, c, a.N)] << (8 * c);
    a.tq[i] = w;
  } else if (i < nq + tiles * (a.K >> 5)) {
    const int64_t k = i - nq, nb = a.K >> 5;
    const int64_t t = k / nb, b = k - t * nb;
#pragma unroll
    for (int c = 0; c < 4; ++c) a.ts[4 * k + c] = a.scales[b * a.NW + t4_src_col(t, c, a.N)];
  }
}

/* GGUF Q8_0 weight W [N, K] (N rows of K/32 34-byte blocks, the layout of
 * an nn::Linear [out, in] weight in the reference's GGUF files) -> the
 * GEMV layouts of W^T: a transpose of the int8 values and of the f16 block
 * scales, no arithmetic. One thread per output word (k fastest, so the
 * reads of a weight row are consecutive); the first four threads of each
 * 32-row block also move that block's four scales (one each), whose bytes
 * sit in the lines their wave reads anyway (a separate pass over the scales
 * read every line of the weight a second time). The workgroups of a quad's
 * rows share lines at their edges and run on one XCD (xcd_contiguous). */
extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8_from_q8_0(const nsr_q8_0_conv_args a) {
  const int64_t i = (int64_t)xcd_contiguous((int)blockIdx.x, (int)gridDim.x) * 256 + threadIdx.x;
  const int64_t K = a.K, nb = K >> 5, quads = (int64_t)a.N >> 2;
  const int64_t nw = quads * K;
  const int64_t rowb = nb * 34; /* bytes per weight row */
  if (i >= nw) return;
  const int64_t q = i / K, k = i - q * K; /* column quad q, row k of W^T */
  const int64_t b = k >> 5;
  uint32_t w = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t n = a.t4 ? t4_src_col(q, c, a.glu_n) : 4 * q + c;
    w |= (uint32_t)a.blocks[n * rowb + b * 34 + 2 + (k & 31)] << (8 * c);
  }
  if (a.t4)
    a.qs[i] = w;
  else
    a.qs[k * quads + q] = w;
  if ((k & 31) < 4) {
    const int c = (int)(k & 31);
    const int64_t j = q * nb + b;
    const int64_t n = a.t4 ? t4_src_col(q, c, a.glu_n) : 4 * q + c;
    const uint16_t d = *(const uint16_t*)(a.blocks + n * rowb + b * 34);
    if (a.t4)
      a.scales[4 * j + c] = d;
    else
      a.scales[b * a.N + n] = d;
  }
}

#define NSR_GEMV_REF(XN, XDT, ON, ODT)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8_##XN##_##ON(const nsr_gemv_args a) {   \
    gemv_ref<XDT, ODT, GEMV_PLAIN>(a);                                                                  \
  }                                                                                                     \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8_glu_##XN##_##ON(const nsr_gemv_args a) { \
    gemv_ref<XDT, ODT, GEMV_GLU>(a);                                                                    \
  }

#define NSR_GEMV_T4(XN, XDT, ON, ODT, B)                                                   \
  extern "C" __global__ void __launch_bounds__(B)                                          \
      nsrk_gemv_q8t4_##XN##_##ON##_b##B(const nsr_gemv_args a) {                           \
    gemv_t4<XDT, ODT, GEMV_PLAIN, B>(a);                                                   \
  }                                                                                        \
  extern "C" __global__ void __launch_bounds__(B)                                          \
      nsrk_gemv_q8t4_glu_##XN##_##ON##_b##B(const nsr_gemv_args a) {                       \
    gemv_t4<XDT, ODT, GEMV_GLU, B>(a);                                                     \
  }

#define NSR_GEMV_ALL(XN, XDT, ON, ODT) \
  NSR_GEMV_REF(XN, XDT, ON, ODT)       \
  NSR_GEMV_T4(XN, XDT, ON, ODT, 256)   \
  NSR_GEMV_T4(XN, XDT, ON, ODT, 512)   \
  NSR_GEMV_T4(XN, XDT, ON, ODT, 1024)

NSR_GEMV_ALL(f16, DT_F16, f16, DT_F16)
NSR_GEMV_ALL(f16, DT_F16, f32, DT_F32)
NSR_GEMV_ALL(f32, DT_F32, f16, DT_F16)
NSR_GEMV_ALL(f32, DT_F32, f32, DT_F32)

#define NSR_GEMV_H(XN, XDT)                                                                       \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8_h_##XN(const nsr_gemv_args a) {   \
    gemv_ref<XDT, DT_F32, GEMV_H>(a);                                                             \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(256) nsrk_gemv_q8t4_h_##XN##_b256(const nsr_gemv_args a) { \
    gemv_t4<XDT, DT_F32, GEMV_H, 256>(a);                                                         \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(512) nsrk_gemv_q8t4_h_##XN##_b512(const nsr_gemv_args a) { \
    gemv_t4<XDT, DT_F32, GEMV_H, 512>(a);                                                         \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(1024) nsrk_gemv_q8t4_h_##XN##_b1024(const nsr_gemv_args a) { \
    gemv_t4<XDT, DT_F32, GEMV_H, 1024>(a);                                                        \
  }

NSR_GEMV_H(f16, DT_F16)
NSR_GEMV_H(f32, DT_F32)
