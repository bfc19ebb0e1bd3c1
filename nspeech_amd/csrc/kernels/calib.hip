/*
 * Measurement floors for the benchmark (no counterpart in the reference).
 *
 * An empty kernel (the cost of one launch on a stream) and a plain device
 * copy of n4 16-byte chunks in two grid forms, so that every fused kernel can
 * be judged against a copy that moves the same bytes:
 *   flat:        one 16-byte chunk per lane, ceil(n4 / 256) workgroups;
 *   persistent:  a fixed grid (the host passes #CU x k workgroups), each lane
 *                keeps U chunks in flight (U loads, then U stores) and the
 *                workgroups walk 256 U-chunk tiles with the grid as stride.
 * Loads and stores are 128-bit and non-temporal, like the fused kernels'.
 * A third form copies row by row the way the AdaIN row kernel reads and
 * writes: one 512-lane workgroup per row of row_bytes, a persistent grid of
 * one workgroup per CU, 8 slots of 16 bytes per lane in flight. It is the
 * floor of that access structure (a few hundred concurrent row streams),
 * which the flat copy does not share.
 */
#include "device_common.h"

extern "C" __global__ void __launch_bounds__(256) nsrk_calib_empty(const nsr_calib_args a) {}

extern "C" __global__ void __launch_bounds__(256) nsrk_calib_copy_flat(const nsr_calib_args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < a.n4) st16(a.dst + 4 * i, ld16(a.src + 4 * i));
}

template <int U>
NSR_DEV void copy_persistent(const nsr_calib_args& a) {
  const int64_t tile = 256 * U;
  const int64_t ntiles = (a.n4 + tile - 1) / tile;
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const int64_t base = t * tile + threadIdx.x;
    nsr_uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + 256 * u;
      v[u] = i < a.n4 ? ld16(a.src + 4 * i) : nsr_uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + 256 * u;
      if (i < a.n4) st16(a.dst + 4 * i, v[u]);
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) nsrk_calib_copy_p4(const nsr_calib_args a) {
  copy_persistent<4>(a);
}
extern "C" __global__ void __launch_bounds__(256) nsrk_calib_copy_p8(const nsr_calib_args a) {
  copy_persistent<8>(a);
}

/* rows: n4 = row_bytes / 16 chunks per row (a.n4), n_rows rows (gridDim-strided) */
extern "C" __global__ void __launch_bounds__(512) nsrk_calib_copy_rows(const nsr_calib_args a, const int64_t n_rows) {
  const int64_t nch = a.n4;
  const uint32_t rbytes = (uint32_t)(nch * 16);
  const uint32_t voff = threadIdx.x * 16u;
  const int ns = (int)((nch + 511) / 512);
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const nsr_rsrc xr = make_rsrc(a.src + row * nch * 4, rbytes);
    const nsr_rsrc orr = make_rsrc(a.dst + row * nch * 4, rbytes);
    for (int k0 = 0; k0 < ns; k0 += 8) {
      nsr_float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = buf_load4(xr, voff, (uint32_t)(k0 + u) * 8192u);
#pragma unroll
      for (int u = 0; u < 8; ++u) buf_store4(orr, voff, (uint32_t)(k0 + u) * 8192u, v[u]);
    }
  }
}
