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
