/*
 * GGUF Q8_0 embedding gather with the dequantisation fused into the gather.
 *
 * Reference semantics: QEmbedding::forward (src/parakeet/quantized_layers.rs:65-71)
 * dequantises the WHOLE table (QTensor::dequantize) and then index_selects
 * rows; a GGUF Q8_0 block is {f16 d; int8 qs[32]} and element j of block b is
 * qs[j] * d. Here only the gathered rows are read: per output float4 one lane
 * reads the block scale and 4 quant bytes, so HBM traffic is n_ids * row_bytes
 * in and n_ids * d * 4 out. int8 * f16 has at most 8 + 11 significant bits,
 * so every product is exact in f32 and the result is bit-identical to the
 * reference's dequantize-then-select, in any evaluation order.
 *
 * Rows are 34*d/32 bytes, so a row start is only 2-byte aligned: each lane
 * reads the block's f16 scale (16 bits) and its 4 quant bytes as one 32-bit
 * load at a 2-byte aligned address (gfx950 global loads take unaligned
 * addresses). Measured on MI355X at config 3: 3.21 us against 3.37 us for
 * two 16-bit loads; a variant that copies each row's 16-byte aligned window
 * to LDS with 128-bit loads and dequantises from LDS took 3.99 us (the LDS
 * round trip and barrier lengthen the id -> row -> output chain that bounds
 * an 8.6 MB gather), and two float4 per lane 3.59 us.
 */
#include "device_common.h"

template <int ACT, bool IDS_I64>
NSR_DEV void q8_0_gather_body(const nsr_q8_args& a) {
  const uint32_t d4 = (uint32_t)a.d4;
  uint32_t f, row, c4; /* float4 index, its id's position, its float4 within the row */
  int64_t id;
  if (a.gw > 0) {
    /* whole waves per id: the id is wave-uniform, read once per wave through the scalar cache (a
     * constant-address-space load at a uniform address) instead of by every lane */
    const uint32_t gw = (uint32_t)a.gw, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    /* wave / gw for wave < 4 and gw <= 4 as a multiply and shift (exact there), not a division ahead of
     * the id load: 256 / gw rounded up */
    const uint32_t wq = (wave * (gw == 3u ? 86u : 256u >> (gw >> 1))) >> 8;
    row = blockIdx.x * (uint32_t)a.ipw + wq;
    if (row >= (uint32_t)a.n_ids) return;
    c4 = (wave - wq * gw) * 64u + (threadIdx.x & 63u);
    if (c4 >= d4) return;
    f = row * d4 + c4;
    if constexpr (IDS_I64) {
      id = ((const __attribute__((address_space(4))) int64_t*)a.ids)[row];
    } else {
      id = (int64_t)((const __attribute__((address_space(4))) uint32_t*)a.ids)[row];
    }
  } else if (a.ipw > 0) {
    /* whole ids per workgroup: no table row is split between two workgroups (which may sit on two
     * XCDs and each fetch the row's shared lines) */
    const uint32_t rl = threadIdx.x / d4;
    if (rl >= (uint32_t)a.ipw) return;
    row = blockIdx.x * (uint32_t)a.ipw + rl;
    if (row >= (uint32_t)a.n_ids) return;
    c4 = threadIdx.x - rl * d4;
    f = row * d4 + c4;
  } else {
    f = blockIdx.x * 256u + threadIdx.x;
    if (f >= (uint32_t)a.total4) return;
    row = f / d4;
    c4 = f - row * d4;
  }
  if (a.gw == 0) {
    if constexpr (IDS_I64) {
      id = ((const int64_t*)a.ids)[row];
    } else {
      id = (int64_t)((const uint32_t*)a.ids)[row];
    }
  }

  nsr_float4 o;
  if (id < 0 || id >= a.vocab) {
    o = nsr_float4{0.f, 0.f, 0.f, 0.f};
    if (a.err_flag) *a.err_flag = 1;
  } else {
    const uint8_t* bp = a.blocks + id * (int64_t)a.row_bytes + (c4 >> 3) * 34u;
    const float d = f16_bits_to_f32(*(const uint16_t*)bp);
    typedef __attribute__((address_space(1))) const uint32_t gword;
    const uint32_t q = *(gword*)(bp + 2 + (c4 & 7u) * 4u);
    o.x = (float)(int32_t)(int8_t)(q & 0xffu) * d;
    o.y = (float)(int32_t)(int8_t)((q >> 8) & 0xffu) * d;
    o.z = (float)(int32_t)(int8_t)((q >> 16) & 0xffu) * d;
    o.w = (float)(int32_t)(int8_t)(q >> 24) * d;
    if constexpr (ACT != ACT_NONE) {
      o.x = apply_act<ACT>(o.x);
      o.y = apply_act<ACT>(o.y);
      o.z = apply_act<ACT>(o.z);
      o.w = apply_act<ACT>(o.w);
    }
  }
  __builtin_nontemporal_store(o, (nsr_float4*)(a.out) + f);
}

#define NSR_Q8_KERNEL(NAME, ACT, I64)                                          \
  extern "C" __global__ void __launch_bounds__(256) NAME(const nsr_q8_args a) { \
    q8_0_gather_body<ACT, I64>(a);                                             \
  }

NSR_Q8_KERNEL(nsrk_q8_0_gather_none_u32, ACT_NONE, false)
NSR_Q8_KERNEL(nsrk_q8_0_gather_silu_u32, ACT_SILU, false)
NSR_Q8_KERNEL(nsrk_q8_0_gather_gelu_u32, ACT_GELU, false)
NSR_Q8_KERNEL(nsrk_q8_0_gather_none_i64, ACT_NONE, true)
NSR_Q8_KERNEL(nsrk_q8_0_gather_silu_i64, ACT_SILU, true)
NSR_Q8_KERNEL(nsrk_q8_0_gather_gelu_i64, ACT_GELU, true)
