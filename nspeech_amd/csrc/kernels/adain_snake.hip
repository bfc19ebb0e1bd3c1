/*
 * Fused AdaIN1d + Snake over x [B, C, T] f32.
 *
 * Reference semantics (src/kokoro/decoder.rs:1416-1428, :1471-1476):
 *   mean = mean_T(x); var = mean_T((x - mean)^2)          (biased)
 *   norm = (x - mean) / sqrt(var + 1e-5)
 *   y    = norm * (gamma + 1) + beta
 *   out  = y + sin(alpha * y)^2 * recip(alpha + 1e-9)
 * gamma/beta come per (batch, channel) from the style Linear (precomputed and
 * rounded to f16 for the GPU backend, decoder.rs:966-981), alpha per channel.
 *
 * Row kernel (aligned rows: x, out 16-byte aligned, T % 4 == 0): the row is
 * read from HBM once into registers and LDS, its statistics are two passes
 * over the on-chip copy, and the output is written once: HBM traffic is the
 * algorithmic 8 bytes per element. Long rows run on a persistent grid that
 * overlaps the next row's reads with the current row's writes.
 *
 * Unaligned rows take the register-resident kernel further down (global
 * loads, partial edge chunks per element). Rows longer than the on-chip
 * budget take the long-row kernel at the end: f64 sum and sum of squares
 * over one read, then a second read to apply.
 */
#include "device_common.h"

/* The three per-row parameters: loaded raw at the top of a kernel (in flight
 * together, before the row's loads) and converted where they are first
 * needed, so the wait for them falls after the row's loads were issued. The
 * loads are branch-free (a dtype branch would make the compiler wait at the
 * join): each reads the aligned dword holding the value (an f16 value and
 * its dword share a page) and the half is selected afterwards. */
struct adain_raw {
  uint32_t g, b, l;
};

NSR_DEV uint32_t adain_raw_load(const void* p, int64_t i, int sz) {
  const uint64_t addr = (uint64_t)p + (uint64_t)(i * sz);
  typedef const __attribute__((address_space(1))) uint32_t gword; /* global, not flat */
  const uint32_t w = *(gword*)(addr & ~(uint64_t)3);
  return sz == 4 ? w : (w >> ((uint32_t)(addr & 2) * 8u)) & 0xffffu;
}

template <typename A>
NSR_DEV adain_raw adain_params_load(const A& a, int pdt, int64_t bi, int64_t ci) {
  const int sz = pdt == DT_F32 ? 4 : 2;
  adain_raw r;
  r.g = adain_raw_load(a.gamma, bi * a.gamma_bstride + ci, sz);
  r.b = adain_raw_load(a.beta, bi * a.beta_bstride + ci, sz);
  r.l = adain_raw_load(a.alpha, ci, sz);
  return r;
}

/* (batch, channel) of a row = (row / C, row % C) in 32-bit arithmetic, for a row below 2^31 (a
 * workgroup index, or any row when n_rows fits): a 64-bit division costs about 150 instructions. */
NSR_DEV void row_bc32(int64_t row, int C, int64_t& bi, int64_t& ci) {
  const uint32_t r = (uint32_t)row, c = (uint32_t)C, q = r / c;
  bi = (int64_t)q;
  ci = (int64_t)(r - q * c);
}

NSR_DEV void adain_params_cvt(const adain_raw& r, int pdt, float& gam, float& bet, float& alp) {
  gam = pdt == DT_F32 ? __uint_as_float(r.g) : f16_bits_to_f32(r.g);
  bet = pdt == DT_F32 ? __uint_as_float(r.b) : f16_bits_to_f32(r.b);
  alp = pdt == DT_F32 ? __uint_as_float(r.l) : f16_bits_to_f32(r.l);
}

typedef __attribute__((address_space(3))) void lds_void;

NSR_DEV nsr_float4 adain_snake4(nsr_float4 d, float A, float bet, const snake_consts& sc) {
  nsr_float4 o;
  o.x = snake_eval(__builtin_fmaf(d.x, A, bet), sc);
  o.y = snake_eval(__builtin_fmaf(d.y, A, bet), sc);
  o.z = snake_eval(__builtin_fmaf(d.z, A, bet), sc);
  o.w = snake_eval(__builtin_fmaf(d.w, A, bet), sc);
  return o;
}

NSR_DEV float sumsq4(nsr_float4 d, float sq) {
  sq = __builtin_fmaf(d.x, d.x, sq);
  sq = __builtin_fmaf(d.y, d.y, sq);
  sq = __builtin_fmaf(d.z, d.z, sq);
  return __builtin_fmaf(d.w, d.w, sq);
}

NSR_DEV float sum4(nsr_float4 d) { return (d.x + d.y) + (d.z + d.w); }

/* ------------------------------------------------------------ row kernel -- */

/* Rows of a workgroup: row = blockIdx.x, + gridDim.x, ... The host launches
 * one workgroup per row when several fit on a CU, and a persistent grid of
 * one workgroup per CU when a row fills a CU's registers and LDS. The row is
 * held on chip as BLOCK-wide slots of 16-byte chunks: NV slots in VGPRs
 * (buffer_load_dwordx4 with the slot offset in an SGPR) and NL slots in LDS
 * (buffer_load_dwordx4 ... lds, each wave's lanes landing in the wave's own
 * LDS region, which only that wave reads).
 *
 * Statistics: one pass over the on-chip row for sum(x) and sum(x^2) and one
 * block reduction, var = E[x^2] - mean^2. Its rounding error relative to var
 * is about (1 + mean^2 / var) f32 ulps of the sums, so a row with
 * 4 mean^2 > var (a workgroup-uniform test) takes a second pass instead: the
 * centred sums of (x - mean)^2 and (x - mean), the second correcting the f32
 * mean (var = (S2 - S1^2 / T) / T, the corrected two-pass form). Measured on
 * MI355X at [8, 128, 115200], with the two-pass form for every row the
 * kernel took 159.9-160.8 us (minimum of 20 calls) against 157.4-158.1 us.
 * Chunks past the row end are masked out of the sums (a VGPR load past the
 * buffer range returns 0, but a load to LDS past it leaves the LDS slot as it
 * was); their stores are dropped by the buffer range check.
 *
 * The store pass of row r refills each slot with row r + gridDim.x once the
 * slot's output is stored (stores and refills in batches of 8 slots), so on a
 * CU the reads of the next row overlap the writes of the current one, and HBM traffic stays the algorithmic
 * 8 bytes per element (x read once, out written once). */
template <int BLOCK, int NV, int NL, bool TL = false>
NSR_DEV void adain_row(const nsr_adain_args& a, int pdt) {
  NSR_NO_CONTRACT
  constexpr int NW = BLOCK / 64;
  constexpr int NS = NV + NL;
  /* only the last MK slots may reach past the row end: the host picks NS
   * with (NS - MK) * BLOCK <= T / 4 */
  constexpr int MK = NS < 4 ? NS : 4;
  extern __shared__ nsr_float4 lds_x[];
  /* two block-sum buffers of 2 NW floats, used in turn: a wave writes one only after the barrier of a block
   * sum on the other, which every wave passes after reading this one's previous sums (no trailing barrier) */
  __shared__ float red[4 * NW];
  int rb = 0;

  const int tid = threadIdx.x;
  int64_t row = blockIdx.x;
  if (row >= a.n_rows) return;
  /* TL: the timeline copy writes s_memrealtime stamps (NSR_ADAIN_TL_WORDS per workgroup, from lane 0 of each
   * wave with vector stores); otherwise it is the same kernel */
  uint64_t* const tl = TL ? a.stamps + (size_t)blockIdx.x * NSR_ADAIN_TL_WORDS : nullptr;
  int tl_row = 0;
  if constexpr (TL) {
    if (tid == 0) {
      uint32_t xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      tl[0] = xcc;
      tl[1] = __builtin_amdgcn_s_memrealtime();
    }
  }
  const int64_t T = a.T;
  const int nch = (int)(T >> 2);
  const uint32_t rbytes = (uint32_t)(T * 4);
  const uint32_t voff = (uint32_t)tid * 16u;
  /* LDS slots of this wave: base address wave-uniform (an SGPR, M0 per load);
   * lane i of the wave lands at base + 16 i, i.e. at lds_x[m * BLOCK + tid] */
  lds_void* const lw = (lds_void*)(lds_x + __builtin_amdgcn_readfirstlane(tid & ~63));

  /* slot k of this lane lies inside the row iff k < nvalid (tested for the
   * last MK slots only; a per-slot lane mask for every slot would be kept in
   * SGPR pairs across the row loop) */
  const int nvalid = nch > tid ? (nch - tid + BLOCK - 1) / BLOCK : 0;
  auto valid = [&](int k) { return k < NS - MK || k < nvalid; };
  const nsr_float4 zero4 = {0.f, 0.f, 0.f, 0.f};

  /* Cache policy of the loads: LDS slots cached, the first KC = min(NV, 8) VGPR slots cached beside 19 LDS
   * slots, the other VGPR slots non-temporal (streamed). Measured on MI355X, [8, 128, T] f32, minimum / median
   * of 5 x 20 calls, against every VGPR slot streamed: T = 115,200 (38 VGPR slots) 151.2-151.7 / 153.3-154.3
   * against 156.5-156.9 / 157.8-158.0 us (4, 6, 10 and 12 cached slots within 1 us of 8; all 19 LDS-slot loads
   * streamed too: 173 us; every load cached: 180 us); T = 81,920 (21) 109.8 / 111.3 against 111.4-111.8 /
   * 112.9-114.2 us; T = 61,440 (11) 73.9 / 76.5 against 78.2 / 80.8 us; T = 53,248 (7, all cached) 65.3-65.5
   * / 67.1-67.3 against 66.4-66.6 / 69.1-69.4 us; T = 40,960 (1) 51.5 / 52.7 against 53.1-53.2 / 54.6-55.1 us.
   * VGPR-only 512-lane kernels of 16 and 20 slots (two workgroups per CU) cache half their slots: T = 38,912
   * (20 slots) 51.6-51.7 against 54.9-55.3 us (8 cached: 53.1-53.3), T = 32,768 (16) 43.5 against 45.3 us;
   * with 10 or 12 slots (three or four workgroups per CU) caching gained nothing (27.1-27.2 / 33.6-33.7
   * against 26.9-27.2 / 33.8 us). Output is the same bits either way. */
  constexpr int KC = NL == 19 ? (NV < 8 ? NV : 8) : (BLOCK == 512 && NV >= 16 ? NV / 2 : 0);
  auto vload = [&](nsr_rsrc r, int k, uint32_t vo, uint32_t so) {
    return k < KC ? buf_load4c(r, vo, so) : buf_load4(r, vo, so);
  };

  /* first row: every slot's load, then the parameters */
  nsr_float4 v[NV];
  {
    const nsr_rsrc xr = make_rsrc(a.x + row * T, rbytes);
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = vload(xr, k, voff, (uint32_t)(k * BLOCK * 16));
#pragma unroll
    for (int m = 0; m < NL; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)((char*)lw + m * BLOCK * 16), 16, voff,
                                               (uint32_t)((NV + m) * BLOCK * 16), 0, 0);
  }
  int64_t bi0, ci0;
  row_bc32(row, a.C, bi0, ci0);
  adain_raw pr = adain_params_load(a, pdt, bi0, ci0);

  while (true) {
    const int64_t next = row + gridDim.x;
    const bool more = next < a.n_rows;
    NSR_WAIT_VMCNT(0); /* every slot of this row has landed (VGPRs and LDS) */
    if constexpr (TL) {
      if ((tid & 63) == 0 && tl_row < 8) tl[10 + 8 * tl_row + (tid >> 6)] = __builtin_amdgcn_s_memrealtime();
      ++tl_row;
    }

    /* one pass: sum and sum of squares */
    float s = 0.f, q = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (valid(k)) {
        s += sum4(v[k]);
        q = sumsq4(v[k], q);
      }
    }
    /* LDS slots in groups of four: the scheduler would otherwise issue every
     * slot's read at once and hold NL x 4 more VGPRs */
    static_for<0, (NL + 3) / 4>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
#pragma unroll
      for (int m = 4 * g; m < (4 * g + 4 < NL ? 4 * g + 4 : NL); ++m) {
        const nsr_float4 xl = lds_x[m * BLOCK + tid];
        if (valid(NV + m)) {
          s += sum4(xl);
          q = sumsq4(xl, q);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    block_sum2<NW, false>(s, q, red + rb);
    rb ^= 2 * NW;
    const float mean = s * a.inv_t;
    float var = __builtin_fmaf(-mean, mean, q * a.inv_t);
    /* the VGPR slots hold x - vbase and the LDS slots x - lbase; (x - mean - c) A + beta = (x - vbase) A + Bc */
    float vshift = mean, lbase = 0.f;
    if (4.0f * mean * mean > var) {
      /* second pass: centred sums; the VGPR slots keep x - mean (0 outside the row) */
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const nsr_float4 d = v[k] - mean;
        v[k] = valid(k) ? d : zero4;
        s1 += sum4(v[k]);
        s2 = sumsq4(v[k], s2);
      }
      static_for<0, (NL + 3) / 4>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
#pragma unroll
        for (int m = 4 * g; m < (4 * g + 4 < NL ? 4 * g + 4 : NL); ++m) {
          nsr_float4 d = lds_x[m * BLOCK + tid] - mean;
          d = valid(NV + m) ? d : zero4;
          s1 += sum4(d);
          s2 = sumsq4(d, s2);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      block_sum2<NW, false>(s1, s2, red + rb);
      rb ^= 2 * NW;
      vshift = s1 * a.inv_t; /* f32 mean correction c */
      lbase = mean;
      var = __builtin_fmaf(-vshift, s1, s2) * a.inv_t;
    }
    var = fmaxf(var, 0.0f);
    const float rstd = __builtin_amdgcn_rsqf(var + a.eps); /* v_rsq_f32, about 1 ulp */
    float gam, bet, alp;
    adain_params_cvt(pr, pdt, gam, bet, alp);
    const float A = (gam + 1.0f) * rstd;
    const float Bc = __builtin_fmaf(-vshift, A, bet);
    const snake_consts sc = make_snake_consts(alp);

    /* store pass; each slot is refilled with the next row once its output is
     * issued (a past-the-end row reads nothing: its range is 0 bytes) */
    if (more) {
      /* 32-bit (batch, channel) when every row index fits (uniform), not a 64-bit division ahead of the stores */
      int64_t bn, cn;
      if (a.n_rows <= 0x7fffffffLL) {
        row_bc32(next, a.C, bn, cn);
      } else {
        bn = next / a.C;
        cn = next - bn * a.C;
      }
      pr = adain_params_load(a, pdt, bn, cn);
    }
    const nsr_rsrc orr = make_rsrc(a.out + row * T, rbytes);
    const nsr_rsrc xn = make_rsrc(a.x + (more ? next : row) * T, more ? rbytes : 0u);
    /* slot offsets are formed from a fresh copy of the lane offset and an
     * opaque zero each row: as loop invariants the compiler would keep all
     * NS of them live in registers across the loop */
    uint32_t vo = voff, so;
    asm volatile("" : "+v"(vo));
    asm volatile("s_mov_b32 %0, 0" : "=s"(so));
    lds_void* lwr = lw;
    asm volatile("" : "+s"(lwr));
    /* in batches of SB slots: SB stores, then the SB refill loads of those slots (sched_barrier keeps the
     * order). Measured on MI355X at [8, 128, 115200]: 160-161 us against 163-165 us with each store followed
     * by its slot's load; batches of 4 or 6 and of 12 or more were slower than 8. */
    constexpr int SB = 8;
    static_for<0, (NV + SB - 1) / SB>([&](auto gc) {
      constexpr int k0 = decltype(gc)::value * SB;
      constexpr int k1 = k0 + SB < NV ? k0 + SB : NV;
#pragma unroll
      for (int k = k0; k < k1; ++k) buf_store4(orr, vo, (uint32_t)(k * BLOCK * 16), adain_snake4(v[k], A, Bc, sc));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = k0; k < k1; ++k) v[k] = vload(xn, k, vo, so + (uint32_t)(k * BLOCK * 16));
      __builtin_amdgcn_sched_barrier(0);
    });
    static_for<0, (NL + SB - 1) / SB>([&](auto gc) {
      constexpr int m0 = decltype(gc)::value * SB;
      constexpr int m1 = m0 + SB < NL ? m0 + SB : NL;
#pragma unroll
      for (int m = m0; m < m1; ++m) {
        const nsr_float4 d = lds_x[m * BLOCK + tid] - lbase;
        buf_store4(orr, vo, (uint32_t)((NV + m) * BLOCK * 16), adain_snake4(d, A, Bc, sc));
      }
      __builtin_amdgcn_sched_barrier(0);
      /* each slot's LDS read above has completed: its value was stored */
#pragma unroll
      for (int m = m0; m < m1; ++m)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xn, (lds_void*)((char*)lwr + m * BLOCK * 16), 16, vo,
                                                 so + (uint32_t)((NV + m) * BLOCK * 16), 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    if (!more) break;
    row = next;
  }
  if constexpr (TL) {
    NSR_WAIT_VMCNT(0); /* this wave's last stores have completed */
    if ((tid & 63) == 0) tl[2 + (tid >> 6)] = __builtin_amdgcn_s_memrealtime();
  }
}

#define NSR_ADAIN_ROW(BLOCK, NV, NL)                                                        \
  extern "C" __global__ void __launch_bounds__(BLOCK)                                      \
      nsrk_adain_row_b##BLOCK##_v##NV##_l##NL(const nsr_adain_args a, const int pdt) {     \
    adain_row<BLOCK, NV, NL>(a, pdt);                                                      \
  }

/* short rows: 256 threads, 1..8 VGPR slots (T <= 8192) */
NSR_ADAIN_ROW(256, 1, 0)
NSR_ADAIN_ROW(256, 2, 0)
NSR_ADAIN_ROW(256, 3, 0)
NSR_ADAIN_ROW(256, 4, 0)
NSR_ADAIN_ROW(256, 5, 0)
NSR_ADAIN_ROW(256, 6, 0)
NSR_ADAIN_ROW(256, 7, 0)
NSR_ADAIN_ROW(256, 8, 0)
/* medium rows: 512 threads, VGPR slots only, 5..20 slots (T <= 40960) */
NSR_ADAIN_ROW(512, 5, 0)
NSR_ADAIN_ROW(512, 6, 0)
NSR_ADAIN_ROW(512, 8, 0)
NSR_ADAIN_ROW(512, 10, 0)
NSR_ADAIN_ROW(512, 12, 0)
NSR_ADAIN_ROW(512, 16, 0)
NSR_ADAIN_ROW(512, 20, 0)
/* long rows, 20..58 slots (T <= 118784): 19 LDS slots (152 KiB) and the rest in VGPRs. Measured on MI355X
 * (1024 rows, us per call, minimum of 20): T = 115200 155.3-155.6 against 157.6-158.7 with 40 VGPR + 18 LDS
 * slots (one slot past the row); T = 92160 123.0-123.4 against 134.3 (40 + 6); T = 60000 76.5-76.8 against
 * 87.3 (32 VGPR slots only); T = 40960 53.3 against 58.9 (20 VGPR slots only). Loads that land in LDS
 * by buffer_load ... lds cost less per slot than loads into VGPRs; below 20 slots the VGPR-only kernels,
 * which fit several workgroups per CU, are faster (T = 24576: 33.9 against 36.1 us with 1 + 11). */
NSR_ADAIN_ROW(512, 1, 19)
NSR_ADAIN_ROW(512, 2, 19)
NSR_ADAIN_ROW(512, 3, 19)
NSR_ADAIN_ROW(512, 4, 19)
NSR_ADAIN_ROW(512, 5, 19)
NSR_ADAIN_ROW(512, 6, 19)
NSR_ADAIN_ROW(512, 7, 19)
NSR_ADAIN_ROW(512, 8, 19)
NSR_ADAIN_ROW(512, 9, 19)
NSR_ADAIN_ROW(512, 10, 19)
NSR_ADAIN_ROW(512, 11, 19)
NSR_ADAIN_ROW(512, 12, 19)
NSR_ADAIN_ROW(512, 13, 19)
NSR_ADAIN_ROW(512, 14, 19)
NSR_ADAIN_ROW(512, 15, 19)
NSR_ADAIN_ROW(512, 16, 19)
NSR_ADAIN_ROW(512, 17, 19)
NSR_ADAIN_ROW(512, 18, 19)
NSR_ADAIN_ROW(512, 19, 19)
NSR_ADAIN_ROW(512, 20, 19)
NSR_ADAIN_ROW(512, 21, 19)
NSR_ADAIN_ROW(512, 22, 19)
NSR_ADAIN_ROW(512, 23, 19)
NSR_ADAIN_ROW(512, 24, 19)
NSR_ADAIN_ROW(512, 25, 19)
NSR_ADAIN_ROW(512, 26, 19)
NSR_ADAIN_ROW(512, 27, 19)
NSR_ADAIN_ROW(512, 28, 19)
NSR_ADAIN_ROW(512, 29, 19)
NSR_ADAIN_ROW(512, 30, 19)
NSR_ADAIN_ROW(512, 31, 19)
NSR_ADAIN_ROW(512, 32, 19)
NSR_ADAIN_ROW(512, 33, 19)
NSR_ADAIN_ROW(512, 34, 19)
NSR_ADAIN_ROW(512, 35, 19)
NSR_ADAIN_ROW(512, 36, 19)
NSR_ADAIN_ROW(512, 37, 19)
NSR_ADAIN_ROW(512, 38, 19)
NSR_ADAIN_ROW(512, 39, 19)

/* The c4b row kernel (T of 56-57 slots) with the timeline stamps, for the measurement entry point
 * nsr_calib_adain_timeline: where in a call each workgroup and wave spends its time. */
extern "C" __global__ void __launch_bounds__(512)
    nsrk_adain_row_tl_b512_v38_l19(const nsr_adain_args a, const int pdt) {
  adain_row<512, 38, 19, true>(a, pdt);
}

/* ------------------------------------------------ unaligned resident rows -- */

/* Rows whose start is not 16-byte aligned (misaligned views, T % 4 != 0).
 * Chunks lie on the float4 grid of the tensor: the row's first and last chunk
 * are partial and taken one element per lane by the last 8 lanes, the
 * interior chunks 1..nch-2 are full and spread as j = 1 + tid + BLOCK*k. Loads of the chunk
 * array are branch-free (index clamped in bounds, out-of-row slots zeroed by
 * a select), which keeps the array in VGPRs. Two-pass statistics over the
 * registers (mean, then centred sums with the corrected two-pass term). */
template <int BLOCK, int NV>
NSR_DEV void adain_resident_u(const nsr_adain_args& a, int pdt) {
  NSR_NO_CONTRACT
  constexpr int NW = BLOCK / 64;
  __shared__ float red[4 * NW]; /* [0, 2 NW): the one-pass sums, [2 NW, 4 NW): the centred sums */
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t T = a.T;
  const int64_t s = row * T;
  const int64_t a0 = s & ~(int64_t)3;
  const int lo = (int)(s - a0);        /* first row element in chunk space */
  const int64_t hi = (int64_t)lo + T;  /* one past the last */
  const int nch = (int)((hi + 3) >> 2);
  const int jlast = nch - 1;
  const float* xb = a.x + a0;
  float* ob = a.out + a0;
  const nsr_float4 zero4 = {0.f, 0.f, 0.f, 0.f};
  const int jbase = 1 + tid;
  const int jmax = nch - 2;

  nsr_float4 v[NV];
  if (jmax >= 1) { /* at least one interior chunk (uniform) */
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = jbase + BLOCK * k;
      const nsr_float4 t = ldf4(xb + 4 * (int64_t)min(j, jmax));
      v[k] = j <= jmax ? t : zero4;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = zero4;
  }
  /* the two edge chunks, one element per lane on the last 8 lanes of the
   * workgroup: lane q = tid - (BLOCK - 8) takes element q & 3 of chunk 0
   * (q < 4) or chunk nch - 1 (q >= 4) when it belongs to the row */
  const int q = tid - (BLOCK - 8);
  const int64_t eidx = q >= 4 ? 4 * (int64_t)jlast + (q & 3) : (int64_t)(q & 3);
  const bool eok = q >= 0 && eidx >= lo && eidx < hi && (q < 4 || jlast > 0);
  const float xe = eok ? xb[eidx] : 0.f;
  /* the row's parameters, after its loads */
  int64_t bi, ci;
  row_bc32(row, a.C, bi, ci);
  const adain_raw pr = adain_params_load(a, pdt, bi, ci);

  /* one pass (sum, sum of squares), the centred pass when 4 mean^2 > var, as adain_row */
  float sum = xe, sq = xe * xe;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    sum += sum4(v[k]);
    sq = sumsq4(v[k], sq);
  }
  block_sum2<NW, false>(sum, sq, red);
  const float mean = sum * a.inv_t;
  float var = __builtin_fmaf(-mean, mean, sq * a.inv_t);
  float vshift = mean, ebase = 0.f; /* (x - mean - c) A + beta = (v - vshift) A + beta, v = x - ebase */
  if (4.0f * mean * mean > var) {
    float s2 = 0.f, sd = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = jbase + BLOCK * k;
      const nsr_float4 d = v[k] - mean;
      v[k] = j <= jmax ? d : zero4;
      s2 = sumsq4(v[k], s2);
      sd += sum4(v[k]);
    }
    if (eok) {
      const float d = xe - mean;
      s2 = __builtin_fmaf(d, d, s2);
      sd += d;
    }
    block_sum2<NW, false>(s2, sd, red + 2 * NW);
    vshift = sd * a.inv_t;
    ebase = mean;
    var = __builtin_fmaf(-vshift, sd, s2) * a.inv_t;
  }
  var = fmaxf(var, 0.0f);
  const float rstd = __builtin_amdgcn_rsqf(var + a.eps); /* v_rsq_f32, about 1 ulp */
  float gam, bet, alp;
  adain_params_cvt(pr, pdt, gam, bet, alp);
  const float A = (gam + 1.0f) * rstd;
  const float Bc = __builtin_fmaf(-vshift, A, bet);
  const snake_consts sc = make_snake_consts(alp);

#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = jbase + BLOCK * k;
    const nsr_float4 o = adain_snake4(v[k], A, Bc, sc);
    if (j <= jmax) stf4(ob + 4 * (int64_t)j, o);
  }
  if (eok) ob[eidx] = snake_eval(__builtin_fmaf(xe - ebase, A, Bc), sc);
}

#define NSR_ADAIN_RES_U(BLOCK, NV)                                                      \
  extern "C" __global__ void __launch_bounds__(BLOCK)                                  \
      nsrk_adain_res_b##BLOCK##_nv##NV##_u(const nsr_adain_args a, const int pdt) {    \
    adain_resident_u<BLOCK, NV>(a, pdt);                                               \
  }

NSR_ADAIN_RES_U(256, 1)
NSR_ADAIN_RES_U(256, 2)
NSR_ADAIN_RES_U(256, 3)
NSR_ADAIN_RES_U(256, 4)
NSR_ADAIN_RES_U(256, 5)
NSR_ADAIN_RES_U(256, 6)
NSR_ADAIN_RES_U(256, 8)
NSR_ADAIN_RES_U(512, 12)
NSR_ADAIN_RES_U(512, 16)
NSR_ADAIN_RES_U(512, 24)
NSR_ADAIN_RES_U(512, 32)

/* ------------------------------------------------------------- f16 rows -- */

/* x, out [B, C, T] f16, the reference's f16-activation form
 * (KokoroGpuBackend::adain_snake, src/kokoro/gpu_backend.rs:55-57; Triton
 * adain_snake_fused / adain_snake_looped, kernels/kokoro_kernels.py:222-331:
 * f16 loaded to f32, f32 statistics and snake, result rounded to f16).
 * The row stays in VGPRs as raw 16-byte chunks (8 halves in 4 VGPRs) on the
 * 16-byte grid of the address space, so any row start works: the row's first
 * and last chunk may be partial and are taken one element per lane by the
 * last 16 lanes, the interior chunks 1..nch-2 are spread as
 * j = 1 + tid + BLOCK k with clamped, branch-free loads. out must share x's offset within 16 bytes (checked by
 * the host). Two-pass statistics over the registers, as the f32 kernels. */
/* pointers rebuilt from integer addresses are generic (flat accesses, which
 * count against both memory counters); these keep them global */
typedef __attribute__((address_space(1))) uint16_t nsr_gh;
NSR_DEV nsr_uint4 ld16g(const nsr_gh* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) nsr_uint4*)p);
}
NSR_DEV void st16g(nsr_gh* p, nsr_uint4 v) {
  __builtin_nontemporal_store(v, (__attribute__((address_space(1))) nsr_uint4*)p);
}

template <int BLOCK, int NV>
NSR_DEV void adain_row_f16(const nsr_adain_h_args& a, int pdt) {
  NSR_NO_CONTRACT
  constexpr int NW = BLOCK / 64;
  __shared__ float red[3 * NW]; /* [0, NW): the mean's sums, [NW, 3 NW): the centred sums */
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (row >= a.n_rows) return; /* whole workgroup: the grid is one per row */
  const int64_t T = a.T;
  const uint64_t xa = (uint64_t)(a.x + row * T);
  const uint64_t oa = (uint64_t)(a.out + row * T);
  const int lo = (int)((xa & 15) >> 1); /* first row element in chunk space */
  const int64_t hi = (int64_t)lo + T;   /* one past the last */
  const int nch = (int)((hi + 7) >> 3);
  const int jlast = nch - 1;
  const int jmax = nch - 2;
  const int jbase = 1 + tid;
  const nsr_gh* xb = (const nsr_gh*)(xa & ~(uint64_t)15);
  nsr_gh* ob = (nsr_gh*)(oa & ~(uint64_t)15);
  const nsr_uint4 zero = {0u, 0u, 0u, 0u};

  nsr_uint4 v[NV];
  if (jmax >= 1) { /* at least one interior chunk (uniform) */
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = jbase + BLOCK * k;
      const nsr_uint4 t = ld16g(xb + 8 * (int64_t)min(j, jmax));
      v[k] = j <= jmax ? t : zero;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = zero;
  }
  /* the two edge chunks, one element per lane on the last 16 lanes of the
   * workgroup: lane q = tid - (BLOCK - 16) takes element q & 7 of chunk 0
   * (q < 8) or chunk nch - 1 (q >= 8) when it belongs to the row */
  const int q = tid - (BLOCK - 16);
  const int64_t eidx = q >= 8 ? 8 * (int64_t)jlast + (q & 7) : (int64_t)(q & 7);
  const bool eok = q >= 0 && eidx >= lo && eidx < hi && (q < 8 || jlast > 0);
  const float xe = eok ? f16_bits_to_f32(xb[eidx]) : 0.f;
  /* the row's parameters, after its loads */
  int64_t bi, ci;
  row_bc32(row, a.C, bi, ci);
  const adain_raw pr = adain_params_load(a, pdt, bi, ci);

  float sum = xe;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float f[8];
    unpack16<DT_F16>(v[k], f);
    sum += ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
  }
  const float mean = block_sum<NW, false>(sum, red) * a.inv_t;

  /* the chunks stay raw (4 VGPRs each) between passes: an empty asm that
   * "modifies" them stops the compiler keeping their unpacked floats (8) live */
#pragma unroll
  for (int k = 0; k < NV; ++k) asm volatile("" : "+v"(v[k]));
  /* centred sums; slots outside the interior hold zeros and are weighted out */
  float sq = 0.f, sd = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = jbase + BLOCK * k;
    float f[8], q = 0.f, t = 0.f;
    unpack16<DT_F16>(v[k], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = f[e] - mean;
      q = __builtin_fmaf(d, d, q);
      t += d;
    }
    sq += j <= jmax ? q : 0.f;
    sd += j <= jmax ? t : 0.f;
  }
  if (eok) {
    const float d = xe - mean;
    sq = __builtin_fmaf(d, d, sq);
    sd += d;
  }
  block_sum2<NW, false>(sq, sd, red + NW);
  const float c = sd * a.inv_t;
  const float var = fmaxf(__builtin_fmaf(-c, sd, sq) * a.inv_t, 0.0f);
  const float rstd = __builtin_amdgcn_rsqf(var + a.eps); /* v_rsq_f32, about 1 ulp */
  float gam, bet, alp;
  adain_params_cvt(pr, pdt, gam, bet, alp);
  const float A = (gam + 1.0f) * rstd;
  const float Bc = __builtin_fmaf(-c, A, bet); /* (x - mean - c) A + beta */
  const snake_consts_h sc = make_snake_consts_h(alp); /* f16 output */

#pragma unroll
  for (int k = 0; k < NV; ++k) asm volatile("" : "+v"(v[k]));
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = jbase + BLOCK * k;
    float f[8], o[8];
    unpack16<DT_F16>(v[k], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = snake_eval(__builtin_fmaf(f[e] - mean, A, Bc), sc);
    if (j <= jmax) st16g(ob + 8 * (int64_t)j, pack16<DT_F16>(o));
  }
  if (eok) ob[eidx] = (uint16_t)f32_to_f16_bits(snake_eval(__builtin_fmaf(xe - mean, A, Bc), sc));
}

#define NSR_ADAIN_F16(BLOCK, NV)                                                        \
  extern "C" __global__ void __launch_bounds__(BLOCK)                                  \
      nsrk_adain_f16_b##BLOCK##_nv##NV(const nsr_adain_h_args a, const int pdt) {      \
    adain_row_f16<BLOCK, NV>(a, pdt);                                                  \
  }

NSR_ADAIN_F16(256, 1)
NSR_ADAIN_F16(256, 2)
NSR_ADAIN_F16(256, 3)
NSR_ADAIN_F16(256, 4)
NSR_ADAIN_F16(256, 6)
NSR_ADAIN_F16(256, 8)
NSR_ADAIN_F16(512, 6)
NSR_ADAIN_F16(512, 8)
NSR_ADAIN_F16(512, 12)
NSR_ADAIN_F16(512, 16)
NSR_ADAIN_F16(512, 20)
NSR_ADAIN_F16(512, 24)
NSR_ADAIN_F16(512, 28)
NSR_ADAIN_F16(512, 32)

/* f16 rows that start on 16 bytes with T % 8 == 0 (every row then does):
 * one 256-lane workgroup per row, NV chunks of 8 halves per lane loaded with
 * 16-byte buffer loads and unpacked to f32 once, then the same statistics and
 * output as the f32 row kernel (only the last chunk of a lane can reach past
 * the row; buffer loads there read 0 and stores are dropped). */
template <int NV>
NSR_DEV void adain_row_f16a(const nsr_adain_h_args& a, int pdt) {
  NSR_NO_CONTRACT
  constexpr int BLOCK = 256, NW = BLOCK / 64;
  __shared__ float red[4 * NW]; /* [0, 2 NW): the one-pass sums, [2 NW, 4 NW): the centred sums */
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (row >= a.n_rows) return;
  const int64_t T = a.T;
  const int nch = (int)(T >> 3);
  const uint32_t rbytes = (uint32_t)(T * 2);
  const uint32_t voff = (uint32_t)tid * 16u;
  const nsr_rsrc xr = make_rsrc(a.x + row * T, rbytes);
  nsr_uint4 raw[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k)
    raw[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, voff, (uint32_t)(k * BLOCK * 16), NSR_AUX_NT);
  int64_t bi, ci;
  row_bc32(row, a.C, bi, ci);
  const adain_raw pr = adain_params_load(a, pdt, bi, ci);
  const int nvalid = nch > tid ? (nch - tid + BLOCK - 1) / BLOCK : 0;
  float f[NV][8];
  /* one pass (sum, sum of squares), the centred pass when 4 mean^2 > var, as adain_row */
  float s = 0.f, q = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    unpack16<DT_F16>(raw[k], f[k]);
    const float t = ((f[k][0] + f[k][1]) + (f[k][2] + f[k][3])) + ((f[k][4] + f[k][5]) + (f[k][6] + f[k][7]));
    float u = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) u = __builtin_fmaf(f[k][e], f[k][e], u);
    s += k < nvalid ? t : 0.f;
    q += k < nvalid ? u : 0.f;
  }
  block_sum2<NW, false>(s, q, red);
  const float mean = s * a.inv_t;
  float var = __builtin_fmaf(-mean, mean, q * a.inv_t);
  float vshift = mean; /* the chunks hold x (one pass) or x - mean (centred) */
  if (4.0f * mean * mean > var) {
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[k][e] = k < nvalid ? f[k][e] - mean : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s1 += f[k][e];
        s2 = __builtin_fmaf(f[k][e], f[k][e], s2);
      }
    }
    block_sum2<NW, false>(s1, s2, red + 2 * NW);
    vshift = s1 * a.inv_t;
    var = __builtin_fmaf(-vshift, s1, s2) * a.inv_t;
  }
  var = fmaxf(var, 0.0f);
  const float rstd = __builtin_amdgcn_rsqf(var + a.eps); /* v_rsq_f32, about 1 ulp */
  float gam, bet, alp;
  adain_params_cvt(pr, pdt, gam, bet, alp);
  const float A = (gam + 1.0f) * rstd;
  const float Bc = __builtin_fmaf(-vshift, A, bet);
  const snake_consts_h sc = make_snake_consts_h(alp); /* f16 output */
  const nsr_rsrc orr = make_rsrc(a.out + row * T, rbytes);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = snake_eval(__builtin_fmaf(f[k][e], A, Bc), sc);
    __builtin_amdgcn_raw_buffer_store_b128(pack16<DT_F16>(o), orr, voff + (uint32_t)(k * BLOCK * 16), 0, NSR_AUX_NT);
  }
}

#define NSR_ADAIN_F16A(NV)                                                                 \
  extern "C" __global__ void __launch_bounds__(256)                                       \
      nsrk_adain_f16a_b256_nv##NV(const nsr_adain_h_args a, const int pdt) {              \
    adain_row_f16a<NV>(a, pdt);                                                           \
  }

/* aligned f16 rows up to T = 8192 */
NSR_ADAIN_F16A(1)
NSR_ADAIN_F16A(2)
NSR_ADAIN_F16A(3)
NSR_ADAIN_F16A(4)

/* Long aligned f16 rows (16-byte aligned, T % 8 == 0, T > 8192): the f32 row kernel's structure over
 * 8 halves per 16-byte slot (a persistent grid, NV VGPR slots and NL LDS slots per lane, one-pass
 * statistics with the centred pass when 4 mean^2 > var, the next row's loads refilling each slot once its
 * output is stored, stores and refills in batches of 8). The slots hold the raw halves: the statistics
 * and the output widen them as they read them, and the centred pass subtracts the mean there. */
template <int BLOCK, int NV, int NL>
NSR_DEV void adain_row_h(const nsr_adain_h_args& a, int pdt) {
  NSR_NO_CONTRACT
  constexpr int NW = BLOCK / 64;
  constexpr int NS = NV + NL;
  /* only the last MK slots may reach past the row end: the host picks NS with (NS - MK) * BLOCK <= T / 8 */
  constexpr int MK = NS < 4 ? NS : 4;
  extern __shared__ nsr_uint4 lds_h[];
  __shared__ float red[4 * NW]; /* two block-sum buffers used in turn, as adain_row */
  int rb = 0;

  const int tid = threadIdx.x;
  int64_t row = blockIdx.x;
  if (row >= a.n_rows) return;
  const int64_t T = a.T;
  const int nch = (int)(T >> 3);
  const uint32_t rbytes = (uint32_t)(T * 2);
  const uint32_t voff = (uint32_t)tid * 16u;
  lds_void* const lw = (lds_void*)(lds_h + __builtin_amdgcn_readfirstlane(tid & ~63));
  const int nvalid = nch > tid ? (nch - tid + BLOCK - 1) / BLOCK : 0;
  auto valid = [&](int k) { return k < NS - MK || k < nvalid; };

  nsr_uint4 v[NV];
  {
    const nsr_rsrc xr = make_rsrc(a.x + row * T, rbytes);
#pragma unroll
    for (int k = 0; k < NV; ++k)
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, voff, (uint32_t)(k * BLOCK * 16), NSR_AUX_NT);
#pragma unroll
    for (int m = 0; m < NL; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)((char*)lw + m * BLOCK * 16), 16, voff,
                                               (uint32_t)((NV + m) * BLOCK * 16), 0, 0);
  }
  int64_t bi0, ci0;
  row_bc32(row, a.C, bi0, ci0);
  adain_raw pr = adain_params_load(a, pdt, bi0, ci0);

  /* sums of a slot's 8 values: SUB = false, the one-pass sums straight from the packed halves with
   * v_dot2_f32_f16 (x0 + x1 and x0^2 + x1^2 per word, the products exact in f32); SUB = true, the centred
   * sums of the widened values minus `sub` */
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  auto sums8 = [&](auto subc, const nsr_uint4 w, float sub, bool ok, float& s, float& q) {
    float t = 0.f, u = 0.f;
    if constexpr (decltype(subc)::value) {
      float f[8];
      unpack16<DT_F16>(w, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] -= sub;
      t = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
#pragma unroll
      for (int e = 0; e < 8; ++e) u = __builtin_fmaf(f[e], f[e], u);
    } else {
      const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wi = w[i]; /* a named copy: a bit_cast of the vector element itself reads element 0 */
        const h2_t hw = __builtin_bit_cast(h2_t, wi);
        t = __builtin_amdgcn_fdot2(hw, one, t, false);
        u = __builtin_amdgcn_fdot2(hw, hw, u, false);
      }
    }
    s += ok ? t : 0.f;
    q += ok ? u : 0.f;
  };
  auto all_sums = [&](auto subc, float sub, float& s, float& q) {
#pragma unroll
    for (int k = 0; k < NV; ++k) sums8(subc, v[k], sub, valid(k), s, q);
    /* LDS slots in groups of four, as adain_row */
    static_for<0, (NL + 3) / 4>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
#pragma unroll
      for (int m = 4 * g; m < (4 * g + 4 < NL ? 4 * g + 4 : NL); ++m)
        sums8(subc, lds_h[m * BLOCK + tid], sub, valid(NV + m), s, q);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  while (true) {
    const int64_t next = row + gridDim.x;
    const bool more = next < a.n_rows;
    NSR_WAIT_VMCNT(0); /* every slot of this row has landed (VGPRs and LDS) */

    float s = 0.f, q = 0.f;
    all_sums(std::integral_constant<bool, false>{}, 0.f, s, q);
    block_sum2<NW, false>(s, q, red + rb);
    rb ^= 2 * NW;
    const float mean = s * a.inv_t;
    float var = __builtin_fmaf(-mean, mean, q * a.inv_t);
    /* the output is (x - sub) A + Bc with Bc = beta - vshift A: sub = 0, vshift = mean in one pass; sub = mean and
     * vshift = the f32 mean's correction c in the centred form */
    float sub = 0.f, vshift = mean;
    if (4.0f * mean * mean > var) {
      float s1 = 0.f, s2 = 0.f;
      all_sums(std::integral_constant<bool, true>{}, mean, s1, s2);
      block_sum2<NW, false>(s1, s2, red + rb);
      rb ^= 2 * NW;
      vshift = s1 * a.inv_t;
      sub = mean;
      var = __builtin_fmaf(-vshift, s1, s2) * a.inv_t;
    }
    var = fmaxf(var, 0.0f);
    const float rstd = __builtin_amdgcn_rsqf(var + a.eps); /* v_rsq_f32, about 1 ulp */
    float gam, bet, alp;
    adain_params_cvt(pr, pdt, gam, bet, alp);
    const float A = (gam + 1.0f) * rstd;
    const float Bc = __builtin_fmaf(-vshift, A, bet);
    const snake_consts_h sc = make_snake_consts_h(alp); /* f16 output */

    if (more) {
      int64_t bn, cn;
      if (a.n_rows <= 0x7fffffffLL) {
        row_bc32(next, a.C, bn, cn);
      } else {
        bn = next / a.C;
        cn = next - bn * a.C;
      }
      pr = adain_params_load(a, pdt, bn, cn);
    }
    const nsr_rsrc orr = make_rsrc(a.out + row * T, rbytes);
    const nsr_rsrc xn = make_rsrc(a.x + (more ? next : row) * T, more ? rbytes : 0u);
    uint32_t vo = voff, so;
    asm volatile("" : "+v"(vo));
    asm volatile("s_mov_b32 %0, 0" : "=s"(so));
    lds_void* lwr = lw;
    asm volatile("" : "+s"(lwr));
    /* SUB = false (one pass): x A + Bc straight from each packed half (v_fma_mix_f32); SUB = true: the widened
     * x minus the mean first, which keeps the cancellation out of rows with |mean| >> std */
    auto out8 = [&](auto subc, const nsr_uint4 w) {
      float f[8];
      if constexpr (decltype(subc)::value) {
        unpack16<DT_F16>(w, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = snake_eval(__builtin_fmaf(f[e] - sub, A, Bc), sc);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wi = w[i];
          const h2_t hw = __builtin_bit_cast(h2_t, wi);
          f[2 * i] = snake_eval(__builtin_fmaf((float)hw.x, A, Bc), sc);
          f[2 * i + 1] = snake_eval(__builtin_fmaf((float)hw.y, A, Bc), sc);
        }
      }
      return pack16<DT_F16>(f);
    };
    constexpr int SB = 8;
    auto store_pass = [&](auto subc) {
    static_for<0, (NV + SB - 1) / SB>([&](auto gc) {
      constexpr int k0 = decltype(gc)::value * SB;
      constexpr int k1 = k0 + SB < NV ? k0 + SB : NV;
#pragma unroll
      for (int k = k0; k < k1; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(out8(subc, v[k]), orr, vo + (uint32_t)(k * BLOCK * 16), 0, NSR_AUX_NT);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = k0; k < k1; ++k)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(xn, vo, so + (uint32_t)(k * BLOCK * 16), NSR_AUX_NT);
      __builtin_amdgcn_sched_barrier(0);
    });
    static_for<0, (NL + SB - 1) / SB>([&](auto gc) {
      constexpr int m0 = decltype(gc)::value * SB;
      constexpr int m1 = m0 + SB < NL ? m0 + SB : NL;
#pragma unroll
      for (int m = m0; m < m1; ++m)
        __builtin_amdgcn_raw_buffer_store_b128(out8(subc, lds_h[m * BLOCK + tid]), orr,
                                               vo + (uint32_t)((NV + m) * BLOCK * 16), 0, NSR_AUX_NT);
      __builtin_amdgcn_sched_barrier(0);
      /* each slot's LDS read above has completed: its value was stored */
#pragma unroll
      for (int m = m0; m < m1; ++m)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xn, (lds_void*)((char*)lwr + m * BLOCK * 16), 16, vo,
                                                 so + (uint32_t)((NV + m) * BLOCK * 16), 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    };
    if (sub == 0.f) {
      store_pass(std::integral_constant<bool, false>{});
    } else {
      store_pass(std::integral_constant<bool, true>{});
    }
    if (!more) break;
    row = next;
  }
}

#define NSR_ADAIN_ROW_H(BLOCK, NV, NL)                                                      \
  extern "C" __global__ void __launch_bounds__(BLOCK)                                      \
      nsrk_adain_rowh_b##BLOCK##_v##NV##_l##NL(const nsr_adain_h_args a, const int pdt) {  \
    adain_row_h<BLOCK, NV, NL>(a, pdt);                                                    \
  }

/* aligned f16 rows of 20-32 slots (77,832 <= T <= 131,072): 10 LDS slots (80 KB) and the VGPR slots the row
 * still needs. Measured on MI355X at [8, 128, 115200] f16 (29 slots), minimum of 5 x 20 calls: 19 VGPR +
 * 10 LDS slots 88.2-88.9 us, 10 + 19 88.5-89.8 us, 29 VGPR slots 92.2-92.5 us, against 113.7-118.2 us for
 * the one-workgroup-per-row kernel above, which holds one row per CU at a time. */
NSR_ADAIN_ROW_H(512, 10, 10)
NSR_ADAIN_ROW_H(512, 11, 10)
NSR_ADAIN_ROW_H(512, 12, 10)
NSR_ADAIN_ROW_H(512, 13, 10)
NSR_ADAIN_ROW_H(512, 14, 10)
NSR_ADAIN_ROW_H(512, 15, 10)
NSR_ADAIN_ROW_H(512, 16, 10)
NSR_ADAIN_ROW_H(512, 17, 10)
NSR_ADAIN_ROW_H(512, 18, 10)
NSR_ADAIN_ROW_H(512, 19, 10)
NSR_ADAIN_ROW_H(512, 20, 10)
NSR_ADAIN_ROW_H(512, 21, 10)
NSR_ADAIN_ROW_H(512, 22, 10)

/* ------------------------------------------------ row statistics, long rows -- */

/* Sum and sum of squares of one row over 1024 lanes in f64, one HBM read:
 * 16-byte loads (eight in flight per lane) when VEC4 (row 16-byte aligned,
 * T % 4 == 0), else element loads. In f64, var = S2/T - (S1/T)^2 keeps
 * about 16 - log10(mean^2 / var) significant digits, far more than f32
 * output needs for any |mean| / std below 1e4. `red` holds 32 doubles. */
template <bool VEC4, bool CACHED = false>
NSR_DEV void row_sums64(const float* xr, int64_t T, double* red, double& s1, double& s2) {
  NSR_NO_CONTRACT
  double a1 = 0.0, a2 = 0.0;
  const int tid = threadIdx.x;
  if constexpr (VEC4) {
    const int64_t n4 = T >> 2;
    auto acc4 = [&](const nsr_float4* v) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double x = (double)v[u][e];
          a1 += x;
          a2 = __builtin_fma(x, x, a2);
        }
      }
    };
    /* Groups of 4096 float4 (four strided loads per lane) that every lane
     * loads in full; the group count is uniform, so the loop branches on
     * scalars, and the next group is issued before the current one is
     * summed: eight loads stay in flight per lane. The loads are buffer
     * loads at the lane's fixed offset plus a scalar group offset, so no
     * address register is rewritten while a load into a neighbour is
     * pending. Each lane still adds its elements in increasing order, then
     * the tail one float4 at a time. Rows past 2^28 float4 (beyond the
     * 32-bit buffer offset) take only the tail loop. */
    const int64_t ngroups = n4 < (int64_t(1) << 28) ? n4 >> 12 : 0;
    const nsr_rsrc rx = make_rsrc_uniform(xr, (uint32_t)(ngroups << 16));
    const uint32_t vo = (uint32_t)tid * 16u;
    auto ld4 = [&](nsr_float4* v, int64_t g) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = CACHED ? buf_load4c(rx, vo, (uint32_t)(g << 16) + (uint32_t)u * 16384u)
                      : buf_load4(rx, vo, (uint32_t)(g << 16) + (uint32_t)u * 16384u);
    };
    int64_t g = 0;
    if (ngroups > 0) {
      nsr_float4 ga[4], gb[4]; /* two groups alternate, no register copies */
      ld4(ga, 0);
      for (;;) {
        if (g + 1 >= ngroups) {
          acc4(ga);
          ++g;
          break;
        }
        ld4(gb, g + 1);
        acc4(ga);
        ++g;
        if (g + 1 >= ngroups) {
          acc4(gb);
          ++g;
          break;
        }
        ld4(ga, g + 1);
        acc4(gb);
        ++g;
      }
    }
    int64_t i = (g << 12) + tid;
    for (; i < n4; i += 1024) {
      const nsr_float4 v = ldf4(xr + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double x = (double)v[e];
        a1 += x;
        a2 = __builtin_fma(x, x, a2);
      }
    }
  } else {
    for (int64_t i = tid; i < T; i += 1024) {
      const double x = (double)__builtin_nontemporal_load(xr + i);
      a1 += x;
      a2 = __builtin_fma(x, x, a2);
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    a1 += __shfl_xor(a1, off);
    a2 += __shfl_xor(a2, off);
  }
  const int wid = tid >> 6;
  if ((tid & 63) == 0) {
    red[wid] = a1;
    red[16 + wid] = a2;
  }
  __syncthreads();
  s1 = 0.0;
  s2 = 0.0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    s1 += red[w];
    s2 += red[16 + w];
  }
  __syncthreads();
}

/* mean as an unevaluated f32 pair (hi + lo) and 1 / sqrt(var + eps) */
NSR_DEV void row_moments(double s1, double s2, int64_t T, float eps, float& mhi, float& mlo, float& rstd) {
  const double mean = s1 / (double)T;
  double var = s2 / (double)T - mean * mean;
  var = var > 0.0 ? var : 0.0;
  mhi = (float)mean;
  mlo = (float)(mean - (double)mhi);
  rstd = 1.0f / sqrtf((float)var + eps);
}

/* Row statistics (mean, 1 / sqrt(var + eps)) of [n_rows][T] f32 into
 * a.stats: one 1024-lane workgroup per row, one read of x. Used where the
 * statistics feed another kernel (the AdaIN + Snake input of the conv). */
template <bool VEC4>
NSR_DEV void adain_stats(const nsr_adain_args& a) {
  __shared__ double red[32];
  const int64_t row = blockIdx.x;
  double s1, s2;
  row_sums64<VEC4>(a.x + row * a.T, a.T, red, s1, s2);
  if (threadIdx.x == 0) {
    float mhi, mlo, rstd;
    row_moments(s1, s2, a.T, a.eps, mhi, mlo, rstd);
    a.stats[2 * row] = mhi;
    a.stats[2 * row + 1] = rstd;
  }
}

extern "C" __global__ void __launch_bounds__(1024) nsrk_adain_stats(const nsr_adain_args a) { adain_stats<false>(a); }
extern "C" __global__ void __launch_bounds__(1024) nsrk_adain_stats4(const nsr_adain_args a) { adain_stats<true>(a); }

/* Rows too long to hold on chip (or unaligned rows past the resident
 * kernels' reach): a persistent grid of 1024-lane workgroups, each taking
 * whole rows. Pass 1 reads the row for its f64 sums; pass 2 reads it again
 * and writes the output, centring with the mean as an f32 pair
 * ((x - mean_hi) - mean_lo: the first difference is exact when x is within
 * a factor of two of the mean). The second read follows the first by one
 * row's time, so with a workgroup per CU the rows in flight (a few hundred
 * MB at most) are mostly still in the 256 MB Infinity Cache: the extra
 * traffic is mostly cache, not HBM. No scratch memory. */
template <bool VEC4>
NSR_DEV void adain_long(const nsr_adain_args& a, int pdt) {
  NSR_NO_CONTRACT
  __shared__ double red[32];
  const int tid = threadIdx.x;
  const int64_t T = a.T;
  for (int64_t row = blockIdx.x; row < a.n_rows; row += gridDim.x) {
    const adain_raw pr = adain_params_load(a, pdt, row / a.C, row % a.C);
    const float* xr = a.x + row * T;
    float* orow = a.out + row * T;
    double s1, s2;
    /* the first read cached, so that the second (streamed) finds much of the row in the caches: measured on
     * MI355X at [8, 128, 131072] f32, 240.7-241.6 us against 280.0-281.0 us with both reads streamed (both
     * cached 255.0-255.5, only the second 290.9-291.9 us); the same output bits */
    row_sums64<VEC4, true>(xr, T, red, s1, s2);
    float mhi, mlo, rstd;
    row_moments(s1, s2, T, a.eps, mhi, mlo, rstd);
    float gam, bet, alp;
    adain_params_cvt(pr, pdt, gam, bet, alp);
    const float A = (gam + 1.0f) * rstd;
    const float Bc = __builtin_fmaf(-mlo, A, bet); /* ((x - mhi) - mlo) A + beta */
    const snake_consts sc = make_snake_consts(alp);
    if constexpr (VEC4) {
      const int64_t n4 = T >> 2;
      for (int64_t i = tid; i < n4; i += 1024) {
        const nsr_float4 d = ldf4(xr + 4 * i) - mhi;
        stf4(orow + 4 * i, adain_snake4(d, A, Bc, sc));
      }
    } else {
      for (int64_t i = tid; i < T; i += 1024)
        orow[i] = snake_eval(__builtin_fmaf(__builtin_nontemporal_load(xr + i) - mhi, A, Bc), sc);
    }
  }
}

extern "C" __global__ void __launch_bounds__(1024) nsrk_adain_long(const nsr_adain_args a, const int pdt) {
  adain_long<false>(a, pdt);
}
extern "C" __global__ void __launch_bounds__(1024) nsrk_adain_long4(const nsr_adain_args a, const int pdt) {
  adain_long<true>(a, pdt);
}
