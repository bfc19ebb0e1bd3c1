/*
 * Decode attention (one query position per head) over f16 K/V.
 *
 * Reference semantics: attention_decode_1d / attention_decode_1d_masked
 * (kernels/moonshine_kernels.py:1525-1625, dispatch triton_attention_decode
 * src/triton_kernels.rs:648-675 and enc_attention_decode :900-923; the
 * decoder's self-attention over its KV cache, src/moonshine/
 * gpu_decoder_metal.rs:158-168) and attention_decode_splitkv_partial /
 * _reduce (moonshine_kernels.py:1631-1716, enc_attention_splitkv
 * triton_kernels.rs:925-973; the decoder's cross-attention over the encoder
 * K/V, gpu_decoder_metal.rs:170-182):
 *   kv_head = q_head * n_kv_heads / n_q_heads
 *   s_j     = sm_scale * sum_d q[d] k_j[d]        (f32)
 *   out[d]  = sum_j softmax(s)_j v_j[d]            (online softmax in f32)
 * stored as f16. Element (head, pos, d) of K and V sits at
 * head * stride_kv_head + pos * stride_kv_seq + d (the self-attention cache
 * [heads, max_kv_len, head_dim] and the encoder's [kv_len, heads, head_dim]
 * are both such layouts).
 *
 * Design (gfx950): a wave walks chunks of 64 positions. It first stages the
 * chunk's K and V rows in its own LDS slice with all loads in flight at once
 * (each load instruction covers whole rows; rows padded by 8 bytes so the
 * per-lane row reads hit distinct bank pairs): a loop of dependent loads
 * would pay one memory latency per position. Each lane then scores one
 * position against q (f16 pairs by v_dot2_f32_f16: exact products, f32
 * sums); the chunk's max and sum are DPP wave reductions; the probabilities
 * go through LDS to a dims x position-groups layout for P.V, whose groups
 * are summed through LDS; chunks merge by online-softmax rescaling. Only the
 * lanes of one wave share an LDS slice, so the wave orders its own LDS
 * traffic (no workgroup barrier inside the walk).
 *   nsrk_attn_head_*:   one workgroup per query head, its waves taking every
 *                       W-th chunk, merged through LDS at the end: one launch,
 *                       no scratch.
 *   nsrk_attn_partial_*: one wave per (query head, split), (m, l, acc) to the
 *                       caller's partial buffer; nsrk_attn_reduce merges the
 *                       splits of a head.
 * HD4 = head_dim / 4 at compile time for the Moonshine sizes (36, 52, 64,
 * 128); 0 = any head_dim (multiple of 4, <= 128) at run time.
 */
#include "device_common.h"

#define NSR_ATT_MAXD 128

typedef _Float16 nsr_h2 __attribute__((ext_vector_type(2)));

template <int CTRL, int ROW_MASK>
NSR_DEV float dpp_max(float v) {
  /* lanes of rows outside ROW_MASK receive -inf (the `old` operand) */
  int t = __builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
  return fmaxf(v, __int_as_float(t));
}

/* Max over the 64 lanes (same DPP pattern as wave_sum), uniform result. */
NSR_DEV float wave_max(float v) {
  v = dpp_max<NSR_DPP_QUAD_1032, 0xF>(v);
  v = dpp_max<NSR_DPP_QUAD_2301, 0xF>(v);
  v = dpp_max<NSR_DPP_ROW_HALF_MIRROR, 0xF>(v);
  v = dpp_max<NSR_DPP_ROW_MIRROR, 0xF>(v);
  v = dpp_max<NSR_DPP_ROW_BCAST15, 0xA>(v);
  v = dpp_max<NSR_DPP_ROW_BCAST31, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* LDS of one wave: K and V rows [64][hd4 + 1] 8-byte pieces, probabilities
 * [64], P.V partials [64][4], the wave's copy of q (up to 32 pieces). */
NSR_DEV int attn_wave_lds_words(int hd4) { return 2 * 64 * (hd4 + 1) * 2 + 64 + 256 + 64; }

/* Orders this wave's LDS writes before its later LDS reads by other lanes
 * (one wave's LDS operations execute in order; this keeps the compiler from
 * moving them across). */
NSR_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* The online-softmax state of a wave: m, l (uniform), acc (lanes < hd4: dims
 * 4 lane .. 4 lane + 3). */
struct attn_state {
  float m, l, acc[4];
};

/* Walk the chunks c0 = first, first + stride, ... (< end) of query head qh
 * with this wave. The wave loads q itself, with its first chunk's K and V
 * (so the two latencies overlap and no workgroup barrier comes first), into
 * its own LDS slice. */
template <int HD4T>
NSR_DEV void attn_walk(const nsr_attn_args& a, int qh, int first, int end, int stride, uint32_t* wl,
                       attn_state& st) {
  const int lane = threadIdx.x & 63;
  const int hd4 = HD4T ? HD4T : (a.head_dim >> 2);
  constexpr int NU = HD4T ? HD4T : NSR_ATT_MAXD / 4; /* 8-byte pieces per lane per row set */
  /* the K/V head of this query head, in 32-bit arithmetic (head counts are small) */
  const int kvh = a.n_kv_heads == a.n_q_heads
                      ? qh
                      : (int)((uint32_t)qh * (uint32_t)a.n_kv_heads / (uint32_t)a.n_q_heads);
  const uint16_t* kb = a.k + (int64_t)kvh * a.stride_kv_head;
  const uint16_t* vb = a.v + (int64_t)kvh * a.stride_kv_head;
  uint2* kl = (uint2*)wl;
  uint2* vl = kl + 64 * (hd4 + 1);
  float* pl = (float*)(vl + 64 * (hd4 + 1));
  float* red = pl + 64;
  uint2* ql = (uint2*)(red + 256);
  /* P.V lane layout: 4 dimensions 4 dq .. 4 dq + 3, position group pg of ng */
  const int dq = lane % hd4, pg = lane / hd4, ng = 64 / hd4;
  const bool pv_lane = pg < ng;

  for (int c0 = first; c0 < end; c0 += stride) {
    const int n = min(64, end - c0);
    uint2 qv = {0u, 0u};
    if (c0 == first && lane < hd4) qv = *(const uint2*)(a.q + (int64_t)qh * a.head_dim + 4 * lane);
    /* in batches of NB pieces (all of them for the compile-time sizes; 8 at a
     * time for the run-time size, whose registers would not hold 2 x 32) */
    constexpr int NB = HD4T ? NU : 8;
#pragma unroll
    for (int ub = 0; ub < NU; ub += NB) {
      if (!HD4T && ub >= hd4) break;
      uint2 kv[NB], vv[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int e = lane + 64 * (ub + u), r = min(e / hd4, n - 1), c = e - (e / hd4) * hd4;
        const int64_t off = (int64_t)(c0 + r) * a.stride_kv_seq + 4 * c;
        kv[u] = *(const uint2*)(kb + off);
        vv[u] = *(const uint2*)(vb + off);
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int e = lane + 64 * (ub + u), r = e / hd4;
        if (HD4T || ub + u < hd4) {
          kl[r * (hd4 + 1) + (e - r * hd4)] = kv[u];
          vl[r * (hd4 + 1) + (e - r * hd4)] = vv[u];
        }
      }
    }
    if (c0 == first && lane < hd4) ql[lane] = qv;
    wave_lds_sync();
    float sc = -INFINITY;
    {
      const uint2* kr = kl + min(lane, n - 1) * (hd4 + 1);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        if (HD4T || i < hd4) {
          const uint2 kk = kr[i], qq = ql[i];
          d = __builtin_amdgcn_fdot2(__builtin_bit_cast(nsr_h2, kk.x), __builtin_bit_cast(nsr_h2, qq.x), d, false);
          d = __builtin_amdgcn_fdot2(__builtin_bit_cast(nsr_h2, kk.y), __builtin_bit_cast(nsr_h2, qq.y), d, false);
        }
      }
      if (lane < n) sc = d * a.sm_scale;
    }
    const float mc = wave_max(sc);
    const float mn = fmaxf(st.m, mc);
    const float alpha = __expf(st.m - mn); /* 0 on the first chunk (m = -inf) */
    const float p = lane < n ? __expf(sc - mn) : 0.f;
    st.l = st.l * alpha + wave_sum(p);
    st.m = mn;
    pl[lane] = p;
    wave_lds_sync();
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    auto pv_step = [&](int j) {
      const uint2 vv = vl[j * (hd4 + 1) + dq];
      const float pj = pl[j];
      const nsr_h2 v01 = __builtin_bit_cast(nsr_h2, vv.x), v23 = __builtin_bit_cast(nsr_h2, vv.y);
      part[0] = __builtin_fmaf(pj, (float)v01.x, part[0]);
      part[1] = __builtin_fmaf(pj, (float)v01.y, part[1]);
      part[2] = __builtin_fmaf(pj, (float)v23.x, part[2]);
      part[3] = __builtin_fmaf(pj, (float)v23.y, part[3]);
    };
    if (pv_lane) {
      if constexpr (HD4T != 0) {
        /* every row of the chunk, all reads in flight at once: rows past n hold row n - 1's values (the
         * staging clamps) and probability 0 */
        constexpr int NG = 64 / HD4T; /* ng at compile time */
#pragma unroll
        for (int jj = 0; jj < (64 + NG - 1) / NG; ++jj) {
          const int j = pg + jj * NG;
          if (jj * NG + NG <= 64 || j < 64) pv_step(j);
        }
      } else {
#pragma unroll 4
        for (int j = pg; j < n; j += ng) pv_step(j);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) red[lane * 4 + e] = part[e];
    wave_lds_sync();
    if (lane < hd4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float s = 0.f;
        for (int g = 0; g < ng; ++g) s += red[(g * hd4 + lane) * 4 + e];
        st.acc[e] = st.acc[e] * alpha + s;
      }
    }
    wave_lds_sync(); /* this chunk's LDS reads are done before the next chunk's writes */
  }
}

/* Split: one wave per (query head, split) -> partial [m, l, acc[hd]]. */
template <int HD4T>
NSR_DEV void attn_partial(const nsr_attn_args& a) {
  extern __shared__ uint32_t att_lds[];
  const int lane = threadIdx.x;
  const uint32_t ns = (uint32_t)a.n_splits, qh32 = blockIdx.x / ns;
  const int qh = (int)qh32, sp = (int)(blockIdx.x - qh32 * ns);
  const int hd = a.head_dim, hd4 = hd >> 2;
  const int p0 = sp * a.kv_per_split, p1 = min(p0 + a.kv_per_split, a.kv_len);
  attn_state st = {-INFINITY, 0.f, {0.f, 0.f, 0.f, 0.f}};
  attn_walk<HD4T>(a, qh, p0, p1, 64, att_lds, st);
  float* po = a.partial + (int64_t)blockIdx.x * (hd + 2);
  if (lane == 0) {
    po[0] = st.m; /* -inf and l = 0 for an empty split */
    po[1] = st.l;
  }
  if (lane < hd4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) po[2 + 4 * lane + e] = st.acc[e];
  }
}

/* One workgroup (W waves) per query head; wave w takes chunks w, w + W, ... */
template <int HD4T>
NSR_DEV void attn_head(const nsr_attn_args& a) {
  extern __shared__ uint32_t att_lds[];
  __shared__ float ms[16], ls[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int qh = blockIdx.x;
  const int hd = a.head_dim, hd4 = hd >> 2;
  uint32_t* wl = att_lds + w * attn_wave_lds_words(hd4);
  attn_state st = {-INFINITY, 0.f, {0.f, 0.f, 0.f, 0.f}};
  attn_walk<HD4T>(a, qh, 64 * w, a.kv_len, 64 * W, wl, st);
  /* merge the waves: (m, l) and the acc rows through LDS (acc in the wave's
   * own K slice, free now) */
  float* accl = (float*)wl;
  if (lane == 0) {
    ms[w] = st.m;
    ls[w] = st.l;
  }
  if (lane < hd4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) accl[4 * lane + e] = st.acc[e];
  }
  __syncthreads();
  if (w == 0) {
    /* lane i < W holds wave i's m and l; every wave's acc row is read at once (rows past W read wave W - 1's
     * with weight 0), then added in wave order: one round of LDS reads instead of a dependent one per wave */
    const float mi = lane < W ? ms[lane] : -INFINITY;
    const float m = wave_max(mi);
    const float wi = lane < W ? __expf(mi - m) : 0.f; /* 0 for a wave that had no chunk (m = -inf) */
    const float li = lane < W ? ls[lane] : 0.f;
    float rows[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float* ai = (const float*)(att_lds + min(i, W - 1) * attn_wave_lds_words(hd4));
#pragma unroll
      for (int e = 0; e < 4; ++e) rows[i][e] = lane < hd4 ? ai[4 * lane + e] : 0.f;
    }
    float l = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float wt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wi), i));
      l = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(li), i)), wt, l);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(rows[i][e], wt, acc[e]);
    }
    if (lane < hd4) {
      uint16_t* o = a.out + (int64_t)qh * hd + 4 * lane;
      const uint32_t w0 = f32_to_f16_bits(acc[0] / l) | (f32_to_f16_bits(acc[1] / l) << 16);
      const uint32_t w1 = f32_to_f16_bits(acc[2] / l) | (f32_to_f16_bits(acc[3] / l) << 16);
      if (((uintptr_t)a.out & 7u) == 0) {
        *(uint2*)o = make_uint2(w0, w1);
      } else {
        o[0] = (uint16_t)w0;
        o[1] = (uint16_t)(w0 >> 16);
        o[2] = (uint16_t)w1;
        o[3] = (uint16_t)(w1 >> 16);
      }
    }
  }
}

#define NSR_ATTN(HD4)                                                                                  \
  extern "C" __global__ void __launch_bounds__(64) nsrk_attn_partial_d##HD4(const nsr_attn_args a) {   \
    attn_partial<HD4>(a);                                                                             \
  }                                                                                                   \
  extern "C" __global__ void __launch_bounds__(512) nsrk_attn_head_d##HD4(const nsr_attn_args a) {     \
    attn_head<HD4>(a);                                                                                \
  }

NSR_ATTN(0)
NSR_ATTN(9)
NSR_ATTN(13)
NSR_ATTN(16)
NSR_ATTN(32)

/* One workgroup per query head, one lane per dimension (hd <= 128). Up to 32
 * splits are read in one round, more 16 at a time, with all of a round's
 * loads in flight (indices clamped, the extras weighted 0): a loop of
 * dependent loads would pay one memory latency per split. */
extern "C" __global__ void __launch_bounds__(128) nsrk_attn_reduce(const nsr_attn_args a) {
  const int qh = blockIdx.x, d = threadIdx.x;
  const int hd = a.head_dim, ns = a.n_splits, st = hd + 2;
  const int dc = min(d, hd - 1);
  const float* pb = a.partial + (int64_t)qh * ns * st;
  if (ns <= 32) {
    /* up to 32 splits (the decoder's cross-attention takes 32): lane u loads split u's m and l, every lane the
     * 32 acc values of its dimension, all in flight at once (one memory latency for the whole merge); the max,
     * the weights and the sums in split order are those of the loop below */
    const int lane = threadIdx.x & 63;
    const float* pu = pb + (int64_t)min(lane, ns - 1) * st;
    const float mu = lane < ns ? pu[0] : -INFINITY;
    const float lu = lane < ns ? pu[1] : 0.f;
    float av[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) av[u] = pb[(int64_t)min(u, ns - 1) * st + 2 + dc];
    __builtin_amdgcn_sched_barrier(0); /* every load issued before the max waits for m */
    const float m = wave_max(mu);
    const float wu = lane < ns ? __expf(mu - m) : 0.f; /* 0 for empty splits (m_s = -inf) */
    float l = 0.f, acc = 0.f;
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wu), u));
      l = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(lu), u)), w, l);
      acc = __builtin_fmaf(av[u], w, acc);
    }
    if (d < hd) a.out[(int64_t)qh * hd + d] = (uint16_t)f32_to_f16_bits(acc / l);
    return;
  }
  float m = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += 16) {
    float mv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) mv[u] = pb[(int64_t)min(s0 + u, ns - 1) * st];
#pragma unroll
    for (int u = 0; u < 16; ++u) m = fmaxf(m, mv[u]);
  }
  float l = 0.f, acc = 0.f;
  for (int s0 = 0; s0 < ns; s0 += 16) {
    float mv[16], lv[16], av[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float* ps = pb + (int64_t)min(s0 + u, ns - 1) * st;
      mv[u] = ps[0];
      lv[u] = ps[1];
      av[u] = ps[2 + dc];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float w = s0 + u < ns ? __expf(mv[u] - m) : 0.f; /* 0 for empty splits (m_s = -inf) */
      l = __builtin_fmaf(lv[u], w, l);
      acc = __builtin_fmaf(av[u], w, acc);
    }
  }
  if (d < hd) a.out[(int64_t)qh * hd + d] = (uint16_t)f32_to_f16_bits(acc / l);
}
