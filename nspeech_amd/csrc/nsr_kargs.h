/*
 * Kernel argument blocks, shared by the host launcher (nsr_runtime.cpp) and
 * the gfx950 kernels (the .hip files under kernels/). Each kernel takes exactly one of these
 * structs by value, so hipModuleLaunchKernel gets a single kernelParams entry
 * and host and device agree on the layout by construction.
 * Plain C: no HIP or C++ types, fixed-width integers only.
 */
#ifndef NSR_KARGS_H
#define NSR_KARGS_H

#include <stdint.h>

#define NSR_MAX_HALF_ROT 128 /* rotary_dim <= 256 */

typedef struct nsr_q8_args {
  const uint8_t* blocks;   /* Q8_0 table, vocab rows of row_bytes */
  const void* ids;         /* n_ids ids, u32 or i64 */
  float* out;              /* [n_ids, d] */
  int32_t* err_flag;       /* may be NULL */
  int64_t vocab;
  int64_t n_ids;
  int64_t total4;          /* n_ids * d / 4 float4 outputs */
  int32_t d4;              /* d / 4 */
  int32_t row_bytes;       /* 34 * d / 32 */
  int32_t act;             /* nsr_act */
  int32_t ids_i64;         /* 1: ids are int64 */
  int32_t ipw;             /* ids per workgroup (whole rows per workgroup); 0: one flat grid */
  int32_t gw;              /* > 0: each id takes gw whole waves (wave-uniform id); 0: ids packed densely */
} nsr_q8_args;

typedef struct nsr_ln_args {
  const void* x;
  const void* res;         /* residual (fused variant) */
  void* h;                 /* x + res output, may be NULL */
  const void* gamma;       /* may be NULL */
  const void* beta;        /* may be NULL */
  void* y;
  int64_t n_rows;
  int64_t ld_x;            /* elements */
  int64_t ld_y;            /* elements */
  int32_t n_cols;
  int32_t unit_offset;     /* scale = gamma + 1 */
  float eps;
  float inv_n;             /* 1 / n_cols */
} nsr_ln_args;

typedef struct nsr_rope_args {
  const float* src[2];     /* q, k */
  float* dst[2];           /* q_out, k_out */
  const float* table;      /* [table_rows][2*half] cos..., sin... or NULL */
  int64_t rows[2];         /* B*Hq*T, B*Hk*T  (k rows 0 when k is NULL) */
  int64_t n4[2];           /* float4 count of q and k */
  int64_t pos0;
  int32_t T;
  int32_t dh4;             /* Dh / 4 */
  int32_t rot4;            /* rotary_dim / 4 */
  int32_t half;            /* rotary_dim / 2 */
  float inv_freq[NSR_MAX_HALF_ROT];
} nsr_rope_args;

typedef struct nsr_rope_cache_args {
  void* q;                 /* [Hq, Dh], rotated in place (may be NULL when nq == 0) */
  void* k;                 /* [Hk, Dh], rotated in place */
  const void* v;           /* [Hk, Dh] */
  const float* table;      /* RoPE table row pos: cos[half] then sin[half] */
  void* cache_k;           /* [Hk, max_kv_len, Dh] */
  void* cache_v;           /* [Hk, max_kv_len, Dh] */
  int64_t pos;
  int64_t max_kv_len;
  int32_t Dh;
  int32_t half;            /* rotary_dim / 2 */
  int32_t nq;              /* lanes (element pairs) of each region: q pairs, */
  int32_t nk;              /*   k pairs, */
  int32_t nkp;             /*   k pass-through pairs, */
  int32_t nv;              /*   v pairs */
} nsr_rope_cache_args;

typedef struct nsr_adain_args {
  const float* x;          /* [B, C, T] */
  const void* gamma;       /* [B?, C] */
  const void* beta;        /* [B?, C] */
  const void* alpha;       /* [C] */
  float* out;              /* [B, C, T] */
  float* stats;            /* [B*C][2] mean, rstd (nsrk_adain_stats* output only) */
  int64_t n_rows;          /* B * C */
  int64_t T;
  int64_t gamma_bstride;
  int64_t beta_bstride;
  int32_t C;
  int32_t lds_chunks;      /* float4 chunks per thread kept in LDS */
  float eps;
  float inv_t;             /* 1 / T */
  uint64_t* stamps;        /* [grid][NSR_ADAIN_TL_WORDS] timeline (nsrk_adain_row_tl_* only) */
} nsr_adain_args;

/* Timeline words per workgroup of nsrk_adain_row_tl_*: [0] XCD (HW_REG_XCC_ID), [1] start,
 * [2 + w] end of wave w's last store (w < 8), [10 + 8 r + w] when row r's data had landed for wave w
 * (r < 8). Times are s_memrealtime ticks (100 MHz). */
#define NSR_ADAIN_TL_WORDS 80

typedef struct nsr_adain_h_args {
  const uint16_t* x;       /* [B, C, T] f16 */
  const void* gamma;       /* [B?, C] */
  const void* beta;        /* [B?, C] */
  const void* alpha;       /* [C] */
  uint16_t* out;           /* [B, C, T] f16 */
  int64_t n_rows;          /* B * C */
  int64_t T;
  int64_t gamma_bstride;
  int64_t beta_bstride;
  int32_t C;
  float eps;
  float inv_t;             /* 1 / T */
  int32_t pad_;
} nsr_adain_h_args;

typedef struct nsr_gemv_args {
  const void* x;           /* [K], f16 or f32 */
  const uint32_t* qs;      /* weights: repacked Q8 [K, NW/4] words, or t4 tiles */
  const uint16_t* scales;  /* f16: [K/32, NW], or t4 tiles [NW/4][K/32][4] */
  const float* bias;       /* [NW] or NULL */
  void* out;               /* [N] */
  const float* residual;   /* [N] (h form) */
  float* out_f32;          /* [N] h = f16(x @ W) + residual (h form) */
  int32_t K;
  int32_t NW;              /* weight columns: N, or 2N for the GLU form */
  int32_t N;               /* output columns */
  int32_t n_tiles;         /* reference layout: 8-column tiles (x-half tiles for the GLU form) */
  int32_t line_groups;     /* reference layout: 1 = each 16-tile line group on one XCD, 0 = contiguous runs */
  int32_t pad_;
} nsr_gemv_args;

typedef struct nsr_q8_pack_args {
  const uint8_t* qs;       /* [K, NW] int8 bytes (the repacked Q8 words, little-endian) */
  const uint16_t* scales;  /* [K/32, NW] f16 */
  uint32_t* tq;            /* [NW/4][K] words: tile t, row r = 4 int8 */
  uint16_t* ts;            /* [NW/4][K/32][4] f16 */
  int32_t K;
  int32_t NW;
  int32_t N;               /* GLU: output columns (NW = 2N); 0 = plain */
  int32_t pad_;
} nsr_q8_pack_args;

typedef struct nsr_q8_0_conv_args {
  const uint8_t* blocks;   /* GGUF Q8_0 weight [N rows][K/32 blocks] of {f16 d; int8 qs[32]} */
  uint32_t* qs;            /* repacked [K, N/4] words, or t4 tiles [N/4][K] */
  uint16_t* scales;        /* repacked [K/32, N], or t4 [N/4][K/32][4] */
  int32_t N;
  int32_t K;
  int32_t t4;              /* 0: repacked layout, 1: t4 tiles */
  int32_t glu_n;           /* t4 GLU: output columns (N = 2 glu_n); 0 = plain */
} nsr_q8_0_conv_args;

typedef struct nsr_attn_args {
  const uint16_t* q;       /* f16 [n_q_heads, head_dim] */
  const uint16_t* k;       /* f16, element (head, pos, d) at head*stride_kv_head + pos*stride_kv_seq + d */
  const uint16_t* v;       /* same layout as k */
  float* partial;          /* f32 [n_q_heads * n_splits][head_dim + 2]: m, l, acc[head_dim] */
  uint16_t* out;           /* f16 [n_q_heads, head_dim] */
  int64_t stride_kv_head;  /* elements */
  int64_t stride_kv_seq;   /* elements */
  int32_t kv_len, n_q_heads, n_kv_heads, head_dim, n_splits, kv_per_split;
  float sm_scale;
  int32_t pad_;
} nsr_attn_args;

typedef struct nsr_conv_args {
  const float* x;          /* [B, C_in, T_in] */
  const uint16_t* w;       /* packed f16 [C_out][K][C_in] */
  const uint16_t* bias;    /* f16 [C_out] or NULL */
  const float* residual;   /* [B, C_out, T_out] or NULL */
  float* out;              /* [B, C_out, T_out] */
  const float* stats;      /* [B*C_in][2] mean, rstd (AdaIN+Snake input) */
  const void* gamma;       /* AdaIN+Snake parameters, as nsr_adain_args */
  const void* beta;
  const void* alpha;
  int64_t gamma_bstride;
  int64_t beta_bstride;
  int32_t B, C_in, C_out, T_in, T_out, K, padding, dilation, pdt;
  int32_t pad_;            /* bit 0: 16-byte epilogue stores allowed */
  float* row_part;         /* STATS kernels: [B*C_out][ceil(T_out/32)][2] (mean, M2) of out */
} nsr_conv_args;

typedef struct nsr_rowstats_args {
  const float* part;       /* [rows][nblk][2] (mean, M2) of 32-column blocks */
  float* stats;            /* [rows][2] mean, 1 / sqrt(var + eps) */
  int32_t nblk;
  int32_t T_out;           /* block i holds min(32, T_out - 32 i) columns */
  float eps;
  int32_t pad_;
} nsr_rowstats_args;

typedef struct nsr_conv_pack_args {
  const uint16_t* w;       /* f16 [C_out][C_in][K] */
  uint16_t* wp;            /* f16 [C_out][K][C_in] */
  int64_t C_out, C_in, K;
} nsr_conv_pack_args;

/* out = lrelu?(((a + b) + c) * scale), b / c optional (NULL), f32 */
typedef struct nsr_combine_args {
  const float* a;
  const float* b;          /* or NULL */
  const float* c;          /* or NULL */
  float* out;
  int64_t n;
  float scale;             /* applied when flags bit 0 */
  float slope;             /* leaky ReLU slope, applied when flags bit 1 */
  int32_t flags;
  int32_t pad_;
} nsr_combine_args;

typedef struct nsr_snake_args {
  const void* x;           /* [rows, T], f32 or f16 */
  const void* alpha;       /* [C], f32 or f16 (pdt) */
  void* out;               /* like x */
  int64_t T;
  int64_t chunks;          /* 1024-element chunks per row */
  int32_t C;               /* channel of a row = row % C */
  int32_t pdt;
} nsr_snake_args;

typedef struct nsr_istft_args {
  const float* x;          /* [2 * bins, n_frames]: log-magnitudes, then raw phases (phase = sin(raw)) */
  float* out;              /* [out_len], centre padding (n_fft / 2 each side) removed */
  int64_t n_frames;
  int64_t out_len;
  int32_t n_fft, hop, frames_per_group, pad_;
} nsr_istft_args;

typedef struct nsr_ew_args {
  const void* a;
  const void* b;
  void* out;
  int64_t n;               /* elements (GLU: output elements) */
  int32_t act;
  int32_t pad_;
} nsr_ew_args;

/* plain device copy of n4 16-byte chunks (measurement floor) */
typedef struct nsr_calib_args {
  const float* src;
  float* dst;
  int64_t n4;
} nsr_calib_args;

#endif /* NSR_KARGS_H */
