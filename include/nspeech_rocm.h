/*
 * nspeech_rocm.h — C ABI of the MI355X (gfx950) fused layer kernels.
 *
 * Drop-in boundary for nspeech's GPU kernel dispatch layer. Every entry point
 * below names the reference interface it replaces (paths relative to the
 * dropbox/nspeech source tree). The reference binds its kernels from Rust
 * (src/triton_kernels.rs, src/kokoro/gpu_backend.rs); a Rust `rocm` feature
 * binds these symbols with plain `extern "C"` declarations.
 *
 * Conventions (mirroring src/triton_kernels.rs):
 *   - All tensor arguments are DEVICE pointers, caller-owned, contiguous,
 *     row-major. Outputs are written, never allocated (the reference's
 *     `out: &Tensor` / `enc_*` style, triton_kernels.rs:598,713,742,862-1423).
 *   - Launches are asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream). Nothing here synchronises, except where noted.
 *   - Every function returns nsr_status. On failure nothing is launched and
 *     nsr_last_error() returns a message (thread-local), the equivalent of the
 *     reference's anyhow::bail! (triton_kernels.rs:138).
 *   - Kernels come from precompiled gfx950 code objects (one per kernel
 *     unit), embedded in the library and loaded with hipModuleLoadData on
 *     first use per device (or from files named by nsr_init). Module handles
 *     are immutable after load; the launch functions are thread-safe.
 */
#ifndef NSPEECH_ROCM_H
#define NSPEECH_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum nsr_status {
  NSR_OK = 0,
  NSR_ERR_BAD_ARG = 1,     /* null pointer, bad shape, misaligned, ... */
  NSR_ERR_NOT_INIT = 2,    /* code object could not be loaded */
  NSR_ERR_HIP = 3,         /* a HIP runtime call failed (message has hipGetErrorString) */
  NSR_ERR_UNSUPPORTED = 4  /* valid request this build does not implement */
} nsr_status;

typedef enum nsr_dtype {
  NSR_F32 = 0,
  NSR_F16 = 1,
  NSR_BF16 = 2
} nsr_dtype;

typedef enum nsr_index_dtype {
  NSR_IDX_U32 = 0,
  NSR_IDX_I64 = 1
} nsr_index_dtype;

/* Epilogue activation applied to a kernel's main output. */
typedef enum nsr_act {
  NSR_ACT_NONE = 0,
  NSR_ACT_SILU = 1,      /* x / (1 + exp(-x))          candle silu */
  NSR_ACT_GELU_ERF = 2   /* x * 0.5 * (1 + erf(x/√2))  candle gelu_erf */
} nsr_act;

/* LayerNorm flags. */
#define NSR_LN_UNIT_OFFSET 1u /* scale = gamma + 1 (moonshine/encoder.rs:68-76) */

typedef void* nsr_stream_t; /* hipStream_t */

/* ---- library ------------------------------------------------------------ */

/* Version string of this library. */
const char* nsr_version(void);

/* Load the gfx950 code objects on the current device. code_object_dir ==
 * NULL uses the code objects embedded in the library; otherwise the directory
 * holding nsr_<unit>_gfx950.hsaco files. Calling it is optional: every launch
 * loads the embedded objects on first use on a device. The first call on a
 * device decides; later calls only report its status.
 * Replaces TritonKernels::load / DecoderKernels::load / KokoroKernels::load
 * (kernels/out/generated/triton_metal_gen.rs:39-106) and load_kernel_pipeline
 * (src/triton_kernels.rs:1401). */
nsr_status nsr_init(const char* code_object_dir);

/* Message describing the last failure on this thread ("" if none). */
const char* nsr_last_error(void);

/* Number of kernels resolved for the current device (0 if its code objects
 * are not loaded): every kernel the library launches is resolved once, when
 * the device's code objects load. Used by tests to check the set is complete. */
int nsr_kernel_count(void);

/* ---- LayerNorm family ---------------------------------------------------- */

/* y[r, :] = act( (x[r,:] - mean) / sqrt(var + eps) * scale + beta )
 *   scale = gamma (or gamma + 1 with NSR_LN_UNIT_OFFSET, or 1 if gamma NULL),
 *   beta NULL = 0. Mean and biased variance over the row, two-pass, fp32.
 * x_dtype/y_dtype: F32, F16 or BF16; gamma/beta: F32 or F16 (param_dtype).
 * ld_x / ld_y: row strides in elements (>= n_cols).
 * Replaces: candle_nn::LayerNorm::forward as configured at
 *   src/parakeet/fast_conformer.rs:721-725,778-782 (f32, affine);
 *   UnitOffsetLayerNorm::forward src/moonshine/encoder.rs:68-76;
 *   LayerNorm::forward (weight only) src/moonshine/decoder.rs:67-74;
 *   triton_layernorm_unit_offset src/triton_kernels.rs:312,
 *   triton_layernorm_bare :345, triton_layernorm_std_f32in :598,
 *   enc_layernorm_std_f32in :880, enc_layernorm_bare :1291,
 *   enc_layernorm_unit_offset :1309. */
nsr_status nsr_layernorm(const void* x, nsr_dtype x_dtype,
                         const void* gamma, const void* beta, nsr_dtype param_dtype,
                         void* y, nsr_dtype y_dtype,
                         int64_t n_rows, int64_t n_cols, int64_t ld_x, int64_t ld_y,
                         float eps, unsigned flags, nsr_act act,
                         nsr_stream_t stream);

/* Fused residual add + LayerNorm (+ activation):
 *   h = x + res            (rounded to h_dtype; written to h_out unless NULL)
 *   y = act(LN(h) * scale + beta)
 * LN statistics are taken over the ROUNDED h, exactly as an unfused
 * add -> store -> LayerNorm chain would see it. Row stride = n_cols.
 * Replaces residual_add_layernorm_fused (kernels/moonshine_kernels.py:955-991)
 * dispatched by triton_residual_add_layernorm src/triton_kernels.rs:742 and
 * enc_residual_add_layernorm :1012; and the CPU chain fast_add
 * (src/fast_ops.rs:41-47) followed by LayerNorm and gelu_erf
 * (src/moonshine/encoder.rs:106). */
nsr_status nsr_residual_add_layernorm(const void* x, nsr_dtype x_dtype,
                                      const void* res, nsr_dtype res_dtype,
                                      void* h_out, nsr_dtype h_dtype,
                                      const void* gamma, const void* beta,
                                      nsr_dtype param_dtype,
                                      void* y, nsr_dtype y_dtype,
                                      int64_t n_rows, int64_t n_cols, float eps,
                                      unsigned flags, nsr_act act,
                                      nsr_stream_t stream);

/* ---- Partial interleaved rotary ----------------------------------------- */

/* Host-side (no GPU work): fill table[max_pos][2*half] (half = rotary_dim/2)
 * with cos (first half) then sin (second half) of pos * inv_freq[i],
 * inv_freq[i] = 1 / theta^(2i/rotary_dim), all in f32 exactly as
 * src/moonshine/gpu_decoder.rs:326-340 builds its RoPE table. */
nsr_status nsr_rope_table_f32(float* host_table, int64_t max_pos, int rotary_dim,
                              float theta);

/* Out-of-place (or in-place when q_out == q) partial interleaved rotary over
 * q [B, Hq, T, Dh] and k [B, Hk, T, Dh] (k may be NULL):
 *   for pair i < rotary_dim/2 at position p = pos0 + t:
 *     o[2i]   = x[2i]*cos(p*f_i) - x[2i+1]*sin(p*f_i)
 *     o[2i+1] = x[2i+1]*cos(p*f_i) + x[2i]*sin(p*f_i)
 *   dims >= rotary_dim are copied unchanged.
 * rope_table: NULL = cos/sin computed in-kernel from theta (f32 angle, as the
 * reference); otherwise a DEVICE table laid out as nsr_rope_table_f32 writes,
 * with at least pos0 + T rows (table_rows).
 * Replaces apply_rotary_pos_emb + RotaryEmbedding::forward
 * (src/moonshine/decoder.rs:85-183) and the rope part of
 * enc_rope_qk_cache_fused (src/triton_kernels.rs:975). */
nsr_status nsr_rotary_partial_interleaved_f32(const float* q, const float* k,
                                              float* q_out, float* k_out,
                                              int64_t B, int64_t Hq, int64_t Hk,
                                              int64_t T, int64_t Dh, int rotary_dim,
                                              float theta, int64_t pos0,
                                              const float* rope_table,
                                              int64_t table_rows,
                                              nsr_stream_t stream);

/* Decode step, one position: rotate q [n_q_heads, head_dim] and k
 * [n_kv_heads, head_dim] IN PLACE on the interleaved pairs < rotary_dim with
 * row `pos` of a DEVICE RoPE table (layout of nsr_rope_table_f32, at least
 * pos + 1 rows), write the rotated k row to cache_k[h, pos, :] and, when v is
 * given, the v row to cache_v[h, pos, :]. Caches are [n_kv_heads,
 * max_kv_len, head_dim]. dtype F16 (the reference decoder's) or F32; each
 * rotated value is rounded to dtype from f32 products. head_dim and
 * rotary_dim even; q/k/v/caches 4-byte (F16) or 8-byte (F32) aligned.
 * One launch replaces the reference's two dispatches per layer and token:
 * enc_rope_qk_cache_fused (src/triton_kernels.rs:975;
 * kernels/moonshine_kernels.py:1372-1454) and enc_kv_cache_append (:993;
 * moonshine_kernels.py:865-883), issued together by
 * MetalBackend::rope_kv_cache (src/moonshine/gpu_decoder_metal.rs:144-156).
 * v == NULL (and cache_v == NULL) is exactly enc_rope_qk_cache_fused. */
nsr_status nsr_rope_qk_cache_append(void* q, void* k, const void* v, nsr_dtype dtype,
                                    const float* rope_table, int64_t table_rows,
                                    void* cache_k, void* cache_v,
                                    int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim,
                                    int rotary_dim, int64_t pos, int64_t max_kv_len,
                                    nsr_stream_t stream);

/* cache[h, pos, :] = new_kv[h, :] for h < n_kv_heads; cache [n_kv_heads,
 * max_kv_len, head_dim], head_dim even, dtype F16 or F32.
 * Replaces enc_kv_cache_append (src/triton_kernels.rs:993) and
 * triton_kv_cache_append (:680); kernels/moonshine_kernels.py:865-883. */
nsr_status nsr_kv_cache_append(const void* new_kv, void* cache, nsr_dtype dtype,
                               int64_t n_kv_heads, int64_t head_dim, int64_t max_kv_len,
                               int64_t pos, nsr_stream_t stream);

/* ---- AdaIN1d + Snake ------------------------------------------------------ */

/* For x [B, C, T] f32, per (b, c) row:
 *   mean, var = biased statistics over T
 *   y   = (1 + gamma[b,c]) * (x - mean) / sqrt(var + eps) + beta[b,c]
 *   out = y + sin(alpha[c]*y)^2 * (1 / (alpha[c] + 1e-9))
 * gamma/beta/alpha have param_dtype F32 or F16. gamma_bstride/beta_bstride:
 * elements between batches of gamma/beta (0 = shared over the batch, C =
 * per batch). alpha is per channel [C].
 * While a row fits on chip (16-byte aligned rows up to T = 118784, other rows
 * up to about 65k elements) x is read from HBM once and the statistics are
 * two passes over the on-chip row in f32 (the mean, then centred sums that
 * also correct the mean). Longer rows take a kernel that reads each row
 * twice (f64 sums, then the output; no scratch memory).
 * Replaces adain (src/kokoro/decoder.rs:1416-1428) followed by
 * snake_activation_tensor (:1471-1476), and
 * KokoroGpuBackend::adain_snake_f32 (src/kokoro/gpu_backend.rs:181-185,
 * Metal impl src/kokoro/gpu_decoder.rs:886-950). */
nsr_status nsr_adain_snake_f32(const float* x, const void* gamma, const void* beta,
                               const void* alpha, nsr_dtype param_dtype,
                               int64_t gamma_bstride, int64_t beta_bstride,
                               float* out, int64_t B, int64_t C, int64_t T,
                               float eps, nsr_stream_t stream);

/* The same with f16 activations: x and out [B, C, T] f16 (f32 arithmetic,
 * out rounded to nearest even). Any row start: x and out 2-byte aligned with
 * the same offset within 16 bytes (two fresh allocations qualify); T up to
 * 131072. Replaces KokoroGpuBackend::adain_snake (src/kokoro/gpu_backend.rs:
 * 55-57; Metal impl src/kokoro/gpu_decoder.rs:563-588 over the Triton
 * adain_snake_fused / adain_snake_looped, kernels/kokoro_kernels.py:222-331),
 * which the decoder's resblocks call when the backend keeps f16
 * intermediates (src/kokoro/decoder.rs:1009, 1035). */
nsr_status nsr_adain_snake_f16(const void* x, const void* gamma, const void* beta,
                               const void* alpha, nsr_dtype param_dtype,
                               int64_t gamma_bstride, int64_t beta_bstride,
                               void* out, int64_t B, int64_t C, int64_t T,
                               float eps, nsr_stream_t stream);

/* ---- GGUF Q8_0 embedding gather-dequant ----------------------------------- */

/* blocks: the GGUF Q8_0 table, vocab rows of d/32 blocks of 34 bytes
 * ({f16 d; int8 qs[32]}), row stride 34*d/32 bytes (2-byte aligned rows are
 * fine). ids: n_ids token ids (U32 or I64). out[n, j] = act(qs * d) as f32.
 * An id >= vocab (or < 0) writes a zero row and, when err_flag is not NULL,
 * stores 1 to *err_flag (device int32); the reference's index_select fails
 * on such ids instead.
 * Replaces QEmbedding::forward (src/parakeet/quantized_layers.rs:65-71:
 * QTensor::dequantize of the whole table, then index_select) and the
 * dequantized-table lookups of src/moonshine/decoder.rs:508-515,569 and
 * src/moonshine/gpu_decoder.rs:244-248,474-477; act = NSR_ACT_SILU fuses the
 * following silu (src/parakeet/fast_conformer.rs:207). */
nsr_status nsr_q8_0_embed_gather(const void* blocks, int64_t vocab, int64_t d,
                                 const void* ids, nsr_index_dtype id_dtype,
                                 int64_t n_ids, float* out, nsr_act act,
                                 int32_t* err_flag, nsr_stream_t stream);

/* ---- Elementwise ----------------------------------------------------------- */

/* y = act(x) elementwise (act SILU or GELU_ERF); dtype F32, F16 or BF16
 * (computed in f32). Replaces triton_gelu src/triton_kernels.rs:412 /
 * enc_gelu :1328 (kernels/moonshine_kernels.py:388-400), Tensor::gelu_erf
 * (src/moonshine/encoder.rs:106), candle_nn::ops::silu
 * (src/moonshine/decoder.rs:409, src/parakeet/fast_conformer.rs:207,574) and
 * silu_forward (kernels/moonshine_kernels.py:473-485). */
nsr_status nsr_activation(const void* x, void* y, nsr_dtype dtype, int64_t n,
                          nsr_act act, nsr_stream_t stream);

/* out[i] = silu(fc1[n + i]) * fc1[i] for i < n (fc1 holds 2n elements:
 * x part first, gate second). Replaces triton_glu_silu
 * src/triton_kernels.rs:713 (glu_silu_fused, kernels/moonshine_kernels.py:846-862)
 * and the GLU of DecoderMLP::forward src/moonshine/decoder.rs:403-411. */
nsr_status nsr_glu_silu(const void* fc1, void* out, nsr_dtype dtype, int64_t n,
                        nsr_stream_t stream);

/* out = x + res elementwise (same dtype). Replaces fast_add
 * (src/fast_ops.rs:16-47), triton_residual_add src/triton_kernels.rs:383 and
 * enc_residual_add :1340. */
nsr_status nsr_residual_add(const void* x, const void* res, void* out,
                            nsr_dtype dtype, int64_t n, nsr_stream_t stream);

/* ---- Kokoro generator tail (f32) --------------------------------------------- */

/* out = x * s. With s = 1/3 (the f32 nearest it): KokoroGpuBackend::
 * scale_third_f32 (src/kokoro/gpu_backend.rs:193-195; kernels/
 * kokoro_kernels.py:957-969); also the backend's `scale` (:39). */
nsr_status nsr_scale_f32(const float* x, float* out, int64_t n, float s, nsr_stream_t stream);

/* out = x > 0 ? x : x * slope. KokoroGpuBackend::leaky_relu_f32
 * (src/kokoro/gpu_backend.rs:197-200; conv_post input, src/kokoro/
 * decoder.rs:574-575). */
nsr_status nsr_leaky_relu_f32(const float* x, float* out, int64_t n, float slope, nsr_stream_t stream);

/* The generator's average of its three resblocks, in one pass:
 *   out = ((r0 + r1) + r2) * f32(1/3), then, if leaky_relu != 0,
 *   out = out > 0 ? out : out * slope
 * with the rounding sequence of the reference GPU path's add_f32, add_f32,
 * scale_third_f32 (and leaky_relu_f32 before conv_post) dispatches
 * (src/kokoro/decoder.rs:540-546, 574-575). The residual add alone
 * (KokoroGpuBackend::add_f32, :186-190) is nsr_residual_add with NSR_F32.
 * No counterpart fuses these in the reference. */
nsr_status nsr_resblock_average_f32(const float* r0, const float* r1, const float* r2, float* out, int64_t n,
                                    int leaky_relu, float slope, nsr_stream_t stream);

/* Snake alone: out = x + sin^2(alpha_c x) * (1 / (alpha_c + 1e-9)) for x
 * [rows, seq_len] (n_elements = rows * seq_len), row r in channel
 * r % channels; x/out F32 or F16 (f32 arithmetic), alpha [channels] F32 or
 * F16. Replaces KokoroGpuBackend::snake (src/kokoro/gpu_backend.rs:51-52;
 * Metal impl src/kokoro/gpu_decoder.rs:545-561 over snake_activation,
 * kernels/kokoro_kernels.py:24-55) and snake_activation_tensor
 * (src/kokoro/decoder.rs:1471-1476). */
nsr_status nsr_snake(const void* x, nsr_dtype dtype, const void* alpha, nsr_dtype alpha_dtype, void* out,
                     int64_t n_elements, int64_t channels, int64_t seq_len, nsr_stream_t stream);

/* Inverse STFT of conv_post's output x [2 (n_fft / 2 + 1), n_frames] f32
 * (log-magnitudes, then raw phases): magnitude exp(x), phase sin(x), one-
 * sided iDFT, periodic Hann window, overlap-add, division by the window-
 * square sum (0 where it is <= 1e-8), n_fft / 2 samples of centre padding
 * removed: out [out_len], out_len <= (n_frames - 1) hop (the decoder asks
 * for exactly that). n_fft 16, 20 or 32 (others: NSR_ERR_UNSUPPORTED), a
 * multiple of hop (Kokoro: 20, 5).
 * Replaces KokoroGpuBackend::istft_gpu (src/kokoro/gpu_backend.rs:220-225;
 * Metal istft_fused, kernels/kokoro_kernels.py:1097-1183) and the CPU
 * exp / sin / istft of src/kokoro/decoder.rs:606-612, 1546-1632. */
nsr_status nsr_istft_f32(const float* x, float* out, int64_t n_frames, int64_t out_len, int n_fft, int hop,
                         nsr_stream_t stream);

/* ---- Decode attention (one query position per head) ----------------------- */

/* out[h, :] f16 = softmax_j(sm_scale * q[h, :] . K[kvh, j, :]) . V[kvh, j, :]
 * over j < kv_len, kvh = h * n_kv_heads / n_q_heads (grouped-query heads);
 * q, out f16 [n_q_heads, head_dim]; K and V f16 with element (kvh, j, d) at
 * kvh * stride_kv_head + j * stride_kv_seq + d (elements). Scores, softmax
 * and the weighted sum in f32. Requirements: head_dim a multiple of 4 in
 * [4, 128]; strides multiples of 4, stride_kv_seq >= head_dim; q, K, V
 * 8-byte aligned; 1 <= n_kv_heads <= n_q_heads; kv_len >= 1.
 *
 * nsr_attention_splitkv_f16: the positions are cut into n_splits ranges of
 * ceil(kv_len / n_splits); `partial` is caller scratch of at least
 * n_q_heads * n_splits * (head_dim + 2) floats (the reference's partial
 * buffer, 3 * 128 floats per (head, split), is large enough). Two launches.
 * Replaces attention_decode_splitkv_partial / _reduce via
 * enc_attention_splitkv (src/triton_kernels.rs:925-973; kernels/
 * moonshine_kernels.py:1631-1716), the decoder's cross-attention over the
 * encoder K/V [kv_len, heads, head_dim] (src/moonshine/gpu_decoder_metal.rs:
 * 170-182). */
nsr_status nsr_attention_splitkv_f16(const void* q, const void* k, const void* v, void* out, float* partial,
                                     int64_t kv_len, int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads,
                                     float sm_scale, int64_t stride_kv_head, int64_t stride_kv_seq, int64_t n_splits,
                                     nsr_stream_t stream);

/* nsr_attention_splitkv_f16 without the `partial` argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The partials go to a fixed scratch array of NSR_NOALLOC_SCRATCH_BYTES
 * (1 MiB) that the library holds on each GPU it runs on until the process
 * ends; calls needing more than that, n_q_heads * n_splits * (head_dim + 2)
 * > 262144 floats, fail with NSR_ERR_UNSUPPORTED. The call allocates
 * nothing. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other host threads) race and must be
 * serialised by the caller. Same results as nsr_attention_splitkv_f16.
 * The array's device address is resolved when the library first loads on a
 * device (nsr_init, or the first entry point called there): under graph
 * capture, call nsr_init on that device before capturing. */
#define NSR_NOALLOC_SCRATCH_BYTES (1024 * 1024)
nsr_status nsr_attention_splitkv_f16_noalloc(const void* q, const void* k, const void* v, void* out,
                                             int64_t kv_len, int64_t head_dim, int64_t n_kv_heads,
                                             int64_t n_q_heads, float sm_scale, int64_t stride_kv_head,
                                             int64_t stride_kv_seq, int64_t n_splits, nsr_stream_t stream);

/* The same attention in one launch and without scratch: one workgroup per
 * query head, whose waves take every W-th chunk of 64 positions and merge
 * in LDS. Replaces triton_attention_decode /
 * enc_attention_decode (src/triton_kernels.rs:648-675, 900-923; kernels/
 * moonshine_kernels.py:1525-1625), the decoder's self-attention over its KV
 * cache [heads, max_kv_len, head_dim] (src/moonshine/gpu_decoder_metal.rs:
 * 158-168). */
nsr_status nsr_attention_decode_f16(const void* q, const void* k, const void* v, void* out, int64_t kv_len,
                                    int64_t head_dim, int64_t n_kv_heads, int64_t n_q_heads, float sm_scale,
                                    int64_t stride_kv_head, int64_t stride_kv_seq, nsr_stream_t stream);

/* ---- Kokoro resblock conv1d (MFMA) ----------------------------------------- */

/* out [B, C_out, T_out] f32 = conv1d(x [B, C_in, T_in] f32, w [C_out, C_in, K]
 * f16) + bias [C_out] f16 (or NULL), stride 1, zero padding `padding` on both
 * sides, dilation `dilation`: T_out = T_in + 2 padding - dilation (K - 1).
 * f32 accuracy on f16 matrix cores (each activation is split into two f16
 * halves; f32 accumulation). Requirements: C_in % 16 == 0; (K - 1) *
 * dilation <= 64; T_in, T_out < 2^23; stride != 1 returns
 * NSR_ERR_UNSUPPORTED, and so do shapes whose rows of one batch reach
 * 4 GiB (4 C_in T_in or 4 C_out T_out >= 2^32: one buffer descriptor
 * addresses a batch's rows). The same holds for every conv entry point. Rows that start 16-byte aligned (T_in % 4 == 0,
 * T_out % 4 == 0, 16-byte aligned x / out / residual) take the faster
 * producer/consumer kernels. Packs the weights into the caller's workspace
 * (NSR_WS_PACKED_WEIGHTS, see nsr_conv1d_workspace_bytes) on every call and
 * allocates nothing; callers that convolve repeatedly with the same weights
 * pack once with nsr_conv1d_pack_f16 and call nsr_conv1d_f16w_packed.
 * Replaces KokoroGpuBackend::conv1d_f32 (src/kokoro/gpu_backend.rs:165-167;
 * Metal impl src/kokoro/gpu_decoder.rs:840, which runs conv1d_f32io,
 * kernels/kokoro_kernels.py:773-816, or an im2col + f16 matmul that rounds
 * x to f16) and Candle's conv1d + bias broadcast_add in ResBlock::forward
 * (src/kokoro/decoder.rs:1366-1367, 1373-1374). */
nsr_status nsr_conv1d_f32io(const float* x, const void* w, const void* bias, float* out, int64_t B,
                            int64_t C_in, int64_t C_out, int64_t T_in, int64_t K, int64_t stride,
                            int64_t padding, int64_t dilation, void* workspace, int64_t workspace_bytes,
                            nsr_stream_t stream);

/* Device workspace of the conv entry points that need one: caller-owned,
 * 256-byte aligned, held by one call until its launches have run on the
 * stream. The library allocates nothing on these paths. Parts (OR them):
 *   NSR_WS_PACKED_WEIGHTS  nsr_conv1d_f32io's packed weights,
 *   NSR_WS_IN_STATS        the input's row statistics (nsr_adain_snake_conv1d_f32,
 *                          and _chain when x_stats is NULL),
 *   NSR_WS_OUT_STATS       per-32-column partials of the output's row
 *                          statistics (_chain and nsr_conv1d_f16w_packed_stats
 *                          when out_stats is not NULL),
 *   NSR_WS_RECORDS         optional, for every entry point with a workspace:
 *                          the conv input as f16 hi / lo records (B x
 *                          ceil(C_in / 128) x (T_in + 2 padding) x 512 bytes,
 *                          rounded up to 256) and the weights in MFMA
 *                          fragment order (ceil(C_out / 128) x 4 x K x
 *                          ceil(C_in / 128) x 8192 bytes). When the
 *                          workspace also covers it (after the parts the call
 *                          needs), rows with T_out % 4 == 0 and 16-byte
 *                          aligned out / residual, and (K - 1) * dilation
 *                          <= 56, take the two-launch record path: a
 *                          bandwidth-bound pass writes the records (AdaIN +
 *                          Snake included in the fused entry points) and the
 *                          fragment weights, then an MFMA kernel with no
 *                          per-element VALU work reads them. Same results as
 *                          the one-launch kernels.
 * nsr_conv1d_workspace_bytes writes the bytes a call of that shape needs for
 * the given parts (each part at a 256-byte aligned offset, in flag order).
 * No counterpart in the reference (its Metal backend allocates per call). */
#define NSR_WS_PACKED_WEIGHTS 1u
#define NSR_WS_IN_STATS 2u
#define NSR_WS_OUT_STATS 4u
#define NSR_WS_RECORDS 8u
nsr_status nsr_conv1d_workspace_bytes(int64_t B, int64_t C_in, int64_t C_out, int64_t T_in, int64_t K,
                                      int64_t padding, int64_t dilation, unsigned parts, int64_t* bytes);

/* Weights [C_out, C_in, K] f16 -> the packed [C_out, K, C_in] f16 layout the
 * conv kernels read (16-byte aligned output, C_out*C_in*K halfs). No
 * counterpart in the reference; done once at load. */
nsr_status nsr_conv1d_pack_f16(const void* w, int64_t C_out, int64_t C_in, int64_t K, void* w_packed,
                               nsr_stream_t stream);

/* nsr_conv1d_f32io over packed weights, plus an optional residual [B, C_out,
 * T_out] f32 added in the epilogue (NULL = none; the `h + residual` that ends
 * each ResBlock iteration, src/kokoro/decoder.rs:1378). */
nsr_status nsr_conv1d_f16w_packed(const float* x, const void* w_packed, const void* bias,
                                  const float* residual, float* out, int64_t B, int64_t C_in,
                                  int64_t C_out, int64_t T_in, int64_t K, int64_t padding,
                                  int64_t dilation, nsr_stream_t stream);

/* One ResBlock stage with the AdaIN1d + Snake of the conv input fused into
 * the conv's load (src/kokoro/decoder.rs:1364-1376):
 *   y   = snake((1 + gamma) * (x - mean) / sqrt(var + eps) + beta, alpha)
 *         (per (b, ci) row statistics over T, as nsr_adain_snake_f32)
 *   out = conv1d(y, w_packed) + bias (+ residual)
 * x [B, C_in, T] f32; gamma/beta/alpha as nsr_adain_snake_f32 (F32 or F16,
 * batch strides); y is never written to memory. Two launches (row
 * statistics into the caller's workspace, NSR_WS_IN_STATS, then the fused
 * conv); allocates nothing. Replaces adain + snake_activation_tensor + conv1d + bias of
 * ResBlock::forward (:1364-1376; Metal: adain_snake then conv1d_f32io,
 * src/kokoro/gpu_decoder.rs:886-950). */
nsr_status nsr_adain_snake_conv1d_f32(const float* x, const void* gamma, const void* beta,
                                      const void* alpha, nsr_dtype param_dtype,
                                      int64_t gamma_bstride, int64_t beta_bstride,
                                      const void* w_packed, const void* bias,
                                      const float* residual, float* out, int64_t B, int64_t C_in,
                                      int64_t C_out, int64_t T, int64_t K, int64_t padding,
                                      int64_t dilation, float eps, void* workspace,
                                      int64_t workspace_bytes, nsr_stream_t stream);

/* The same ResBlock stage with the row statistics handed along the chain
 * instead of re-read. x_stats ([B*C_in][2]: mean, 1 / sqrt(var + eps) of
 * each x row) replaces the statistics pass over x when not NULL (the
 * previous stage's out_stats); out_stats, when not NULL, receives the same
 * pair for each row of out (after bias and residual), for the next stage's
 * AdaIN. With 16-byte aligned rows the conv's epilogue produces them from
 * registers (per 32-column block count, mean and M2, merged per row by
 * Chan's pairwise formula) instead of a second read of out. Workspace:
 * NSR_WS_IN_STATS when x_stats is NULL, NSR_WS_OUT_STATS when out_stats is
 * not NULL (0 bytes, workspace may be NULL, when neither). No counterpart
 * in the reference, whose ResBlock (src/kokoro/decoder.rs:1352-1380, GPU
 * path :1087-1160) runs adain_snake_f32 and conv1d_f32 one after the other;
 * the results match nsr_adain_snake_conv1d_f32 within the fp32 bar. */
nsr_status nsr_adain_snake_conv1d_chain_f32(const float* x, const float* x_stats, const void* gamma,
                                            const void* beta, const void* alpha, nsr_dtype param_dtype,
                                            int64_t gamma_bstride, int64_t beta_bstride,
                                            const void* w_packed, const void* bias,
                                            const float* residual, float* out, float* out_stats,
                                            int64_t B, int64_t C_in, int64_t C_out, int64_t T, int64_t K,
                                            int64_t padding, int64_t dilation, float eps, void* workspace,
                                            int64_t workspace_bytes, nsr_stream_t stream);

/* nsr_conv1d_f16w_packed that also writes out_stats ([B*C_out][2]: mean,
 * 1 / sqrt(var + eps) of each output row), for an AdaIN that follows.
 * Workspace: NSR_WS_OUT_STATS. */
nsr_status nsr_conv1d_f16w_packed_stats(const float* x, const void* w_packed, const void* bias,
                                        const float* residual, float* out, float* out_stats, int64_t B,
                                        int64_t C_in, int64_t C_out, int64_t T_in, int64_t K,
                                        int64_t padding, int64_t dilation, float eps, void* workspace,
                                        int64_t workspace_bytes, nsr_stream_t stream);

/* ---- Repacked-Q8 GEMV (decoder projections at M = 1) ---------------------- */

/* Weights W [K, NW] in the repacked Q8 layout of the reference's decoder
 * kernels: qs u32 [K, NW/4] with the int8 weight of column c in byte c % 4
 * (lowest byte first) of word c / 4, and scales f16 [K/32, NW], one per
 * 32-row block and column: W[k, c] = int8 * f32(scale[k / 32, c]). x [K] is
 * F16 or F32. Accumulation is f32 in a fixed order (no atomics, no scratch):
 * results are reproducible run to run.
 * Requirements: K % 32 == 0 and K > 0, N % 16 == 0, qs and scales 16-byte
 * aligned. N == 0 is a no-op. */

/* out[N] = x @ W (+ bias[N] f32 when bias != NULL); out F16 or F32.
 * Replaces gemv_q8 / gemv_q8_bias (kernels/moonshine_kernels.py:616-644,
 * 647-677). */
nsr_status nsr_gemv_q8(const void* x, nsr_dtype x_dtype, const uint32_t* qs,
                       const uint16_t* scales, const float* bias, void* out,
                       nsr_dtype out_dtype, int64_t K, int64_t N,
                       nsr_stream_t stream);

/* W is [K, 2N]: x-half in columns [0, N), gate-half in [N, 2N); bias [2N]
 * f32 or NULL. out[i] = silu(x@Wg[i] + bg[i]) * (x@Wx[i] + bx[i]), i < N.
 * Replaces gemv_q8_bias_glu (kernels/moonshine_kernels.py:1721-1772), the
 * fused fc1 + GLU of DecoderMLP::forward (src/moonshine/decoder.rs:403-411). */
nsr_status nsr_gemv_q8_bias_glu(const void* x, nsr_dtype x_dtype, const uint32_t* qs,
                                const uint16_t* scales, const float* bias, void* out,
                                nsr_dtype out_dtype, int64_t K, int64_t N,
                                nsr_stream_t stream);

/* proj = f16-rounded x @ W (W [K, dim]); out_f32 = proj + residual (f32;
 * out_f32 may be residual itself); norm = (out_f32 - mean) / sqrt(var + eps)
 * * ln_weight (biased variance over dim; ln_weight F16 or F32; norm F16 or
 * F32). Two launches on `stream`: the projection, then the row LayerNorm.
 * Replaces gemv_q8_resadd_ln (kernels/moonshine_kernels.py:1775-1819), the
 * fused out-projection + residual + next LayerNorm of the decoder step
 * (triton_residual_add_layernorm src/triton_kernels.rs:742 after the
 * projection). */
nsr_status nsr_gemv_q8_resadd_ln(const void* x, nsr_dtype x_dtype, const uint32_t* qs,
                                 const uint16_t* scales, const float* residual,
                                 float* out_f32, const void* ln_weight, nsr_dtype w_dtype,
                                 void* norm, nsr_dtype norm_dtype, int64_t K, int64_t dim,
                                 float eps, nsr_stream_t stream);

/* ---- t4 tiles: the same weights packed for coalesced reads --------------- */

/* Packs a repacked-Q8 weight (qs u32 [K, NW/4], scales f16 [K/32, NW], as
 * above) into t4 tiles, once, at load time: tile t holds 4 weight columns
 * for all K rows contiguously (t4_qs [NW/4][K] u32, one int8 per byte) and
 * their scales (t4_scales [NW/4][K/32][4] f16). glu != 0 packs a GLU weight
 * ([K, 2N], NW = 2N): tile t holds x-half columns 2t, 2t+1 and gate-half
 * columns 2t, 2t+1. The packing is a byte permutation: dequantised values
 * are unchanged. t4_qs takes K*NW bytes, t4_scales K/32*NW*2 bytes, both
 * 16-byte aligned. Requirements: K % 32 == 0, NW % 16 == 0 (NW % 32 == 0
 * for GLU). Has no counterpart in the reference, which defines only the
 * [K, N/4] layout (kernels/moonshine_kernels.py:611-614) and reads it with
 * one thread per column; on gfx950 a workgroup that owns a few columns of
 * that layout scatters its reads over all K rows. */
nsr_status nsr_q8_pack_t4(const uint32_t* qs, const uint16_t* scales, int64_t K,
                          int64_t NW, int glu, uint32_t* t4_qs, uint16_t* t4_scales,
                          nsr_stream_t stream);

/* From a GGUF Q8_0 weight, on the device: `blocks` is an nn::Linear weight
 * W [N, K] (out, in) as the reference's GGUF files store it (N rows of K/32
 * blocks {f16 d; int8 qs[32]}, 34 bytes each; tools/quantize-moonshine/src/
 * main.rs:63-150), for example uploaded by nsr_gguf_upload. These write the
 * GEMV layouts of W^T (x[K] @ W^T = the layer's output): the repacked Q8
 * qs [K, N/4] + scales [K/32, N] of nsr_gemv_q8*, or t4 tiles (glu != 0:
 * rows [0, N/2) are the x half and [N/2, N) the gate half, as
 * DecoderMLP::forward chunks fc1's output, src/moonshine/decoder.rs:
 * 403-411). A transpose of the stored int8 values and f16 scales: the
 * dequantised weights are unchanged. Replaces the reference's host-side
 * dequantise + transpose of decoder weights (dequant_2d,
 * src/moonshine/gpu_decoder.rs:180-184). Requirements: K % 32 == 0,
 * N % 16 == 0 (N % 32 == 0 for GLU), blocks 2-byte and outputs 16-byte
 * aligned. */
nsr_status nsr_q8_0_to_gemv_q8(const void* blocks, int64_t N, int64_t K, uint32_t* qs,
                               uint16_t* scales, nsr_stream_t stream);
nsr_status nsr_q8_0_to_t4(const void* blocks, int64_t N, int64_t K, int glu, uint32_t* t4_qs,
                          uint16_t* t4_scales, nsr_stream_t stream);

/* nsr_gemv_q8 / nsr_gemv_q8_bias_glu / nsr_gemv_q8_resadd_ln over t4 tiles
 * (same results up to f32 summation order; x additionally aligned to 4
 * elements). Replace the same reference kernels as the functions above. */
nsr_status nsr_gemv_q8_t4(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs,
                          const uint16_t* t4_scales, const float* bias, void* out,
                          nsr_dtype out_dtype, int64_t K, int64_t N, nsr_stream_t stream);
nsr_status nsr_gemv_q8_t4_bias_glu(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs,
                                   const uint16_t* t4_scales, const float* bias, void* out,
                                   nsr_dtype out_dtype, int64_t K, int64_t N,
                                   nsr_stream_t stream);
nsr_status nsr_gemv_q8_t4_resadd_ln(const void* x, nsr_dtype x_dtype, const uint32_t* t4_qs,
                                    const uint16_t* t4_scales, const float* residual,
                                    float* out_f32, const void* ln_weight, nsr_dtype w_dtype,
                                    void* norm, nsr_dtype norm_dtype, int64_t K, int64_t dim,
                                    float eps, nsr_stream_t stream);

/* ---- Measurement floors ---------------------------------------------------- */

/* No counterpart in the reference: the benchmark's floors, launched through
 * the same runtime as every fused kernel.
 * nsr_calib_empty: one empty kernel (the cost of a launch on the stream).
 * nsr_calib_copy: device copy of `bytes` (a multiple of 16, src and dst
 * 16-byte aligned) with 128-bit loads and stores. form 0: one 16-byte chunk
 * per lane, ceil(bytes / 4096) workgroups of 256; form 1 / 2: persistent,
 * groups_per_cu x #CU workgroups (0: 8) each keeping 4 / 8 chunks per lane
 * in flight. */
nsr_status nsr_calib_empty(nsr_stream_t stream);
nsr_status nsr_calib_copy(const void* src, void* dst, int64_t bytes, int form, int groups_per_cu,
                          nsr_stream_t stream);
/* nsr_calib_copy_rows: device copy of n_rows rows of row_bytes (a multiple of
 * 16, 16-byte aligned) row by row, the AdaIN row kernel's access structure:
 * one 512-lane workgroup per row, a persistent grid of one per CU. */
nsr_status nsr_calib_copy_rows(const void* src, void* dst, int64_t n_rows, int64_t row_bytes, nsr_stream_t stream);
/* nsr_calib_adain_timeline: nsr_adain_snake_f32 on the row kernel of the
 * [8, 128, 115200] benchmark shape (rows of 114692..116736 floats, f32
 * gamma / beta [B, C], alpha [C], eps 1e-5), with the same output, writing
 * a timeline of the call: 80 uint64 words per workgroup into `stamps`
 * (device memory, at least 80 x #workgroups words; #workgroups = min(B * C,
 * #CU) for this kernel). Per workgroup: [0] its XCD, [1] its start, [2 + w]
 * the end of wave w's last store, [10 + 8 r + w] when row r's data had
 * landed for wave w (r < 8); times in ticks of the GPU's 100 MHz clock. */
nsr_status nsr_calib_adain_timeline(const float* x, const float* gamma, const float* beta, const float* alpha,
                                    float* out, int64_t B, int64_t C, int64_t T, uint64_t* stamps,
                                    int64_t stamps_words, nsr_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NSPEECH_ROCM_H */
