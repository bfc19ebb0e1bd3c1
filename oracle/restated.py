"""ctypes bindings to oracle/_build/libnsr_oracle.so (TEST INFRASTRUCTURE).

Every function takes and returns numpy arrays. See nsr_oracle.c for the
reference file:line each restatement follows.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "libnsr_oracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_I64 = C.c_int64


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise FileNotFoundError(f"{_LIB_PATH} missing: run python -m nspeech_amd.build (or oracle/build.py)")
        L = C.CDLL(str(_LIB_PATH))
        L.orc_f16_to_f32.argtypes = [_u16p, _f32p, _I64]
        L.orc_f32_to_f16.argtypes = [_f32p, _u16p, _I64]
        _u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        L.orc_gemv_q8_f32.argtypes = [_f32p, _u32p, _u16p, C.c_void_p, _f32p, _I64, _I64, C.c_int]
        L.orc_gemv_q8_resadd_ln.argtypes = [_f32p, _u32p, _u16p, _f32p, _u16p, _f32p, _u16p, _I64, _I64, C.c_float]
        L.orc_rope_qk_cache_f16.argtypes = [_u16p, _u16p, C.c_void_p, _f32p, _I64, _I64, _I64, C.c_int, _I64, _I64,
                                            _u16p, C.c_void_p]
        L.orc_f32_to_bf16.argtypes = [_f32p, _u16p, _I64]
        L.orc_bf16_to_f32.argtypes = [_u16p, _f32p, _I64]
        L.orc_q8_0_dequantize.argtypes = [_u8p, _I64, _I64, _f32p]
        L.orc_index_select_rows.argtypes = [_f32p, _I64, _I64, _i64p, _I64, _f32p]
        L.orc_index_select_rows.restype = _I64
        L.orc_q8_0_embedding.argtypes = [_u8p, _I64, _I64, _i64p, _I64, C.c_int, _f32p, _f32p]
        L.orc_q8_0_embedding.restype = _I64
        L.orc_silu_f32.argtypes = [_f32p, _f32p, _I64]
        L.orc_gelu_erf_f32.argtypes = [_f32p, _f32p, _I64]
        L.orc_glu_silu_f32.argtypes = [_f32p, _f32p, _I64]
        L.orc_fast_add_f32.argtypes = [_f32p, _f32p, _f32p, _I64]
        L.orc_layernorm_candle_f32.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p, _I64, _I64, C.c_float, C.c_int]
        L.orc_layernorm_twopass_f32.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p, _I64, _I64, C.c_float,
                                                C.c_int, C.c_int]
        L.orc_resadd_ln_gelu_bf16.argtypes = [_u16p, _u16p, _u16p, _u16p, C.c_void_p, _u16p, _I64, _I64,
                                              C.c_float, C.c_int, C.c_int]
        L.orc_rope_table_f32.argtypes = [_f32p, _I64, C.c_int, C.c_float]
        L.orc_rotary_f32.argtypes = [_f32p, _f32p, _I64, _I64, _I64, _I64, C.c_int, C.c_float, _I64, _f32p, C.c_int]
        L.orc_adain_snake_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _I64, _I64, _I64, _I64, _I64,
                                          C.c_float, C.c_int]
        L.orc_attention_decode_f16.argtypes = [_u16p, _u16p, _u16p, _f32p, _I64, _I64, _I64, _I64, C.c_float,
                                               _I64, _I64]
        L.orc_combine_f32.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p, _I64, C.c_int, C.c_float, C.c_int,
                                      C.c_float]
        L.orc_istft_f32.argtypes = [_f32p, _f32p, _I64, _I64, _I64]
        L.orc_snake_f32.argtypes = [_f32p, _f32p, _f32p, _I64, _I64, _I64]
        L.orc_conv1d_f32io.argtypes = [_f32p, _u16p, C.c_void_p, _f32p, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                       _I64, _I64, C.c_int]
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# -------------------------------------------------------------- dtypes ---

def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32(h.ravel(), out.ravel(), h.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(x.ravel(), out.ravel(), x.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = _c(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32(b.ravel(), out.ravel(), b.size)
    return out


# ---------------------------------------------------------------- Q8_0 ---

def q8_0_dequantize(blocks: np.ndarray, vocab: int, d: int) -> np.ndarray:
    blocks = _c(blocks, np.uint8)
    assert blocks.size == vocab * (d // 32) * 34
    out = np.empty((vocab, d), np.float32)
    lib().orc_q8_0_dequantize(blocks.ravel(), vocab, d, out.ravel())
    return out


def q8_0_embedding(blocks: np.ndarray, vocab: int, d: int, ids: np.ndarray, act: int = 0):
    """QEmbedding::forward (+ silu when act == 1). Returns (out, n_bad_ids)."""
    blocks = _c(blocks, np.uint8)
    ids64 = _c(ids, np.int64).ravel()
    table = np.empty(vocab * d, np.float32)
    out = np.empty((ids64.size, d), np.float32)
    bad = lib().orc_q8_0_embedding(blocks.ravel(), vocab, d, ids64, ids64.size, act, table, out.ravel())
    return out, int(bad)


# --------------------------------------------------------- activations ---

def silu(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_silu_f32(x.ravel(), y.ravel(), x.size)
    return y


def gelu_erf(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_gelu_erf_f32(x.ravel(), y.ravel(), x.size)
    return y


def glu_silu(fc1: np.ndarray) -> np.ndarray:
    fc1 = _c(fc1, np.float32).ravel()
    n = fc1.size // 2
    out = np.empty(n, np.float32)
    lib().orc_glu_silu_f32(fc1, out, n)
    return out


def fast_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    out = np.empty_like(a)
    lib().orc_fast_add_f32(a.ravel(), b.ravel(), out.ravel(), a.size)
    return out


# ----------------------------------------------------------- LayerNorm ---

def layernorm_candle(x, w=None, b=None, eps=1e-5, nthreads=1):
    x = _c(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    w = None if w is None else _c(w, np.float32)
    b = None if b is None else _c(b, np.float32)
    y = np.empty_like(x)
    lib().orc_layernorm_candle_f32(x.ravel(), _ptr(w), _ptr(b), y.ravel(), rows, cols, eps, nthreads)
    return y


def layernorm_twopass(x, w=None, b=None, eps=1e-5, unit_offset=False, nthreads=1):
    x = _c(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    w = None if w is None else _c(w, np.float32)
    b = None if b is None else _c(b, np.float32)
    y = np.empty_like(x)
    lib().orc_layernorm_twopass_f32(x.ravel(), _ptr(w), _ptr(b), y.ravel(), rows, cols, eps, int(unit_offset),
                                    nthreads)
    return y


def resadd_ln_gelu_bf16(x_bits, res_bits, w_bits, b_bits, eps=1e-5, gelu=True, nthreads=1):
    """bf16 chain (all arguments/outputs are bf16 bit patterns). Returns (h, y)."""
    x_bits = _c(x_bits, np.uint16)
    res_bits = _c(res_bits, np.uint16)
    cols = x_bits.shape[-1]
    rows = x_bits.size // cols
    h = np.empty_like(x_bits)
    y = np.empty_like(x_bits)
    lib().orc_resadd_ln_gelu_bf16(x_bits.ravel(), res_bits.ravel(), _c(w_bits, np.uint16), _c(b_bits, np.uint16),
                                  h.ctypes.data_as(C.c_void_p), y.ravel(), rows, cols, eps, int(gelu), nthreads)
    return h, y


# -------------------------------------------------------------- rotary ---

def rope_table(max_pos: int, rot: int, theta: float) -> np.ndarray:
    t = np.empty((max_pos, rot), np.float32)
    lib().orc_rope_table_f32(t.ravel(), max_pos, rot, theta)
    return t


def rotary(x, rot: int, theta: float, pos0: int = 0, nthreads=1):
    """x [B, H, T, Dh] -> rotated copy (apply_rotary_pos_emb on one tensor)."""
    x = _c(x, np.float32)
    B, H, T, Dh = x.shape
    out = np.empty_like(x)
    cs = np.empty(max(1, T * rot), np.float32)
    lib().orc_rotary_f32(x.ravel(), out.ravel(), B, H, T, Dh, rot, theta, pos0, cs, nthreads)
    return out


# ------------------------------------------------------ AdaIN + Snake ---

def adain_snake(x, gamma, beta, alpha, eps=1e-5, nthreads=1):
    """x [B, C, T]; gamma/beta [C] (shared) or [B, C]; alpha [C]."""
    x = _c(x, np.float32)
    B, Cc, T = x.shape
    gamma = _c(gamma, np.float32)
    beta = _c(beta, np.float32)
    gs = Cc if gamma.ndim == 2 else 0
    bs = Cc if beta.ndim == 2 else 0
    out = np.empty_like(x)
    lib().orc_adain_snake_f32(x.ravel(), gamma.ravel(), beta.ravel(), _c(alpha, np.float32).ravel(), out.ravel(),
                              B, Cc, T, gs, bs, eps, nthreads)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> IEEE half bits, round to nearest even (orc_f32_to_f16)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16(x.ravel(), out.ravel(), x.size)
    return out


def rope_qk_cache_f16(q_bits, k_bits, v_bits, table, pos, rot, cache_k_bits, cache_v_bits=None):
    """Decode-step RoPE(q, k) + K (and V) cache append on f16 bit patterns
    (orc_rope_qk_cache_f16). q [Hq, Dh], k/v [Hk, Dh], caches [Hk, L, Dh];
    returns (q, k, cache_k, cache_v) as new arrays."""
    q = _c(q_bits, np.uint16).copy()
    k = _c(k_bits, np.uint16).copy()
    ck = _c(cache_k_bits, np.uint16).copy()
    cv = None if cache_v_bits is None else _c(cache_v_bits, np.uint16).copy()
    v = None if v_bits is None else _c(v_bits, np.uint16)
    Hq, Dh = q.shape
    Hk = k.shape[0]
    L = ck.shape[1]
    t = _c(table, np.float32)
    lib().orc_rope_qk_cache_f16(q.ravel(), k.ravel(), _ptr(v), t.ravel(), Hq, Hk, Dh, rot, pos, L, ck.ravel(),
                                _ptr(cv))
    return q, k, ck, cv


def gemv_q8(x, qs, scales_bits, bias=None, glu=False):
    """Q8 GEMV (M = 1) as gemv_q8 / gemv_q8_bias / gemv_q8_bias_glu compute it, f32
    result before the output rounding. qs u32 [K, NW/4], scales f16 bits [K/32, NW]."""
    x = _c(x, np.float32)
    qs = _c(qs, np.uint32)
    sc = _c(scales_bits, np.uint16)
    K = x.shape[0]
    NW = sc.shape[1]
    N = NW // 2 if glu else NW
    out = np.empty(N, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_gemv_q8_f32(x, qs.ravel(), sc.ravel(), _ptr(b), out, K, N, 1 if glu else 0)
    return out


def gemv_q8_resadd_ln(x, qs, scales_bits, residual, ln_w_bits, eps=1e-5):
    """gemv_q8_resadd_ln: returns (h f32 [dim], norm f16 bits [dim])."""
    x = _c(x, np.float32)
    qs = _c(qs, np.uint32)
    sc = _c(scales_bits, np.uint16)
    res = _c(residual, np.float32)
    w = _c(ln_w_bits, np.uint16)
    K, dim = x.shape[0], sc.shape[1]
    h = np.empty(dim, np.float32)
    norm = np.empty(dim, np.uint16)
    lib().orc_gemv_q8_resadd_ln(x, qs.ravel(), sc.ravel(), res, w, h, norm, K, dim, eps)
    return h, norm


def q8_pack_t4(qs, scales_bits, glu=False):
    """t4 tile packing of a repacked-Q8 weight (the layout nsr_q8_pack_t4
    writes): tiles [NW/4][K][4] int8 (returned as u32 words, byte c = slot c)
    and scales [NW/4][K/32][4] f16 bits. Slot c of tile t is weight column
    4t + c, or for a GLU weight [K, 2N] x-half column 2t + c (c < 2) and
    gate-half column N + 2t + c - 2. A byte permutation of the input; the
    GEMV over the tiles is the GEMV over the original columns."""
    qs = np.ascontiguousarray(qs, np.uint32)
    sc = np.ascontiguousarray(scales_bits, np.uint16)
    K, NW = qs.shape[0], 4 * qs.shape[1]
    q8 = qs.view(np.uint8).reshape(K, NW)
    t = np.arange(NW // 4)
    if glu:
        N = NW // 2
        cols = np.stack([2 * t, 2 * t + 1, N + 2 * t, N + 2 * t + 1], axis=1)
    else:
        cols = 4 * t[:, None] + np.arange(4)[None, :]
    tiles = np.ascontiguousarray(q8[:, cols].transpose(1, 0, 2))        # [T, K, 4]
    tsc = np.ascontiguousarray(sc[:, cols].transpose(1, 0, 2))          # [T, K/32, 4]
    return tiles.reshape(-1).view(np.uint32).copy(), tsc.reshape(-1).copy()


def q8_0_quantize(x):
    """GGUF Q8_0 quantisation of a float32 matrix [rows, cols] (cols % 32 == 0)
    as the reference's quantizer calls it (QTensor::quantize(.., Q8_0),
    tools/quantize-moonshine/src/main.rs:118), following ggml's published
    quantize_row_q8_0 (candle's BlockQ8_0::from_float): per 32 values,
    d = max|x| / 127 (f32), q = round(x / d) half away from zero (0 when d is
    0), stored as {f16 d; int8 q[32]}. Returns uint8 [rows, cols/32*34]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    xb = x.reshape(rows, cols // 32, 32)
    amax = np.max(np.abs(xb), axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (xb * idv[:, :, None]).astype(np.float32)
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)   # round half away from zero
    out = np.empty((rows, cols // 32, 34), np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, cols // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(rows, cols // 32 * 34)


def q8_0_to_gemv_q8(blocks, N, K):
    """A GGUF Q8_0 weight W [N, K] (rows of 34-byte blocks) as the repacked
    Q8 layout of W^T: qs u32 [K, N/4] (qs[k] byte c of word w = int8 of
    W[4w + c, k]) and scales f16 bits [K/32, N] (W's block scales,
    transposed)."""
    b = np.ascontiguousarray(blocks, np.uint8).reshape(N, K // 32, 34)
    d = np.ascontiguousarray(b[:, :, 0:2]).view(np.uint16).reshape(N, K // 32)
    q = np.ascontiguousarray(b[:, :, 2:]).reshape(N, K)
    qs = np.ascontiguousarray(q.T).view(np.uint32).reshape(K, N // 4)
    return qs, np.ascontiguousarray(d.T)


def conv1d_f32io(x, w_bits, bias_bits=None, stride=1, padding=0, dilation=1, nthreads=1):
    """conv1d_f32io over a batch: x f32 [B, C_in, T_in], w f16 bits [C_out, C_in, K],
    bias f16 bits [C_out] or None -> f32 [B, C_out, T_out]."""
    x = _c(x, np.float32)
    if x.ndim == 2:
        x = x[None]
    w = _c(w_bits, np.uint16)
    B, C_in, T_in = x.shape
    C_out, _, K = w.shape
    T_out = (T_in + 2 * padding - dilation * (K - 1) - 1) // stride + 1
    out = np.empty((B, C_out, T_out), np.float32)
    b = None if bias_bits is None else _c(bias_bits, np.uint16)
    lib().orc_conv1d_f32io(x.ravel(), w.ravel(), _ptr(b), out.ravel(), B, C_in, C_out, T_in, T_out, K, stride,
                           padding, dilation, nthreads)
    return out


def attention_decode(q_bits, k_bits, v_bits, kv_len, n_kv_heads, sm_scale, stride_kv_head, stride_kv_seq):
    """attention_decode_1d_masked restated: q f16 bits [n_q_heads, head_dim]; k, v f16 bits (flat, addressed as
    head * stride_kv_head + pos * stride_kv_seq + d) -> f32 [n_q_heads, head_dim] before the f16 store."""
    q = _c(q_bits, np.uint16)
    n_q_heads, head_dim = q.shape
    out = np.empty((n_q_heads, head_dim), np.float32)
    lib().orc_attention_decode_f16(q.ravel(), _c(k_bits, np.uint16).ravel(), _c(v_bits, np.uint16).ravel(),
                                   out.ravel(), kv_len, head_dim, n_kv_heads, n_q_heads, sm_scale, stride_kv_head,
                                   stride_kv_seq)
    return out


def combine(a, b=None, c=None, scale=None, lrelu_slope=None):
    """((a + b) + c) * scale, then x > 0 ? x : x * slope (each step optional)."""
    a = _c(a, np.float32).ravel()
    b = None if b is None else _c(b, np.float32).ravel()
    c = None if c is None else _c(c, np.float32).ravel()
    out = np.empty_like(a)
    lib().orc_combine_f32(a, _ptr(b), _ptr(c), out, a.size, int(scale is not None),
                          0.0 if scale is None else float(scale), int(lrelu_slope is not None),
                          0.0 if lrelu_slope is None else float(lrelu_slope))
    return out


def resblock_average(r0, r1, r2, lrelu_slope=None):
    """The Kokoro MRF average ((r0 + r1) + r2) * f32(1/3) (+ leaky ReLU)."""
    return combine(r0, r1, r2, np.float32(0.3333333333333333), lrelu_slope)


def istft(x, n_fft: int, hop: int):
    """x [2 * (n_fft // 2 + 1), n_frames] f32 (log-magnitudes, raw phases) ->
    trimmed audio of (n_frames - 1) * hop samples."""
    x = _c(x, np.float32)
    bins = n_fft // 2 + 1
    assert x.ndim == 2 and x.shape[0] == 2 * bins
    n_frames = x.shape[1]
    out = np.empty((n_frames - 1) * hop, np.float32)
    lib().orc_istft_f32(x, out, n_frames, n_fft, hop)
    return out


def snake(x, alpha):
    """x [..., C, T] (rows in channel row % C), alpha [C] -> x + sin^2(alpha x) / (alpha + 1e-9)."""
    x = _c(x, np.float32)
    alpha = _c(alpha, np.float32).ravel()
    T = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_snake_f32(x, alpha, out, x.size // T, alpha.size, T)
    return out

