"""ctypes binding of libnspeech_rocm.so (include/nspeech_rocm.h) for torch tensors.

PyTorch supplies device memory and streams; every computation happens in the
library's gfx950 kernels. Importing this module imports torch first so the
library binds to the HIP runtime torch already loaded (same SONAME).
There is no fallback: if the library is missing or a call fails, NsrError
is raised.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before the library)

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libnspeech_rocm.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "nspeech_rocm.h"

NSR_OK, NSR_ERR_BAD_ARG, NSR_ERR_NOT_INIT, NSR_ERR_HIP, NSR_ERR_UNSUPPORTED = range(5)
NSR_F32, NSR_F16, NSR_BF16 = 0, 1, 2
NSR_IDX_U32, NSR_IDX_I64 = 0, 1
ACT = {"none": 0, "silu": 1, "gelu": 2, "gelu_erf": 2}
NSR_LN_UNIT_OFFSET = 1

_DT = {torch.float32: NSR_F32, torch.float16: NSR_F16, torch.bfloat16: NSR_BF16}


class NsrError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"nspeech_rocm error {status}: {msg}")
        self.status = status


_lib = None
_P = C.c_void_p
_I64 = C.c_int64


def lib() -> C.CDLL:
    """Load the library (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built: run `python -m nspeech_amd.build`")
        L = C.CDLL(str(LIB_PATH))
        L.nsr_version.restype = C.c_char_p
        L.nsr_last_error.restype = C.c_char_p
        L.nsr_init.argtypes = [C.c_char_p]
        L.nsr_kernel_count.restype = C.c_int
        L.nsr_layernorm.argtypes = [_P, C.c_int, _P, _P, C.c_int, _P, C.c_int, _I64, _I64, _I64, _I64,
                                    C.c_float, C.c_uint, C.c_int, _P]
        L.nsr_residual_add_layernorm.argtypes = [_P, C.c_int, _P, C.c_int, _P, C.c_int, _P, _P, C.c_int, _P,
                                                 C.c_int, _I64, _I64, C.c_float, C.c_uint, C.c_int, _P]
        L.nsr_rope_table_f32.argtypes = [_P, _I64, C.c_int, C.c_float]
        L.nsr_rotary_partial_interleaved_f32.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, C.c_int,
                                                         C.c_float, _I64, _P, _I64, _P]
        L.nsr_rope_qk_cache_append.argtypes = [_P, _P, _P, C.c_int, _P, _I64, _P, _P, _I64, _I64, _I64, C.c_int,
                                                _I64, _I64, _P]
        L.nsr_kv_cache_append.argtypes = [_P, _P, C.c_int, _I64, _I64, _I64, _I64, _P]
        L.nsr_adain_snake_f32.argtypes = [_P, _P, _P, _P, C.c_int, _I64, _I64, _P, _I64, _I64, _I64, C.c_float,
                                          _P]
        L.nsr_adain_snake_f16.argtypes = [_P, _P, _P, _P, C.c_int, _I64, _I64, _P, _I64, _I64, _I64, C.c_float,
                                          _P]
        L.nsr_q8_0_embed_gather.argtypes = [_P, _I64, _I64, _P, C.c_int, _I64, _P, C.c_int, _P, _P]
        L.nsr_activation.argtypes = [_P, _P, C.c_int, _I64, C.c_int, _P]
        L.nsr_glu_silu.argtypes = [_P, _P, C.c_int, _I64, _P]
        L.nsr_residual_add.argtypes = [_P, _P, _P, C.c_int, _I64, _P]
        L.nsr_gemv_q8.argtypes = [_P, C.c_int, _P, _P, _P, _P, C.c_int, _I64, _I64, _P]
        L.nsr_gemv_q8_bias_glu.argtypes = [_P, C.c_int, _P, _P, _P, _P, C.c_int, _I64, _I64, _P]
        L.nsr_gemv_q8_resadd_ln.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P, C.c_int, _P, C.c_int, _I64, _I64,
                                            C.c_float, _P]
        L.nsr_q8_pack_t4.argtypes = [_P, _P, _I64, _I64, C.c_int, _P, _P, _P]
        L.nsr_q8_0_to_gemv_q8.argtypes = [_P, _I64, _I64, _P, _P, _P]
        L.nsr_conv1d_f32io.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P]
        L.nsr_conv1d_workspace_bytes.argtypes = [_I64, _I64, _I64, _I64, _I64, _I64, _I64, C.c_uint,
                                                 C.POINTER(C.c_int64)]
        L.nsr_conv1d_pack_f16.argtypes = [_P, _I64, _I64, _I64, _P, _P]
        L.nsr_conv1d_f16w_packed.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]
        L.nsr_adain_snake_conv1d_f32.argtypes = [_P, _P, _P, _P, C.c_int, _I64, _I64, _P, _P, _P, _P, _I64, _I64,
                                                 _I64, _I64, _I64, _I64, _I64, C.c_float, _P, _I64, _P]
        L.nsr_adain_snake_conv1d_chain_f32.argtypes = [_P, _P, _P, _P, _P, C.c_int, _I64, _I64, _P, _P, _P, _P, _P,
                                                       _I64, _I64, _I64, _I64, _I64, _I64, _I64, C.c_float, _P, _I64,
                                                       _P]
        L.nsr_conv1d_f16w_packed_stats.argtypes = [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                                   C.c_float, _P, _I64, _P]
        L.nsr_q8_0_to_t4.argtypes = [_P, _I64, _I64, C.c_int, _P, _P, _P]
        L.nsr_gemv_q8_t4.argtypes = [_P, C.c_int, _P, _P, _P, _P, C.c_int, _I64, _I64, _P]
        L.nsr_gemv_q8_t4_bias_glu.argtypes = [_P, C.c_int, _P, _P, _P, _P, C.c_int, _I64, _I64, _P]
        L.nsr_gemv_q8_t4_resadd_ln.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P, C.c_int, _P, C.c_int, _I64, _I64,
                                               C.c_float, _P]
        L.nsr_attention_splitkv_f16.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, C.c_float, _I64, _I64,
                                                _I64, _P]
        L.nsr_attention_decode_f16.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, C.c_float, _I64, _I64, _P]
        L.nsr_scale_f32.argtypes = [_P, _P, _I64, C.c_float, _P]
        L.nsr_leaky_relu_f32.argtypes = [_P, _P, _I64, C.c_float, _P]
        L.nsr_resblock_average_f32.argtypes = [_P, _P, _P, _P, _I64, C.c_int, C.c_float, _P]
        L.nsr_istft_f32.argtypes = [_P, _P, _I64, _I64, C.c_int, C.c_int, _P]
        L.nsr_snake.argtypes = [_P, C.c_int, _P, C.c_int, _P, _I64, _I64, _I64, _P]
        L.nsr_attention_splitkv_f16_noalloc.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, C.c_float, _I64,
                                                        _I64, _I64, _P]
        L.nsr_calib_empty.argtypes = [_P]
        L.nsr_calib_copy.argtypes = [_P, _P, _I64, C.c_int, C.c_int, _P]
        L.nsr_calib_copy_rows.argtypes = [_P, _P, _I64, _I64, _P]
        L.nsr_calib_adain_timeline.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _P]
        for name in ("nsr_init", "nsr_layernorm", "nsr_residual_add_layernorm", "nsr_rope_table_f32",
                     "nsr_rope_qk_cache_append", "nsr_kv_cache_append",
                     "nsr_rotary_partial_interleaved_f32", "nsr_adain_snake_f32", "nsr_adain_snake_f16",
                     "nsr_q8_0_embed_gather",
                     "nsr_activation", "nsr_glu_silu", "nsr_residual_add", "nsr_gemv_q8",
                     "nsr_gemv_q8_bias_glu", "nsr_gemv_q8_resadd_ln", "nsr_q8_pack_t4", "nsr_gemv_q8_t4", "nsr_q8_0_to_gemv_q8", "nsr_q8_0_to_t4",
                     "nsr_conv1d_f32io", "nsr_conv1d_pack_f16", "nsr_conv1d_f16w_packed",
                     "nsr_adain_snake_conv1d_f32", "nsr_attention_splitkv_f16", "nsr_attention_decode_f16",
                     "nsr_scale_f32", "nsr_leaky_relu_f32", "nsr_resblock_average_f32", "nsr_istft_f32", "nsr_snake",
                     "nsr_adain_snake_conv1d_chain_f32", "nsr_conv1d_f16w_packed_stats",
                     "nsr_gemv_q8_t4_bias_glu", "nsr_gemv_q8_t4_resadd_ln", "nsr_calib_empty", "nsr_calib_copy",
                     "nsr_attention_splitkv_f16_noalloc", "nsr_conv1d_workspace_bytes", "nsr_calib_copy_rows",
                     "nsr_calib_adain_timeline"):
            getattr(L, name).restype = C.c_int
        _lib = L
    return _lib


def header_functions() -> list[str]:
    """Names of the functions include/nspeech_rocm.h declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nsr_[a-z0-9_]+)\s*\(", text)))


def check(status: int) -> None:
    if status != NSR_OK:
        raise NsrError(status, lib().nsr_last_error().decode())


def version() -> str:
    return lib().nsr_version().decode()


def init(code_object_dir: str | None = None) -> None:
    check(lib().nsr_init(code_object_dir.encode() if code_object_dir else None))


def _stream(stream) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _ptr(t: torch.Tensor | None):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("nspeech_rocm kernels take device tensors")
    if not t.is_contiguous():
        raise ValueError("nspeech_rocm kernels take contiguous tensors")
    return t.data_ptr()


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


# ------------------------------------------------------------------ ops ---

def layernorm(x, gamma=None, beta=None, *, eps=1e-5, unit_offset=False, act="none", out=None,
              out_dtype=None, stream=None):
    """LN over the last dim of a contiguous tensor."""
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    pdt = NSR_F32
    if gamma is not None:
        pdt = _dt(gamma)
    elif beta is not None:
        pdt = _dt(beta)
    check(lib().nsr_layernorm(_ptr(x), _dt(x), _ptr(gamma), _ptr(beta), pdt, _ptr(out), _dt(out), rows, cols,
                              cols, cols, eps, NSR_LN_UNIT_OFFSET if unit_offset else 0, ACT[act], _stream(stream)))
    return out


def residual_add_layernorm(x, res, gamma=None, beta=None, *, eps=1e-5, act="none", h_out=None, write_h=True,
                           out=None, h_dtype=None, out_dtype=None, unit_offset=False, stream=None):
    """Returns (h, y); h is None when write_h is False."""
    cols = x.shape[-1]
    rows = x.numel() // cols
    if write_h and h_out is None:
        h_out = torch.empty(x.shape, dtype=h_dtype or x.dtype, device=x.device)
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    hd = _dt(h_out) if h_out is not None else (_DT[h_dtype] if h_dtype is not None else _dt(x))
    pdt = _dt(gamma) if gamma is not None else (_dt(beta) if beta is not None else NSR_F32)
    check(lib().nsr_residual_add_layernorm(_ptr(x), _dt(x), _ptr(res), _dt(res), _ptr(h_out), hd, _ptr(gamma),
                                           _ptr(beta), pdt, _ptr(out), _dt(out), rows, cols, eps,
                                           NSR_LN_UNIT_OFFSET if unit_offset else 0, ACT[act], _stream(stream)))
    return h_out, out


def rope_table(max_pos: int, rotary_dim: int, theta: float) -> torch.Tensor:
    """Host-built f32 RoPE table [max_pos, rotary_dim] (CPU tensor)."""
    t = torch.empty((max_pos, rotary_dim), dtype=torch.float32)
    check(lib().nsr_rope_table_f32(t.data_ptr(), max_pos, rotary_dim, theta))
    return t


def rotary(q, k, rotary_dim, theta=10000.0, pos0=0, *, table=None, q_out=None, k_out=None, stream=None):
    """q [B,Hq,T,Dh], k [B,Hk,T,Dh] or None. Returns (q_out, k_out)."""
    B, Hq, T, Dh = q.shape
    Hk = k.shape[1] if k is not None else 0
    if q_out is None:
        q_out = torch.empty_like(q)
    if k is not None and k_out is None:
        k_out = torch.empty_like(k)
    rows = table.shape[0] if table is not None else 0
    check(lib().nsr_rotary_partial_interleaved_f32(_ptr(q), _ptr(k), _ptr(q_out), _ptr(k_out), B, Hq, Hk, T, Dh,
                                                   rotary_dim, theta, pos0, _ptr(table), rows, _stream(stream)))
    return q_out, k_out


def rope_qk_cache_append(q, k, v, table, cache_k, cache_v, pos, rotary_dim, *, stream=None):
    """Decode step, in place: q [Hq, Dh], k [Hk, Dh] rotated with table row pos;
    rotated k and v (or v None) written to the caches [Hk, L, Dh] at pos."""
    Hq, Dh = q.shape
    Hk = k.shape[0]
    check(lib().nsr_rope_qk_cache_append(_ptr(q), _ptr(k), _ptr(v), _dt(q), _ptr(table), table.shape[0],
                                         _ptr(cache_k), _ptr(cache_v), Hq, Hk, Dh, rotary_dim, pos, cache_k.shape[1],
                                         _stream(stream)))


def kv_cache_append(new_kv, cache, pos, *, stream=None):
    """cache[h, pos, :] = new_kv[h, :]; cache [Hk, L, Dh]."""
    Hk, L, Dh = cache.shape
    check(lib().nsr_kv_cache_append(_ptr(new_kv), _ptr(cache), _dt(cache), Hk, Dh, L, pos, _stream(stream)))


def adain_snake(x, gamma, beta, alpha, *, eps=1e-5, out=None, stream=None):
    """x [B,C,T] f32 or f16 (out the same dtype); gamma/beta [C] or [B,C]; alpha [C]; params f32 or f16."""
    B, Cc, T = x.shape
    if out is None:
        out = torch.empty_like(x)
    if out.dtype != x.dtype or x.dtype not in (torch.float32, torch.float16):
        raise ValueError("x and out must both be float32 or both float16")
    gs = Cc if gamma.dim() == 2 else 0
    bs = Cc if beta.dim() == 2 else 0
    fn = lib().nsr_adain_snake_f32 if x.dtype == torch.float32 else lib().nsr_adain_snake_f16
    check(fn(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(alpha), _dt(gamma), gs, bs, _ptr(out), B, Cc, T, eps,
             _stream(stream)))
    return out


def q8_0_embed_gather(blocks, vocab, d, ids, *, act="none", out=None, err_flag=None, stream=None):
    """blocks: uint8 device tensor of the GGUF Q8_0 table; ids int32/uint32 or int64."""
    n = ids.numel()
    if out is None:
        out = torch.empty((n, d), dtype=torch.float32, device=ids.device)
    idt = NSR_IDX_I64 if ids.dtype == torch.int64 else NSR_IDX_U32
    check(lib().nsr_q8_0_embed_gather(_ptr(blocks), vocab, d, _ptr(ids), idt, n, _ptr(out), ACT[act],
                                      _ptr(err_flag), _stream(stream)))
    return out


def activation(x, act, *, out=None, stream=None):
    if out is None:
        out = torch.empty_like(x)
    check(lib().nsr_activation(_ptr(x), _ptr(out), _dt(x), x.numel(), ACT[act], _stream(stream)))
    return out


def glu_silu(fc1, *, out=None, stream=None):
    n = fc1.numel() // 2
    if out is None:
        out = torch.empty(n, dtype=fc1.dtype, device=fc1.device)
    check(lib().nsr_glu_silu(_ptr(fc1), _ptr(out), _dt(fc1), n, _stream(stream)))
    return out


def residual_add(x, res, *, out=None, stream=None):
    if out is None:
        out = torch.empty_like(x)
    check(lib().nsr_residual_add(_ptr(x), _ptr(res), _ptr(out), _dt(x), x.numel(), _stream(stream)))
    return out


def _q8_shape(qs, scales):
    """K and weight columns of a repacked Q8 weight: qs int32/uint32 [K, NW/4],
    scales f16 [K/32, NW]."""
    if qs.dim() != 2 or scales.dim() != 2 or scales.dtype != torch.float16:
        raise ValueError("qs must be [K, NW/4] 32-bit words and scales [K/32, NW] f16")
    K, nw = qs.shape[0], 4 * qs.shape[1]
    if scales.shape[1] != nw or scales.shape[0] * 32 != K:
        raise ValueError(f"scales {tuple(scales.shape)} do not match qs {tuple(qs.shape)}")
    return K, nw


def gemv_q8(x, qs, scales, bias=None, *, out=None, out_dtype=torch.float16, stream=None):
    """out[N] = x[K] @ dequant(W) (+ bias); W in the repacked Q8 layout."""
    K, N = _q8_shape(qs, scales)
    if out is None:
        out = torch.empty(N, dtype=out_dtype, device=x.device)
    check(lib().nsr_gemv_q8(_ptr(x), _dt(x), _ptr(qs), _ptr(scales), _ptr(bias), _ptr(out), _dt(out), K, N,
                            _stream(stream)))
    return out


def gemv_q8_bias_glu(x, qs, scales, bias=None, *, out=None, out_dtype=torch.float16, stream=None):
    """out[N] = silu(x @ Wg + bg) * (x @ Wx + bx); W [K, 2N]: x half, then gate half."""
    K, nw = _q8_shape(qs, scales)
    N = nw // 2
    if out is None:
        out = torch.empty(N, dtype=out_dtype, device=x.device)
    check(lib().nsr_gemv_q8_bias_glu(_ptr(x), _dt(x), _ptr(qs), _ptr(scales), _ptr(bias), _ptr(out), _dt(out), K,
                                     N, _stream(stream)))
    return out


def gemv_q8_resadd_ln(x, qs, scales, residual, ln_weight, *, eps=1e-5, out_f32=None, norm=None,
                      norm_dtype=torch.float16, stream=None):
    """h = f16(x @ W) + residual (f32), norm = LN(h) * ln_weight. Returns (h, norm)."""
    K, dim = _q8_shape(qs, scales)
    if out_f32 is None:
        out_f32 = torch.empty(dim, dtype=torch.float32, device=x.device)
    if norm is None:
        norm = torch.empty(dim, dtype=norm_dtype, device=x.device)
    check(lib().nsr_gemv_q8_resadd_ln(_ptr(x), _dt(x), _ptr(qs), _ptr(scales), _ptr(residual), _ptr(out_f32),
                                      _ptr(ln_weight), _dt(ln_weight), _ptr(norm), _dt(norm), K, dim, eps,
                                      _stream(stream)))
    return out_f32, norm


class Q8T4:
    """A repacked-Q8 weight packed into t4 tiles on the device (nsr_q8_pack_t4),
    or built from a GGUF Q8_0 weight with Q8T4.from_q8_0."""

    def __init__(self, qs, scales, *, glu=False, stream=None):
        if qs is None:
            return
        K, nw = _q8_shape(qs, scales)
        self._alloc(K, nw, glu, qs.device)
        check(lib().nsr_q8_pack_t4(_ptr(qs), _ptr(scales), K, nw, 1 if glu else 0, _ptr(self.qs),
                                   _ptr(self.scales), _stream(stream)))

    def _alloc(self, K, nw, glu, device):
        self.K, self.NW, self.glu = K, nw, glu
        self.qs = torch.empty(K * nw // 4, dtype=torch.int32, device=device)
        self.scales = torch.empty((K // 32) * nw, dtype=torch.float16, device=device)

    @classmethod
    def from_q8_0(cls, blocks, N, K, *, glu=False, stream=None):
        """blocks: uint8 device tensor of a GGUF Q8_0 weight [N, K] (nn::Linear [out, in])."""
        w = cls(None, None)
        w._alloc(K, N, glu, blocks.device)
        check(lib().nsr_q8_0_to_t4(_ptr(blocks), N, K, 1 if glu else 0, _ptr(w.qs), _ptr(w.scales),
                                   _stream(stream)))
        return w


def q8_0_to_gemv_q8(blocks, N, K, *, stream=None):
    """GGUF Q8_0 weight [N, K] on the device -> (qs int32 [K, N/4], scales f16 [K/32, N]) of W^T."""
    qs = torch.empty((K, N // 4), dtype=torch.int32, device=blocks.device)
    sc = torch.empty((K // 32, N), dtype=torch.float16, device=blocks.device)
    check(lib().nsr_q8_0_to_gemv_q8(_ptr(blocks), N, K, _ptr(qs), _ptr(sc), _stream(stream)))
    return qs, sc


def gemv_q8_t4(x, w: Q8T4, bias=None, *, out=None, out_dtype=torch.float16, stream=None):
    N = w.NW
    if out is None:
        out = torch.empty(N, dtype=out_dtype, device=x.device)
    check(lib().nsr_gemv_q8_t4(_ptr(x), _dt(x), _ptr(w.qs), _ptr(w.scales), _ptr(bias), _ptr(out), _dt(out), w.K,
                               N, _stream(stream)))
    return out


def gemv_q8_t4_bias_glu(x, w: Q8T4, bias=None, *, out=None, out_dtype=torch.float16, stream=None):
    N = w.NW // 2
    if out is None:
        out = torch.empty(N, dtype=out_dtype, device=x.device)
    check(lib().nsr_gemv_q8_t4_bias_glu(_ptr(x), _dt(x), _ptr(w.qs), _ptr(w.scales), _ptr(bias), _ptr(out),
                                        _dt(out), w.K, N, _stream(stream)))
    return out


def gemv_q8_t4_resadd_ln(x, w: Q8T4, residual, ln_weight, *, eps=1e-5, out_f32=None, norm=None,
                         norm_dtype=torch.float16, stream=None):
    dim = w.NW
    if out_f32 is None:
        out_f32 = torch.empty(dim, dtype=torch.float32, device=x.device)
    if norm is None:
        norm = torch.empty(dim, dtype=norm_dtype, device=x.device)
    check(lib().nsr_gemv_q8_t4_resadd_ln(_ptr(x), _dt(x), _ptr(w.qs), _ptr(w.scales), _ptr(residual),
                                         _ptr(out_f32), _ptr(ln_weight), _dt(ln_weight), _ptr(norm), _dt(norm),
                                         w.K, dim, eps, _stream(stream)))
    return out_f32, norm


# ------------------------------------------------------ Kokoro conv1d ---

def _conv_tout(T, K, padding, dilation):
    return T + 2 * padding - dilation * (K - 1)


WS_PACKED_WEIGHTS, WS_IN_STATS, WS_OUT_STATS, WS_RECORDS = 1, 2, 4, 8


def conv1d_workspace_bytes(B, C_in, C_out, T, K, padding, dilation, parts) -> int:
    """Bytes of device workspace a conv entry point of this shape needs for `parts` (WS_* flags ORed)."""
    n = C.c_int64(0)
    check(lib().nsr_conv1d_workspace_bytes(B, C_in, C_out, T, K, padding, dilation, parts, C.byref(n)))
    return n.value


def conv_workspace(B, C_in, C_out, T, K, padding, dilation, parts, device="cuda"):
    """A device workspace (uint8 tensor, 256-byte aligned as torch allocates) for those parts, or None."""
    n = conv1d_workspace_bytes(B, C_in, C_out, T, K, padding, dilation, parts)
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def _ws(t):
    return (_ptr(t), t.numel()) if t is not None else (None, 0)


def conv1d_f32io(x, w, bias=None, *, padding=0, dilation=1, out=None, workspace=None, records=True, stream=None):
    """x f32 [B, C_in, T]; w f16 [C_out, C_in, K]; bias f16 [C_out] or None. The packed weights (and with
    `records`, the input records of the two-launch path) go to `workspace` (allocated here when not given)."""
    B, C_in, T = x.shape
    C_out, _, K = w.shape
    if out is None:
        out = torch.empty((B, C_out, _conv_tout(T, K, padding, dilation)), dtype=torch.float32, device=x.device)
    if workspace is None:
        workspace = conv_workspace(B, C_in, C_out, T, K, padding, dilation,
                                   WS_PACKED_WEIGHTS | (WS_RECORDS if records else 0), x.device)
    check(lib().nsr_conv1d_f32io(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), B, C_in, C_out, T, K, 1, padding,
                                 dilation, *_ws(workspace), _stream(stream)))
    return out


def conv1d_pack_f16(w, *, stream=None):
    """[C_out, C_in, K] f16 -> packed [C_out, K, C_in] f16."""
    C_out, C_in, K = w.shape
    wp = torch.empty((C_out, K, C_in), dtype=torch.float16, device=w.device)
    check(lib().nsr_conv1d_pack_f16(_ptr(w), C_out, C_in, K, _ptr(wp), _stream(stream)))
    return wp


def conv1d_f16w_packed(x, wp, bias=None, residual=None, *, padding=0, dilation=1, out=None, stream=None):
    B, C_in, T = x.shape
    C_out, K, _ = wp.shape
    if out is None:
        out = torch.empty((B, C_out, _conv_tout(T, K, padding, dilation)), dtype=torch.float32, device=x.device)
    check(lib().nsr_conv1d_f16w_packed(_ptr(x), _ptr(wp), _ptr(bias), _ptr(residual), _ptr(out), B, C_in, C_out, T,
                                       K, padding, dilation, _stream(stream)))
    return out


def adain_snake_conv1d_chain(x, gamma, beta, alpha, wp, bias=None, residual=None, *, x_stats=None, want_stats=True,
                             padding=0, dilation=1, eps=1e-5, out=None, records=True, stream=None):
    """adain_snake_conv1d with the row statistics handed along: x_stats f32 [B*C_in, 2] (mean, rstd) or None
    (computed here); returns (out, out_stats) with out_stats f32 [B*C_out, 2] (None if not want_stats).
    `records`: give the workspace the records part (the two-launch path where the rows qualify)."""
    B, C_in, T = x.shape
    C_out, K, _ = wp.shape
    if out is None:
        out = torch.empty((B, C_out, _conv_tout(T, K, padding, dilation)), dtype=torch.float32, device=x.device)
    st = torch.empty((B * C_out, 2), dtype=torch.float32, device=x.device) if want_stats else None
    gs = C_in if gamma.dim() == 2 else 0
    bs = C_in if beta.dim() == 2 else 0
    parts = (0 if x_stats is not None else WS_IN_STATS) | (WS_OUT_STATS if want_stats else 0) | \
        (WS_RECORDS if records else 0)
    ws = conv_workspace(B, C_in, C_out, T, K, padding, dilation, parts, x.device)
    check(lib().nsr_adain_snake_conv1d_chain_f32(_ptr(x), _ptr(x_stats), _ptr(gamma), _ptr(beta), _ptr(alpha),
                                                 _dt(gamma), gs, bs, _ptr(wp), _ptr(bias), _ptr(residual), _ptr(out),
                                                 _ptr(st), B, C_in, C_out, T, K, padding, dilation, eps, *_ws(ws),
                                                 _stream(stream)))
    return out, st


def conv1d_f16w_packed_stats(x, wp, bias=None, residual=None, *, padding=0, dilation=1, eps=1e-5, out=None,
                             records=True, stream=None):
    """conv1d_f16w_packed that also returns the output rows' (mean, rstd) f32 [B*C_out, 2]."""
    B, C_in, T = x.shape
    C_out, K, _ = wp.shape
    if out is None:
        out = torch.empty((B, C_out, _conv_tout(T, K, padding, dilation)), dtype=torch.float32, device=x.device)
    st = torch.empty((B * C_out, 2), dtype=torch.float32, device=x.device)
    ws = conv_workspace(B, C_in, C_out, T, K, padding, dilation, WS_OUT_STATS | (WS_RECORDS if records else 0),
                        x.device)
    check(lib().nsr_conv1d_f16w_packed_stats(_ptr(x), _ptr(wp), _ptr(bias), _ptr(residual), _ptr(out), _ptr(st), B,
                                             C_in, C_out, T, K, padding, dilation, eps, *_ws(ws), _stream(stream)))
    return out, st


def adain_snake_conv1d(x, gamma, beta, alpha, wp, bias=None, residual=None, *, padding=0, dilation=1, eps=1e-5,
                       out=None, records=True, stream=None):
    """conv1d(snake(AdaIN(x))) + bias (+ residual); x f32 [B, C_in, T]; gamma/beta [C_in] or [B, C_in];
    alpha [C_in] (f32 or f16); wp packed f16 [C_out, K, C_in]."""
    B, C_in, T = x.shape
    C_out, K, _ = wp.shape
    if out is None:
        out = torch.empty((B, C_out, _conv_tout(T, K, padding, dilation)), dtype=torch.float32, device=x.device)
    gs = C_in if gamma.dim() == 2 else 0
    bs = C_in if beta.dim() == 2 else 0
    ws = conv_workspace(B, C_in, C_out, T, K, padding, dilation, WS_IN_STATS | (WS_RECORDS if records else 0),
                        x.device)
    check(lib().nsr_adain_snake_conv1d_f32(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(alpha), _dt(gamma), gs, bs,
                                           _ptr(wp), _ptr(bias), _ptr(residual), _ptr(out), B, C_in, C_out, T, K,
                                           padding, dilation, eps, *_ws(ws), _stream(stream)))
    return out


# ------------------------------------------------------ decode attention ---

def attention_decode(q, k, v, kv_len, n_kv_heads, sm_scale, *, stride_kv_head, stride_kv_seq, n_splits=None,
                     partial=None, out=None, stream=None):
    """f16 q [n_q_heads, head_dim]; k, v f16 device tensors addressed as (head, pos, d) ->
    head * stride_kv_head + pos * stride_kv_seq + d. n_splits None: the library picks the split
    (nsr_attention_decode_f16); else nsr_attention_splitkv_f16 with `partial` (allocated if None)."""
    n_q_heads, head_dim = q.shape
    if out is None:
        out = torch.empty((n_q_heads, head_dim), dtype=torch.float16, device=q.device)
    if n_splits is None:
        check(lib().nsr_attention_decode_f16(_ptr(q), _ptr(k), _ptr(v), _ptr(out), kv_len, head_dim, n_kv_heads,
                                             n_q_heads, sm_scale, stride_kv_head, stride_kv_seq, _stream(stream)))
    else:
        if partial is None:
            partial = torch.empty(n_q_heads * n_splits * (head_dim + 2), dtype=torch.float32, device=q.device)
        check(lib().nsr_attention_splitkv_f16(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(partial), kv_len, head_dim,
                                              n_kv_heads, n_q_heads, sm_scale, stride_kv_head, stride_kv_seq,
                                              n_splits, _stream(stream)))
    return out


# ------------------------------------------------- Kokoro generator tail ---

def _same_f32(*ts):
    n = ts[0].numel()
    for t in ts:
        if t.dtype != torch.float32:
            raise ValueError("expected float32 tensors")
        if t.numel() != n:
            raise ValueError("element counts differ")
    return n


def snake(x, alpha, *, out=None, stream=None):
    """x [..., C, T] f32 or f16 (out the same dtype), alpha [C] f32 or f16."""
    out = torch.empty_like(x) if out is None else out
    if out.dtype != x.dtype or out.numel() != x.numel():
        raise ValueError("out must match x")
    C, T = alpha.numel(), x.shape[-1]
    check(lib().nsr_snake(_ptr(x), _dt(x), _ptr(alpha), _dt(alpha), _ptr(out), x.numel(), C, T, _stream(stream)))
    return out


def scale_f32(x, s, *, out=None, stream=None):
    out = torch.empty_like(x) if out is None else out
    n = _same_f32(x, out)
    check(lib().nsr_scale_f32(_ptr(x), _ptr(out), n, s, _stream(stream)))
    return out


def leaky_relu_f32(x, slope, *, out=None, stream=None):
    out = torch.empty_like(x) if out is None else out
    n = _same_f32(x, out)
    check(lib().nsr_leaky_relu_f32(_ptr(x), _ptr(out), n, slope, _stream(stream)))
    return out


def resblock_average_f32(r0, r1, r2, *, leaky_slope=None, out=None, stream=None):
    """((r0 + r1) + r2) * f32(1/3), then leaky ReLU when leaky_slope is given."""
    out = torch.empty_like(r0) if out is None else out
    n = _same_f32(r0, r1, r2, out)
    check(lib().nsr_resblock_average_f32(_ptr(r0), _ptr(r1), _ptr(r2), _ptr(out), n,
                                         0 if leaky_slope is None else 1,
                                         0.0 if leaky_slope is None else leaky_slope, _stream(stream)))
    return out


def istft_f32(x, *, n_fft=20, hop=5, out_len=None, out=None, stream=None):
    """x f32 [2 (n_fft/2 + 1), n_frames] (log-magnitude, raw phase) -> audio f32 [(n_frames - 1) hop]."""
    if x.dim() != 2 or x.shape[0] != 2 * (n_fft // 2 + 1) or x.dtype != torch.float32:
        raise ValueError("x must be f32 [2 * (n_fft // 2 + 1), n_frames]")
    n_frames = x.shape[1]
    out_len = (n_frames - 1) * hop if out_len is None else out_len
    out = torch.empty(out_len, dtype=torch.float32, device=x.device) if out is None else out
    if out.dtype != torch.float32 or out.numel() < out_len:
        raise ValueError("out must be f32 with at least out_len elements")
    check(lib().nsr_istft_f32(_ptr(x), _ptr(out), n_frames, out_len, n_fft, hop, _stream(stream)))
    return out
