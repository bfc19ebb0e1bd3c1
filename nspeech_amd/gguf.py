"""ctypes binding of the GGUF reader (include/nspeech_gguf.h, in
libnspeech_rocm_host.so): parse a GGUF model file and copy its tensors to the
GPU as stored (Q8_0 tables stay Q8_0 in HBM).

    with GgufFile("moonshine_q8_0.gguf") as g:
        emb = g.upload("model.decoder.embed_tokens.weight")   # uint8 device tensor
        vocab, dim = g.tensor("model.decoder.embed_tokens.weight").shape
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi

HOST_LIB_PATH = abi.LIB_DIR / "libnspeech_rocm_host.so"

GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
(U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64) = range(13)
_INT_TYPES = {U8, I8, U16, I16, U32, I32, U64, I64, BOOL}


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("shape", C.c_int64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("data", C.c_void_p)]


@dataclass(frozen=True)
class TensorInfo:
    name: str
    type: int
    shape: tuple          # outermost first
    offset: int           # from the start of the file
    nbytes: int


class GgufError(RuntimeError):
    pass


_hl = None


def host_lib() -> C.CDLL:
    global _hl
    if _hl is None:
        abi.lib()  # the host library links against libnspeech_rocm.so
        if not HOST_LIB_PATH.exists():
            raise ImportError(f"{HOST_LIB_PATH} is not built: run `python -m nspeech_amd.build`")
        L = C.CDLL(str(HOST_LIB_PATH))
        P, I64, U64 = C.c_void_p, C.c_int64, C.c_uint64
        L.nsr_gguf_open.argtypes = [C.c_char_p, C.POINTER(P)]
        L.nsr_gguf_open_buffer.argtypes = [P, U64, C.POINTER(P)]
        L.nsr_gguf_close.argtypes = [P]
        L.nsr_gguf_close.restype = None
        L.nsr_gguf_last_error.restype = C.c_char_p
        for n, r in (("nsr_gguf_version", C.c_uint32), ("nsr_gguf_alignment", U64), ("nsr_gguf_data_offset", U64),
                     ("nsr_gguf_tensor_count", I64), ("nsr_gguf_metadata_count", I64)):
            getattr(L, n).argtypes = [P]
            getattr(L, n).restype = r
        L.nsr_gguf_tensor_at.argtypes = [P, I64, C.POINTER(_Tensor)]
        L.nsr_gguf_find_tensor.argtypes = [P, C.c_char_p, C.POINTER(_Tensor)]
        L.nsr_gguf_upload.argtypes = [P, C.POINTER(_Tensor), P, P]
        L.nsr_gguf_metadata_at.argtypes = [P, I64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32)]
        L.nsr_gguf_get_int.argtypes = [P, C.c_char_p, C.POINTER(I64)]
        L.nsr_gguf_get_float.argtypes = [P, C.c_char_p, C.POINTER(C.c_double)]
        L.nsr_gguf_get_string.argtypes = [P, C.c_char_p, C.POINTER(C.c_char_p)]
        L.nsr_gguf_get_array.argtypes = [P, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(U64)]
        L.nsr_gguf_get_array_int.argtypes = [P, C.c_char_p, U64, C.POINTER(I64)]
        L.nsr_gguf_get_array_float.argtypes = [P, C.c_char_p, U64, C.POINTER(C.c_double)]
        L.nsr_gguf_get_array_string.argtypes = [P, C.c_char_p, U64, C.POINTER(C.c_char_p)]
        _hl = L
    return _hl


def _check(st: int) -> None:
    if st != abi.NSR_OK:
        raise GgufError(host_lib().nsr_gguf_last_error().decode())


class GgufFile:
    """A parsed GGUF file (memory-mapped) or in-memory image (bytes)."""

    def __init__(self, path=None, *, buffer: bytes | None = None):
        L = host_lib()
        self._h = C.c_void_p()
        self._buf = None
        if buffer is not None:
            self._buf = C.create_string_buffer(bytes(buffer), len(buffer))
            _check(L.nsr_gguf_open_buffer(C.cast(self._buf, C.c_void_p), len(buffer), C.byref(self._h)))
        else:
            _check(L.nsr_gguf_open(str(path).encode(), C.byref(self._h)))

    def close(self):
        if self._h:
            host_lib().nsr_gguf_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self) -> int:
        return host_lib().nsr_gguf_version(self._h)

    @property
    def alignment(self) -> int:
        return host_lib().nsr_gguf_alignment(self._h)

    @property
    def data_offset(self) -> int:
        return host_lib().nsr_gguf_data_offset(self._h)

    def _raw(self, name: str) -> _Tensor:
        t = _Tensor()
        _check(host_lib().nsr_gguf_find_tensor(self._h, name.encode(), C.byref(t)))
        return t

    @staticmethod
    def _info(t: _Tensor) -> TensorInfo:
        return TensorInfo(t.name.decode(), t.type, tuple(t.shape[: t.n_dims]), t.offset, t.nbytes)

    def tensors(self) -> list[TensorInfo]:
        out = []
        for i in range(host_lib().nsr_gguf_tensor_count(self._h)):
            t = _Tensor()
            _check(host_lib().nsr_gguf_tensor_at(self._h, i, C.byref(t)))
            out.append(self._info(t))
        return out

    def tensor(self, name: str) -> TensorInfo:
        return self._info(self._raw(name))

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's stored bytes (host)."""
        t = self._raw(name)
        return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_uint8)), shape=(t.nbytes,)).copy() \
            if t.nbytes else np.zeros(0, np.uint8)

    def upload(self, name: str, *, out=None, stream=None):
        """The tensor's stored bytes as a uint8 device tensor (copy enqueued on `stream`)."""
        import torch

        t = self._raw(name)
        if out is None:
            out = torch.empty(t.nbytes, dtype=torch.uint8, device="cuda")
        if out.numel() * out.element_size() < t.nbytes:
            raise ValueError("output tensor too small")
        _check(host_lib().nsr_gguf_upload(self._h, C.byref(t), out.data_ptr(), abi._stream(stream)))
        return out

    def metadata(self) -> dict:
        L = host_lib()
        out = {}
        for i in range(L.nsr_gguf_metadata_count(self._h)):
            k, ty = C.c_char_p(), C.c_uint32()
            _check(L.nsr_gguf_metadata_at(self._h, i, C.byref(k), C.byref(ty)))
            out[k.value.decode()] = self._value(k.value, ty.value)
        return out

    def _value(self, key: bytes, ty: int):
        L = host_lib()
        if ty in _INT_TYPES:
            v = C.c_int64()
            _check(L.nsr_gguf_get_int(self._h, key, C.byref(v)))
            return bool(v.value) if ty == BOOL else v.value
        if ty in (F32, F64):
            v = C.c_double()
            _check(L.nsr_gguf_get_float(self._h, key, C.byref(v)))
            return v.value
        if ty == STRING:
            v = C.c_char_p()
            _check(L.nsr_gguf_get_string(self._h, key, C.byref(v)))
            return v.value.decode()
        et, n = C.c_uint32(), C.c_uint64()
        _check(L.nsr_gguf_get_array(self._h, key, C.byref(et), C.byref(n)))
        vals = []
        for j in range(n.value):
            if et.value in _INT_TYPES:
                v = C.c_int64()
                _check(L.nsr_gguf_get_array_int(self._h, key, j, C.byref(v)))
                vals.append(v.value)
            elif et.value in (F32, F64):
                v = C.c_double()
                _check(L.nsr_gguf_get_array_float(self._h, key, j, C.byref(v)))
                vals.append(v.value)
            elif et.value == STRING:
                v = C.c_char_p()
                _check(L.nsr_gguf_get_array_string(self._h, key, j, C.byref(v)))
                vals.append(v.value.decode())
            else:
                vals.append(None)  # nested arrays: reported as None by this binding
        return vals
