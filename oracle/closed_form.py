"""float64 closed forms of the hot-path ops (TEST INFRASTRUCTURE).

Independent of the C restatement: plain numpy in float64 (math.erf for GELU),
written from the mathematics of each op. Used to pin the restatement and to
bound the HIP kernels' error at sizes where the C oracle would be slow.
"""
from __future__ import annotations

import math

import numpy as np


def layernorm(x, w=None, b=None, eps=1e-5, unit_offset=False):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    scale = np.ones(x.shape[-1]) if w is None else np.asarray(w, np.float64)
    if unit_offset:
        scale = scale + 1.0
    y = y * scale
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return y


def gelu_erf(x):
    x = np.asarray(x, np.float64)
    erf = np.vectorize(math.erf, otypes=[np.float64])
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def inv_freq_f32(rot: int, theta: float) -> np.ndarray:
    """inv_freq with the reference's f32 roundings: exponent e = f32(2i/rot),
    p = f32(theta^e) (the power correctly rounded from float64), 1/p in f32."""
    i = np.arange(rot // 2, dtype=np.float32)
    e = (np.float32(2.0) * i) / np.float32(rot)
    p = np.power(np.float64(np.float32(theta)), e.astype(np.float64)).astype(np.float32)
    return np.float32(1.0) / p


def rotary(x, rot: int, theta: float, pos0: int = 0, inv_freq=None):
    """Rotation of interleaved pairs as complex multiplication by e^{i angle}.

    angle = f32(f32(pos) * inv_freq) (the reference's f32 angle), cos/sin of
    that angle in float64. x [B, H, T, Dh]."""
    x = np.asarray(x, np.float64)
    B, H, T, Dh = x.shape
    f = inv_freq_f32(rot, theta) if inv_freq is None else np.asarray(inv_freq, np.float32)
    pos = (pos0 + np.arange(T)).astype(np.float32)
    ang = (pos[:, None] * f[None, :]).astype(np.float32).astype(np.float64)  # [T, half]
    z = x[..., :rot:2] + 1j * x[..., 1:rot:2]  # [B, H, T, half]
    zr = z * np.exp(1j * ang)[None, None]
    out = x.copy()
    out[..., :rot:2] = zr.real
    out[..., 1:rot:2] = zr.imag
    return out


def adain_snake(x, gamma, beta, alpha, eps=1e-5):
    """x [B, C, T]; gamma/beta [C] or [B, C]; alpha [C]."""
    x = np.asarray(x, np.float64)
    B, C, T = x.shape
    g = np.broadcast_to(np.asarray(gamma, np.float64), (B, C))[..., None]
    bt = np.broadcast_to(np.asarray(beta, np.float64), (B, C))[..., None]
    a = np.asarray(alpha, np.float64)[None, :, None]
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps) * (1.0 + g) + bt
    # recip(alpha + 1e-9) is an f32 tensor op in the reference (decoder.rs:1474)
    inv_a = (np.float32(1.0) / (np.asarray(alpha, np.float32) + np.float32(1e-9))).astype(np.float64)[None, :, None]
    return y + np.sin(a * y) ** 2 * inv_a


def q8_0_decode(blocks: np.ndarray, vocab: int, d: int) -> np.ndarray:
    """GGUF Q8_0 table decoded with a numpy structured dtype {<f2 d, i1 qs[32]}."""
    dt = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])
    rec = np.frombuffer(np.ascontiguousarray(blocks, np.uint8).tobytes(), dtype=dt)
    rec = rec.reshape(vocab, d // 32)
    vals = rec["qs"].astype(np.float64) * rec["d"].astype(np.float64)[..., None]
    return vals.reshape(vocab, d)
