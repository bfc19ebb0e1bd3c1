"""Synthetic workloads of the benchmark configurations (numpy, seeded).

configs[0..4] of the benchmark definition, with numpy PCG64 seeds
1000 + config index (4a: 1004, 4b: 1005). Distributions and shapes:

  c0  LayerNorm f32 x[1,125,1024] ~N(0,1), gamma ~N(1,0.02), beta ~N(0,0.02), eps 1e-5
  c1  partial rotary f32 q,k [1,8,1024,64] ~N(0,1), rot 32, theta 1e4, pos 0..1023
  c2  AdaIN1d+Snake f32 x[1,512,4800] ~N(0,1), gamma,beta[512] ~N(0,0.1), alpha ~U(0.5,1.5)
  c3  Q8_0 gather: 32768 x 416 table, qs ~U{-127..127}, d = f16(U(1e-3,2e-2)),
      4096 ids ~U[0,32768), f32 out [4096,416], SiLU fused
  c4a residual add + LN + GELU(erf) bf16 x,res[32,750,1024] ~N(0,1), eps 1e-5,
      gamma = bf16(1+N(0,0.02)), beta = bf16(N(0,0.02)) (bf16-exact f32 values)
  c4b AdaIN1d+Snake f32 x[8,128,115200] ~N(0,1), gamma,beta[8,128] ~N(0,0.1),
      alpha[128] ~U(0.5,1.5)

Each generator returns a dict of numpy arrays (bf16 tensors as uint16 bits).
"""
from __future__ import annotations

import numpy as np

Q8_BLOCK = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])  # 34 bytes, GGUF block_q8_0


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (numpy)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_q8_0_table(g: np.random.Generator, vocab: int, d: int) -> np.ndarray:
    """GGUF Q8_0 table bytes [vocab * d/32 * 34] (uint8)."""
    nb = d // 32
    rec = np.empty(vocab * nb, dtype=Q8_BLOCK)
    rec["d"] = g.uniform(1e-3, 2e-2, size=vocab * nb).astype(np.float16)
    rec["qs"] = g.integers(-127, 128, size=(vocab * nb, 32), dtype=np.int8)
    return rec.view(np.uint8).copy()


def c0(seed: int = 1000):
    g = rng(seed)
    return {
        "x": g.standard_normal((1, 125, 1024), dtype=np.float32),
        "gamma": (1.0 + 0.02 * g.standard_normal(1024)).astype(np.float32),
        "beta": (0.02 * g.standard_normal(1024)).astype(np.float32),
        "eps": 1e-5,
    }


def c1(seed: int = 1001, B=1, H=8, T=1024, Dh=64):
    g = rng(seed)
    return {
        "q": g.standard_normal((B, H, T, Dh), dtype=np.float32),
        "k": g.standard_normal((B, H, T, Dh), dtype=np.float32),
        "rot": 32,
        "theta": 10000.0,
        "pos0": 0,
    }


def c2(seed: int = 1002, B=1, C=512, T=4800):
    g = rng(seed)
    return {
        "x": g.standard_normal((B, C, T), dtype=np.float32),
        "gamma": (0.1 * g.standard_normal(C)).astype(np.float32),
        "beta": (0.1 * g.standard_normal(C)).astype(np.float32),
        "alpha": g.uniform(0.5, 1.5, size=C).astype(np.float32),
        "eps": 1e-5,
    }


def c3(seed: int = 1003, vocab=32768, d=416, n_ids=4096):
    g = rng(seed)
    return {
        "blocks": make_q8_0_table(g, vocab, d),
        "vocab": vocab,
        "d": d,
        "ids": g.integers(0, vocab, size=n_ids, dtype=np.int64).astype(np.uint32),
    }


def c4a(seed: int = 1004, rows=32 * 750, cols=1024):
    g = rng(seed)
    x = f32_to_bf16_bits(g.standard_normal((rows, cols), dtype=np.float32))
    res = f32_to_bf16_bits(g.standard_normal((rows, cols), dtype=np.float32))
    gamma = bf16_bits_to_f32(f32_to_bf16_bits((1.0 + 0.02 * g.standard_normal(cols)).astype(np.float32)))
    beta = bf16_bits_to_f32(f32_to_bf16_bits((0.02 * g.standard_normal(cols)).astype(np.float32)))
    return {"x": x, "res": res, "gamma": gamma, "beta": beta, "eps": 1e-5}


def c4b(seed: int = 1005, B=8, C=128, T=115200):
    g = rng(seed)
    return {
        "x": g.standard_normal((B, C, T), dtype=np.float32),
        "gamma": (0.1 * g.standard_normal((B, C))).astype(np.float32),
        "beta": (0.1 * g.standard_normal((B, C))).astype(np.float32),
        "alpha": g.uniform(0.5, 1.5, size=C).astype(np.float32),
        "eps": 1e-5,
    }


def kokoro_kat(channels: int, seq_len: int):
    """Known-answer inputs of the reference's Kokoro GPU self-tests
    (src/kokoro/gpu_decoder.rs:84-87, :308-311): x[i] = sin(0.001 i) * 3 in
    f32, gamma/beta/alpha per channel rounded to f16."""
    i = np.arange(channels * seq_len, dtype=np.float32)
    x = (np.sin(i * np.float32(0.001)) * np.float32(3.0)).astype(np.float32)
    c = np.arange(channels, dtype=np.float32)
    gamma = (np.sin(c * np.float32(0.01)) * np.float32(0.5)).astype(np.float16)
    beta = (np.cos(c * np.float32(0.02)) * np.float32(0.3)).astype(np.float16)
    alpha = (np.float32(1.0) + np.sin(c * np.float32(0.005))).astype(np.float16)
    return {"x": x.reshape(1, channels, seq_len), "gamma": gamma, "beta": beta, "alpha": alpha}


# Algorithmic HBM bytes per call (minimum traffic of each kernel contract).
def algorithmic_bytes(name: str) -> int:
    return {
        "c0": 4 * (2 * 125 * 1024 + 2 * 1024),
        "c1": 4 * (4 * 8 * 1024 * 64),
        "c2": 4 * (2 * 512 * 4800 + 3 * 512),
        "c3": 4096 * 442 + 4096 * 4 + 4096 * 416 * 4,
        "c4a": 2 * 4 * 32 * 750 * 1024 + 2 * 4 * 1024,
        "c4b": 4 * (2 * 8 * 128 * 115200 + 2 * 8 * 128 + 128),
    }[name]
