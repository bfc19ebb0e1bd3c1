"""Pin the CPU oracle (oracle/nsr_oracle.c) before trusting it (CPU only).

Every restated function is checked against something it was not written
from: torch/numpy library routines in float64, numpy's own float16/bfloat16
conversions, a complex-number formulation of the rotation, the structured
GGUF block decode, and invariants chosen so that a plausible mistake (a
dropped eps, a wrong pair sign, a transposed index, n-1 instead of n) fails.
"""
import math

import numpy as np
import pytest
import torch

from nspeech_amd import configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_F32, assert_bitexact, assert_close, rel_err


# ------------------------------------------------------------- dtypes ---

def test_f16_decode_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = R.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bitexact(got[~nan], ref[~nan], "f16 -> f32")


def test_bf16_rounding_matches_torch():
    g = configs.rng(7)
    x = np.concatenate([
        g.standard_normal(100000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32),
        # exact ties: 1 + k*2^-8 + 2^-9 (round half to even)
        (1.0 + np.arange(16) / 256.0 + 1.0 / 512.0).astype(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_bitexact(R.f32_to_bf16_bits(x), ref, "oracle f32->bf16")
    assert_bitexact(configs.f32_to_bf16_bits(x), ref, "configs f32->bf16")
    back = R.bf16_bits_to_f32(ref)
    assert_bitexact(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy(), "bf16->f32")


# --------------------------------------------------------------- Q8_0 ---

def test_q8_0_dequant_matches_structured_decode():
    g = configs.rng(11)
    vocab, d = 257, 96
    blocks = configs.make_q8_0_table(g, vocab, d)
    got = R.q8_0_dequantize(blocks, vocab, d)
    ref = CF.q8_0_decode(blocks, vocab, d)
    # int8 * f16 is exact in f32, so the f64 decode rounds to the same f32
    assert_bitexact(got, ref.astype(np.float32), "q8_0 dequant")


def test_q8_0_known_blocks():
    # block 0: d = 0.5, qs = -127..-96 ; block 1: d = smallest f16 subnormal, qs = 127
    rec = np.zeros(2, dtype=configs.Q8_BLOCK)
    rec["d"][0] = np.float16(0.5)
    rec["qs"][0] = np.arange(-127, -95, dtype=np.int8)
    rec["d"][1] = np.uint16(1).view(np.float16)
    rec["qs"][1] = 127
    got = R.q8_0_dequantize(rec.view(np.uint8), 1, 64)
    exp0 = np.arange(-127, -95, dtype=np.float32) * np.float32(0.5)
    exp1 = np.full(32, 127 * 2.0 ** -24, np.float32)
    assert_bitexact(got[0, :32], exp0, "block 0")
    assert_bitexact(got[0, 32:], exp1, "block 1")


def test_q8_0_embedding_is_row_select_of_dequant():
    g = configs.rng(12)
    vocab, d = 50, 64
    blocks = configs.make_q8_0_table(g, vocab, d)
    ids = np.array([0, 49, 3, 3, 17, 49, 0], np.int64)
    out, bad = R.q8_0_embedding(blocks, vocab, d, ids)
    assert bad == 0
    dense = CF.q8_0_decode(blocks, vocab, d).astype(np.float32)
    assert_bitexact(out, dense[ids], "embedding rows")
    out2, bad2 = R.q8_0_embedding(blocks, vocab, d, np.array([1, 50, -1], np.int64))
    assert bad2 == 2 and not out2[1:].any()
    silu, _ = R.q8_0_embedding(blocks, vocab, d, ids, act=1)
    ref = torch.nn.functional.silu(torch.from_numpy(dense[ids].astype(np.float64))).numpy()
    assert_close(silu, ref, 1e-6, "embedding + silu vs torch f64")


# -------------------------------------------------------- activations ---

def _act_inputs():
    g = configs.rng(13)
    return np.concatenate([g.standard_normal(20000).astype(np.float32) * 4,
                           np.linspace(-30, 30, 2001, dtype=np.float32),
                           np.array([0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, -104.0], np.float32)])


def test_silu_matches_torch_f64():
    x = _act_inputs()
    ref = torch.nn.functional.silu(torch.from_numpy(x.astype(np.float64))).numpy()
    assert_close(R.silu(x), ref, 1e-6, "silu")
    assert R.silu(np.zeros(1, np.float32))[0] == 0.0


def test_gelu_erf_matches_torch_f64():
    x = _act_inputs()
    ref = torch.nn.functional.gelu(torch.from_numpy(x.astype(np.float64)), approximate="none").numpy()
    assert_close(R.gelu_erf(x), ref, 1e-6, "gelu")
    # odd part of gelu is x/2: gelu(x) - gelu(-x) = x
    xs = np.linspace(-5, 5, 101).astype(np.float32)
    assert_close(R.gelu_erf(xs).astype(np.float64) - R.gelu_erf(-xs), xs, 1e-6, "gelu odd part")
    assert np.array_equal(CF.gelu_erf(x[:50]), CF.gelu_erf(x[:50]))


def test_glu_and_fast_add():
    g = configs.rng(14)
    fc1 = g.standard_normal(2 * 1000).astype(np.float32)
    ref = torch.nn.functional.silu(torch.from_numpy(fc1[1000:].astype(np.float64))).numpy() * fc1[:1000]
    assert_close(R.glu_silu(fc1), ref, 1e-6, "glu")
    a, b = g.standard_normal(999).astype(np.float32), g.standard_normal(999).astype(np.float32)
    assert_bitexact(R.fast_add(a, b), a + b, "fast_add")


# --------------------------------------------------------- LayerNorm ---

def test_layernorm_candle_matches_torch_f64():
    c = configs.c0()
    ref = torch.nn.functional.layer_norm(torch.from_numpy(c["x"].astype(np.float64)), (1024,),
                                         torch.from_numpy(c["gamma"].astype(np.float64)),
                                         torch.from_numpy(c["beta"].astype(np.float64)), eps=1e-5).numpy()
    e1 = assert_close(R.layernorm_candle(c["x"], c["gamma"], c["beta"]), ref, RTOL_F32, "candle LN")
    e2 = assert_close(R.layernorm_twopass(c["x"], c["gamma"], c["beta"]), ref, RTOL_F32, "two-pass LN")
    assert e1 < 2e-6 and e2 < 2e-6


def test_layernorm_unit_offset_and_invariants():
    g = configs.rng(15)
    x = (g.standard_normal((64, 288)) * 3 + 5).astype(np.float32)
    w = (0.1 * g.standard_normal(288)).astype(np.float32)
    got = R.layernorm_twopass(x, w, unit_offset=True)
    assert_close(got, CF.layernorm(x, w, unit_offset=True), RTOL_F32, "unit offset LN")
    # no affine: per-row mean 0 and variance var/(var+eps)
    y = R.layernorm_twopass(x).astype(np.float64)
    var = x.astype(np.float64).var(axis=-1)
    assert np.abs(y.mean(axis=-1)).max() < 1e-6
    assert np.abs(y.var(axis=-1) - var / (var + 1e-5)).max() < 1e-5
    # constant row -> exactly beta (x - mean == 0)
    xc = np.full((2, 128), 0.5, np.float32)
    b = g.standard_normal(128).astype(np.float32)
    assert_bitexact(R.layernorm_candle(xc, np.ones(128, np.float32), b)[0], b, "constant row")
    assert_bitexact(R.layernorm_twopass(xc, np.ones(128, np.float32), b)[1], b, "constant row")


def test_resadd_ln_gelu_bf16_chain():
    c = configs.c4a(rows=96)
    wb = configs.f32_to_bf16_bits(c["gamma"])
    bb = configs.f32_to_bf16_bits(c["beta"])
    h, y = R.resadd_ln_gelu_bf16(c["x"], c["res"], wb, bb)
    xf, rf = configs.bf16_bits_to_f32(c["x"]), configs.bf16_bits_to_f32(c["res"])
    h_ref = torch.from_numpy(xf + rf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_bitexact(h, h_ref, "h = bf16(x + res)")
    hf = configs.bf16_bits_to_f32(h).astype(np.float64)
    ref = CF.gelu_erf(CF.layernorm(hf, c["gamma"], c["beta"]))
    yf = configs.bf16_bits_to_f32(y)
    assert_close(yf, ref, 1e-2, "bf16 chain vs f64")
    # the chain rounds n = LN(h)*w+b to bf16 (unit roundoff 2^-8 |n|, carried
    # by gelu' <= 1.13) and then y (2^-8 |y|): bound each element by that
    n = CF.layernorm(hf, c["gamma"], c["beta"])
    bound = 1.13 * 2.0 ** -8 * np.abs(n) * 1.01 + 2.0 ** -8 * np.abs(ref) * 1.01 + 1e-6
    assert np.all(np.abs(yf - ref) <= bound)


# ------------------------------------------------------------ rotary ---

def test_rope_table_matches_f64_of_f32_angles():
    tab = R.rope_table(1024, 32, 10000.0)
    f = CF.inv_freq_f32(32, 10000.0)
    ang = (np.arange(1024, dtype=np.float32)[:, None] * f[None, :]).astype(np.float32).astype(np.float64)
    assert_close(tab[:, :16], np.cos(ang), 1.2e-7, "cos")
    assert_close(tab[:, 16:], np.sin(ang), 1.2e-7, "sin")


def test_rope_table_of_product_equals_oracle():
    """The library's host-side table builder (CPU only) equals the oracle's."""
    from nspeech_amd import abi

    for max_pos, rot, theta in [(1024, 32, 10000.0), (17, 64, 500000.0), (3, 4, 10.0)]:
        assert_bitexact(abi.rope_table(max_pos, rot, theta).numpy(), R.rope_table(max_pos, rot, theta),
                        f"table {max_pos},{rot},{theta}")


def test_rotary_matches_complex_rotation():
    c = configs.c1(T=256)
    for pos0 in (0, 700):
        got = R.rotary(c["q"], c["rot"], c["theta"], pos0)
        ref = CF.rotary(c["q"], c["rot"], c["theta"], pos0)
        assert_close(got, ref, 1e-6, f"rotary pos0={pos0}")


def test_rotary_invariants():
    c = configs.c1(T=64)
    q = c["q"]
    out = R.rotary(q, 32, 10000.0, 0)
    assert_bitexact(out[:, :, 0], q[:, :, 0], "position 0 is identity")
    assert_bitexact(out[..., 32:], q[..., 32:], "pass-through dims")
    n_in = q[..., :32:2].astype(np.float64) ** 2 + q[..., 1:32:2].astype(np.float64) ** 2
    n_out = out[..., :32:2].astype(np.float64) ** 2 + out[..., 1:32:2].astype(np.float64) ** 2
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-3)) < 1e-5
    # a rotation by +angle (not -angle): pair (1, 0) at pos 1, i=0 goes to (cos 1, sin 1)
    e = np.zeros((1, 1, 2, 4), np.float32)
    e[0, 0, 1, 0] = 1.0
    o = R.rotary(e, 4, 10000.0, 0)
    assert abs(o[0, 0, 1, 0] - math.cos(1.0)) < 1e-7 and abs(o[0, 0, 1, 1] - math.sin(1.0)) < 1e-7


# ----------------------------------------------------- AdaIN + Snake ---

def test_adain_snake_matches_torch_instance_norm():
    c = configs.c2(C=64)
    x64 = torch.from_numpy(c["x"].astype(np.float64))
    xn = torch.nn.functional.instance_norm(x64, eps=1e-5).numpy()
    y = xn * (1.0 + c["gamma"].astype(np.float64))[None, :, None] + c["beta"].astype(np.float64)[None, :, None]
    a = c["alpha"].astype(np.float64)[None, :, None]
    inv_a = (1.0 / (c["alpha"] + np.float32(1e-9))).astype(np.float64)[None, :, None]
    ref = y + np.sin(a * y) ** 2 * inv_a
    got = R.adain_snake(c["x"], c["gamma"], c["beta"], c["alpha"])
    assert_close(got, ref, RTOL_F32, "adain+snake vs torch instance_norm")
    assert_close(CF.adain_snake(c["x"], c["gamma"], c["beta"], c["alpha"]), ref, 1e-12, "closed form")


def test_adain_snake_kokoro_known_answer():
    """Inputs and expected formula of test_adain_snake_f32_large
    (src/kokoro/gpu_decoder.rs:78-129): f64 statistics, f32 apply."""
    for C_, T_ in ((4, 100), (128, 11281)):
        k = configs.kokoro_kat(C_, T_)
        g32, b32, a32 = (k[n].astype(np.float32) for n in ("gamma", "beta", "alpha"))
        got = R.adain_snake(k["x"], g32, b32, a32)
        x = k["x"][0]
        mean = (x.astype(np.float64).sum(axis=1) / T_).astype(np.float32)
        var = ((x.astype(np.float64) - mean.astype(np.float64)[:, None]) ** 2).sum(axis=1) / T_
        rstd = (np.float32(1.0) / np.sqrt(var.astype(np.float32) + np.float32(1e-5))).astype(np.float32)
        scale = (g32 + np.float32(1.0)) * rstd
        inv_a = np.float32(1.0) / (a32 + np.float32(1e-9))
        styled = scale[:, None] * (x - mean[:, None]) + b32[:, None]
        s = np.sin(a32[:, None] * styled)
        expected = styled + s * s * inv_a[:, None]
        assert_close(got[0], expected, RTOL_F32, f"kokoro KAT C={C_} T={T_}")


def test_adain_snake_invariants():
    g = configs.rng(16)
    x = (g.standard_normal((2, 3, 500)) * 2 + 3).astype(np.float32)
    z = np.zeros(3, np.float32)
    big = np.full(3, 1e6, np.float32)
    # gamma = beta = 0: y is the plain two-pass LN (same f32 ops), and the
    # snake term sin^2(alpha y)/alpha lies in [0, 1/alpha]
    out = R.adain_snake(x, z, z, big).astype(np.float64)
    y = R.layernorm_twopass(x.reshape(6, 500)).reshape(2, 3, 500).astype(np.float64)
    assert np.all(out - y >= 0.0) and np.all(out - y <= 1e-6 * (1 + 1e-6) + 1e-6 * np.abs(y))
    # per-batch gamma/beta index b*C + c
    gb = g.standard_normal((2, 3)).astype(np.float32) * 0.1
    assert_close(R.adain_snake(x, gb, gb, np.ones(3, np.float32)), CF.adain_snake(x, gb, gb, np.ones(3)), RTOL_F32,
                 "per-batch params")


def test_adain_snake_large_offset_conditioning():
    """Rows with |mean| >> std: the reference's sequential f32 mean loses
    about log2(n |mean| / std) bits, so the restatement is only ~1e-4 from
    exact here (the GPU kernels are checked against the f64 closed form on
    such rows)."""
    g = configs.rng(17)
    x = (g.standard_normal((2, 3, 500)) * 2 + 100).astype(np.float32)
    ref = CF.adain_snake(x, np.zeros(3), np.zeros(3), np.ones(3))
    e = rel_err(R.adain_snake(x, np.zeros(3, np.float32), np.zeros(3, np.float32), np.ones(3, np.float32)), ref)
    assert 1e-6 < e < 2e-4


# ------------------------------------------------------------ golden ---

def test_golden_fixtures_reproduce():
    from .golden import make_golden

    for name, case in make_golden.load_all().items():
        fresh = make_golden.compute(name, case)
        for key, val in fresh.items():
            assert_bitexact(val, case[key], f"golden {name}:{key}")


# ------------------------------------------------- decode RoPE + cache ---

def test_f32_to_f16_rounding_matches_numpy():
    g = configs.rng(31)
    x = np.concatenate([g.standard_normal(100000).astype(np.float32) * 300,
                        g.standard_normal(100000).astype(np.float32) * 1e-5,
                        np.array([65504, 65519, 65520, 6e-8, 2.9802322e-08, -0.0, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert_bitexact(R.f32_to_f16_bits(x), ref, "f32 -> f16 RNE")


def test_rope_qk_cache_f16_against_f64_rotation_and_copies():
    """rope_qk_cache_fused + kv_cache_append restated: each rotated value is
    the f16 rounding of its f32 expression, which lies within half an f16
    ulp (plus f32 rounding) of the f64 rotation; the caches hold exact
    copies of the rotated k and of v at row pos, nothing else changes."""
    g = configs.rng(32)
    Hq, Hk, Dh, rot, L, pos = 10, 4, 64, 32, 50, 37
    q = g.standard_normal((Hq, Dh)).astype(np.float16).view(np.uint16)
    k = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16)
    v = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16)
    ck0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16)
    cv0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16)
    tab = R.rope_table(64, rot, 1e4)
    qo, ko, ck, cv = R.rope_qk_cache_f16(q, k, v, tab, pos, rot, ck0, cv0)
    ang = tab[pos, :rot // 2].astype(np.float64), tab[pos, rot // 2:].astype(np.float64)
    for x_in, x_out in ((q, qo), (k, ko)):
        xi = x_in.view(np.float16).astype(np.float64)
        xo = x_out.view(np.float16).astype(np.float64)
        c, s = ang
        e0 = xi[:, 0:rot:2] * c - xi[:, 1:rot:2] * s
        e1 = xi[:, 1:rot:2] * c + xi[:, 0:rot:2] * s
        for got, exp in ((xo[:, 0:rot:2], e0), (xo[:, 1:rot:2], e1)):
            assert np.all(np.abs(got - exp) <= np.abs(exp) * 2.0 ** -11 * 1.01 + 2.0 ** -24 * 4)
        assert_bitexact(x_out[:, rot:], x_in[:, rot:], "pass-through dims untouched")
    assert_bitexact(ck[:, pos], ko, "k cache row = rotated k")
    assert_bitexact(cv[:, pos], v, "v cache row = v")
    others = np.arange(L) != pos
    assert_bitexact(ck[:, others], ck0[:, others], "other k cache rows")
    assert_bitexact(cv[:, others], cv0[:, others], "other v cache rows")
    # position 0: cos = 1, sin = 0 -> identity
    q0, k0, _, _ = R.rope_qk_cache_f16(q, k, None, tab, 0, rot, ck0)
    assert_bitexact(q0, q, "pos 0 identity q")
    assert_bitexact(k0, k, "pos 0 identity k")


# -------------------------------------------------------------- Q8 GEMV ---

def _q8_weight(g, K, NW, scale=0.02):
    """Random repacked-Q8 weight: qs u32 [K, NW/4], scales f16 bits [K/32, NW],
    and its dequantisation in float64, decoded independently of the oracle
    (little-endian int8 view of the packed words: column c = byte c % 4 of
    word c / 4)."""
    qs = g.integers(0, 2 ** 32, size=(K, NW // 4), dtype=np.uint64).astype(np.uint32)
    sc = (g.standard_normal((K // 32, NW)) * scale).astype(np.float16)
    q = qs.view(np.int8).reshape(K, NW).astype(np.float64)
    W = q * np.repeat(sc.astype(np.float64), 32, axis=0)
    return qs, sc.view(np.uint16), W


def _acc_bound(x, W):
    """Forward error bound of an f32 dot product of length K (Higham's
    gamma_K), applied to |x| @ |W|."""
    K = x.shape[0]
    u = 2.0 ** -24
    gam = (K + 2) * u / (1 - (K + 2) * u)
    return gam * (np.abs(x.astype(np.float64)) @ np.abs(W))


def test_gemv_q8_matches_f64_matmul_of_dequant():
    g = configs.rng(41)
    for K, N in ((32, 16), (256, 96), (640, 640)):
        qs, sc, W = _q8_weight(g, K, N)
        x = g.standard_normal(K).astype(np.float16).astype(np.float32)
        bias = g.standard_normal(N).astype(np.float32)
        for b in (None, bias):
            got = R.gemv_q8(x, qs, sc, b)
            ref = x.astype(np.float64) @ W + (0 if b is None else b.astype(np.float64))
            bound = _acc_bound(x, W) + np.abs(ref) * 2.0 ** -23
            assert np.all(np.abs(got - ref) <= bound), (K, N, float(np.max(np.abs(got - ref) - bound)))


def test_gemv_q8_one_hot_selects_a_dequantised_row():
    """x = e_k: every product is exact, so out = f32(q[k, c] * scale) (+ bias
    rounded once) bit for bit."""
    g = configs.rng(42)
    K, N = 96, 48
    qs, sc, W = _q8_weight(g, K, N)
    bias = g.standard_normal(N).astype(np.float32)
    for k in (0, 31, 32, 95):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        # + 0.0: the accumulator starts at +0, so a zero weight gives +0
        assert_bitexact(R.gemv_q8(x, qs, sc), (W[k] + 0.0).astype(np.float32), f"row {k}")
        assert_bitexact(R.gemv_q8(x, qs, sc, bias), (W[k] + bias.astype(np.float64)).astype(np.float32),
                        f"row {k} + bias")


def test_gemv_q8_glu_matches_f64_silu_gate():
    g = configs.rng(43)
    K, N = 320, 80
    qs, sc, W = _q8_weight(g, K, 2 * N)
    x = g.standard_normal(K).astype(np.float16).astype(np.float32)
    bias = g.standard_normal(2 * N).astype(np.float32)
    got = R.gemv_q8(x, qs, sc, bias, glu=True)
    pre = x.astype(np.float64) @ W + bias
    xa, ga = pre[:N], pre[N:]
    sil = ga / (1 + np.exp(-ga))
    ref = sil * xa
    e = _acc_bound(x, W) + np.abs(pre) * 2.0 ** -23
    # |d silu / dg| <= 1.1; silu and the product add a few f32 roundings
    bound = 1.1 * e[N:] * np.abs(xa) + np.abs(sil) * e[:N] + np.abs(ref) * 2.0 ** -20
    assert np.all(np.abs(got - ref) <= bound)
    # the halves are not interchangeable: swapping them changes the result
    swapped = xa / (1 + np.exp(-xa)) * ga
    assert np.max(np.abs(swapped - ref)) > 1e-2


def test_gemv_q8_resadd_ln_against_f64():
    """h = f16(x @ W) + residual: the f16-rounded f32 sum lies within the
    accumulation bound plus one f16 ulp of the f64 projection's f16 rounding;
    norm is LN(h) * w rounded to f16 once, within one f16 ulp of
    the f64 LN of the oracle's own h."""
    g = configs.rng(44)
    for K, dim in ((2560, 640), (288, 288)):
        qs, sc, W = _q8_weight(g, K, dim)
        x = g.standard_normal(K).astype(np.float16).astype(np.float32)
        res = g.standard_normal(dim).astype(np.float32)
        w = (1 + 0.1 * g.standard_normal(dim)).astype(np.float16)
        h, norm = R.gemv_q8_resadd_ln(x, qs, sc, res, w.view(np.uint16), 1e-5)
        proj64 = x.astype(np.float64) @ W
        p16 = proj64.astype(np.float16).astype(np.float64)
        e = _acc_bound(x, W)
        # f16 rounding is monotone: |f16(acc) - f16(proj)| <= e + one f16 ulp at |proj| + e
        ulp = np.spacing((np.abs(proj64) + e).astype(np.float16)).astype(np.float64)
        hr = p16 + res
        assert np.all(np.abs(h - hr) <= e + ulp + np.abs(hr) * 2.0 ** -23)
        # with a zero residual h is the projection itself, an f16 value, and
        # the f16 rounding of the plain GEMV's f32 result
        h0, _ = R.gemv_q8_resadd_ln(x, qs, sc, np.zeros(dim, np.float32), w.view(np.uint16), 1e-5)
        assert_bitexact(h0, h0.astype(np.float16).astype(np.float32), "projection is rounded to f16")
        assert_bitexact(h0, R.gemv_q8(x, qs, sc).astype(np.float16).astype(np.float32), "same sums as gemv_q8")
        h64 = h.astype(np.float64)
        mu = h64.mean()
        var = ((h64 - mu) ** 2).mean()
        n64 = (h64 - mu) / np.sqrt(var + 1e-5) * w.astype(np.float64)
        got = norm.view(np.float16).astype(np.float64)
        ulpn = np.spacing(np.abs(n64).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - n64) <= ulpn + 1e-6)


def test_q8_pack_t4_is_a_column_permutation():
    """The t4 packing restatement moves bytes only: every tile slot holds the
    weight column the layout names (checked against an explicit loop on a
    small weight), and the GEMV over the unpacked tiles equals the GEMV over
    the original weight bit for bit."""
    g = configs.rng(45)
    K, NW = 64, 32
    qs, sc, _ = _q8_weight(g, K, NW)
    for glu in (False, True):
        tq, ts = R.q8_pack_t4(qs, sc, glu=glu)
        q8 = qs.view(np.uint8).reshape(K, NW)
        tb = tq.view(np.uint8).reshape(NW // 4, K, 4)
        tsc = ts.reshape(NW // 4, K // 32, 4)
        N = NW // 2
        for t in range(NW // 4):
            for c in range(4):
                col = (2 * t + c if c < 2 else N + 2 * t + c - 2) if glu else 4 * t + c
                assert np.array_equal(tb[t, :, c], q8[:, col]), (glu, t, c)
                assert np.array_equal(tsc[t, :, c], sc[:, col]), (glu, t, c)
        # unpack back to [K, NW] and compare the GEMVs
        order = np.array([(2 * t + c if c < 2 else N + 2 * t + c - 2) if glu else 4 * t + c
                          for t in range(NW // 4) for c in range(4)])
        q8u = np.empty_like(q8)
        q8u[:, order] = tb.transpose(1, 0, 2).reshape(K, NW)
        scu = np.empty_like(sc)
        scu[:, order] = tsc.transpose(1, 0, 2).reshape(K // 32, NW)
        assert np.array_equal(q8u, q8) and np.array_equal(scu, sc)


# ------------------------------------------------ Kokoro resblock conv1d ---

def _conv_f64(x, w, bias, stride, padding, dilation):
    B, C_in, T_in = x.shape
    C_out, _, K = w.shape
    T_out = (T_in + 2 * padding - dilation * (K - 1) - 1) // stride + 1
    xp = np.zeros((B, C_in, T_in + 2 * padding + stride * T_out + dilation * K), np.float64)
    xp[:, :, padding:padding + T_in] = x
    out = np.zeros((B, C_out, T_out))
    for k in range(K):
        cols = xp[:, :, k * dilation: k * dilation + stride * (T_out - 1) + 1: stride]   # [B, C_in, T_out]
        out += np.einsum("oc,bct->bot", w[:, :, k].astype(np.float64), cols)
    absum = np.zeros_like(out)
    for k in range(K):
        cols = np.abs(xp[:, :, k * dilation: k * dilation + stride * (T_out - 1) + 1: stride])
        absum += np.einsum("oc,bct->bot", np.abs(w[:, :, k].astype(np.float64)), cols)
    if bias is not None:
        out += bias.astype(np.float64)[None, :, None]
    return out, absum


@pytest.mark.parametrize("C_in,C_out,T,K,stride,padding,dilation", [
    (16, 8, 50, 3, 1, 1, 1), (8, 12, 40, 7, 1, 9, 3), (12, 4, 33, 11, 1, 25, 5), (6, 6, 31, 4, 2, 3, 1)])
def test_conv1d_f32io_matches_f64(C_in, C_out, T, K, stride, padding, dilation):
    g = configs.rng(80 + K)
    x = g.standard_normal((2, C_in, T)).astype(np.float32)
    w = (g.standard_normal((C_out, C_in, K)) * 0.2).astype(np.float16)
    b = g.standard_normal(C_out).astype(np.float16)
    got = R.conv1d_f32io(x, w.view(np.uint16), b.view(np.uint16), stride, padding, dilation)
    ref, absum = _conv_f64(x, w, b, stride, padding, dilation)
    assert got.shape == ref.shape
    n = C_in * K + 1
    gam = n * 2.0 ** -24 / (1 - n * 2.0 ** -24)
    assert np.all(np.abs(got - ref) <= gam * (absum + np.abs(b.astype(np.float64))[None, :, None]) + 1e-30)


def test_conv1d_f32io_identity_and_delta():
    g = configs.rng(85)
    x = g.standard_normal((1, 8, 20)).astype(np.float32)
    eye = np.eye(8, dtype=np.float16)[:, :, None]
    assert_bitexact(R.conv1d_f32io(x, eye.view(np.uint16)), x, "K=1 identity")
    # delta input: out[co, t] = w[co, c*, k] where t - padding + k*dilation = t*
    w = (g.standard_normal((5, 3, 7)) * 0.3).astype(np.float16)
    d = np.zeros((1, 3, 40), np.float32)
    d[0, 1, 17] = 1.0
    out = R.conv1d_f32io(d, w.view(np.uint16), None, 1, 9, 3)
    exp = np.zeros((1, 5, 40), np.float32)
    for k in range(7):
        t = 17 + 9 - 3 * k
        if 0 <= t < 40:
            exp[0, :, t] = w[:, 1, k].astype(np.float32)
    assert_bitexact(out, exp, "delta response")


# ------------------------------------------------------------ decode attention

def _attn_f64(q, k, v, kv_len, n_kv_heads, sm_scale, skh, sks):
    """softmax(sm_scale q.K^T) V per query head in float64 (numpy), K/V addressed as
    head * skh + pos * sks + d in the flat f16 arrays."""
    nq, hd = q.shape
    kf = k.astype(np.float64).ravel()
    vf = v.astype(np.float64).ravel()
    out = np.empty((nq, hd))
    for h in range(nq):
        kvh = h * n_kv_heads // nq
        idx = kvh * skh + np.arange(kv_len)[:, None] * sks + np.arange(hd)[None, :]
        s = kf[idx] @ q[h].astype(np.float64) * sm_scale
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ vf[idx]
    return out


@pytest.mark.parametrize("nq,nkv,hd,kv_len,layout", [
    (4, 2, 64, 100, "cache"), (8, 8, 52, 37, "encoder"), (10, 10, 64, 1, "cache"), (6, 3, 128, 300, "encoder")])
def test_attention_oracle_matches_f64_softmax(nq, nkv, hd, kv_len, layout):
    g = configs.rng(nq * 31 + kv_len)
    q = g.standard_normal((nq, hd)).astype(np.float16)
    if layout == "cache":  # [heads, max_kv_len, hd], max_kv_len > kv_len
        mx = kv_len + 5
        k = g.standard_normal((nkv, mx, hd)).astype(np.float16)
        v = g.standard_normal((nkv, mx, hd)).astype(np.float16)
        skh, sks = mx * hd, hd
    else:                  # [kv_len, heads, hd]
        k = g.standard_normal((kv_len, nkv, hd)).astype(np.float16)
        v = g.standard_normal((kv_len, nkv, hd)).astype(np.float16)
        skh, sks = hd, nkv * hd
    scale = 1.0 / math.sqrt(hd)
    got = R.attention_decode(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), kv_len, nkv, scale, skh, sks)
    ref = _attn_f64(q, k, v, kv_len, nkv, scale, skh, sks)
    assert np.max(np.abs(got - ref)) <= 2e-6 * max(1.0, float(np.max(np.abs(ref))))


def test_attention_oracle_special_cases():
    g = configs.rng(77)
    hd, L = 64, 50
    v = g.standard_normal((1, L, hd)).astype(np.float16)
    # one position: the output is that V row exactly (p = 1, l = 1)
    q = g.standard_normal((1, hd)).astype(np.float16)
    k = g.standard_normal((1, L, hd)).astype(np.float16)
    one = R.attention_decode(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), 1, 1, 0.125, L * hd, hd)
    assert np.array_equal(one[0], v[0, 0].astype(np.float32))
    # q = 0: every score is 0, the output is the mean of the V rows
    z = np.zeros((1, hd), np.float16)
    mean = R.attention_decode(z.view(np.uint16), k.view(np.uint16), v.view(np.uint16), L, 1, 0.125, L * hd, hd)
    assert np.max(np.abs(mean[0] - v[0].astype(np.float64).mean(axis=0))) < 1e-6
    # one key aligned with q and a large scale: that position's V row dominates
    k2 = np.zeros((1, L, hd), np.float16)
    k2[0, 17] = q[0]
    dom = R.attention_decode(q.view(np.uint16), k2.view(np.uint16), v.view(np.uint16), L, 1, 50.0, L * hd, hd)
    assert np.max(np.abs(dom[0] - v[0, 17].astype(np.float32))) < 1e-6
    # a permutation of the positions leaves the output unchanged (up to f32 rounding)
    perm = g.permutation(L)
    a = R.attention_decode(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), L, 1, 0.125, L * hd, hd)
    b = R.attention_decode(q.view(np.uint16), np.ascontiguousarray(k[:, perm]).view(np.uint16),
                           np.ascontiguousarray(v[:, perm]).view(np.uint16), L, 1, 0.125, L * hd, hd)
    assert np.max(np.abs(a - b)) < 1e-6


# ------------------------------------------------------- Kokoro tail ---

def _istft_f64(x, n_fft, hop):
    """torch.istft(center=True, periodic Hann) semantics in float64 via numpy's
    irfft: a different route (FFT, not the cos/sin basis sums)."""
    x = x.astype(np.float64)
    bins = n_fft // 2 + 1
    n_frames = x.shape[1]
    spec = np.exp(x[:bins]) * np.exp(1j * np.sin(x[bins:]))
    # irfft drops the imaginary parts of the DC and Nyquist bins, as the
    # basis sum does (sin(0) = sin(pi n) = 0)
    frames = np.fft.irfft(spec.T, n=n_fft, axis=1)
    w = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(n_fft) / n_fft)
    full = (n_frames - 1) * hop + n_fft
    y = np.zeros(full)
    ws = np.zeros(full)
    for f in range(n_frames):
        y[f * hop:f * hop + n_fft] += frames[f] * w
        ws[f * hop:f * hop + n_fft] += w * w
    y = np.where(ws > 1e-8, y / np.where(ws > 1e-8, ws, 1.0), y)
    return y[n_fft // 2: full - n_fft // 2]


@pytest.mark.parametrize("n_fft,hop,n_frames", [(20, 5, 64), (20, 5, 2), (16, 4, 33), (32, 8, 17), (20, 10, 9)])
def test_istft_oracle_matches_f64_irfft(n_fft, hop, n_frames):
    g = configs.rng(n_fft * 100 + n_frames)
    x = (g.standard_normal((2 * (n_fft // 2 + 1), n_frames)) * 0.7).astype(np.float32)
    got = R.istft(x, n_fft, hop)
    ref = _istft_f64(x, n_fft, hop)
    assert got.shape == ref.shape == ((n_frames - 1) * hop,)
    # f32 tables and sums over n_fft / 2 + 1 bins: a few f32 ulps of the peak
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert err < 5e-6, err


@pytest.mark.parametrize("N,hop,k0,A,x0", [(20, 5, 0, 1.5, 0.0), (20, 5, 4, 0.8, 0.0), (20, 5, 4, 0.8, 0.9),
                                          (20, 5, 8, 2.0, -1.3), (16, 4, 8, 0.5, 0.0), (16, 4, 8, 0.5, 1.1),
                                          (16, 4, 4, 1.0, 0.4)])
def test_istft_oracle_closed_forms(N, hop, k0, A, x0):
    """Interior samples (all N / hop = 4 frames overlap) of a periodic Hann
    at 75% overlap: sum w = 2 and sum w^2 = 3/2. A bin-k0 spectrum of
    magnitude A and phase phi with k0 hop / N an integer adds the same
    sample in every frame, so it comes back as s (A / N)(4/3) cos(2 pi k0 p
    / N + phi) (s = 2, or 1 for DC; the Nyquist bin keeps only A cos(phi))."""
    F = 40
    bins = N // 2 + 1
    assert (k0 * hop) % N == 0
    p = np.arange(N // 2, (F - 1) * hop + N // 2)  # untrimmed positions of the outputs
    interior = (p >= N - hop) & (p < (F - 1) * hop + hop)
    x = np.full((2 * bins, F), -200.0, np.float32)  # exp(-200) = 0 in f32
    x[bins:] = 0.0
    x[k0] = np.log(A)
    x[bins + k0] = x0
    phi = np.sin(np.float64(np.float32(x0)))
    out = R.istft(x, N, hop).astype(np.float64)
    if k0 == bins - 1:
        want = A / N * (4.0 / 3.0) * np.cos(phi) * np.cos(np.pi * p)
    else:
        scale = 1.0 if k0 == 0 else 2.0
        want = scale * A / N * (4.0 / 3.0) * np.cos(2 * np.pi * k0 * p / N + phi)
    assert np.max(np.abs(out[interior] - want[interior])) < 2e-6 * A


def test_istft_oracle_layout_and_trim():
    """A single frame carrying energy shows where it lands: frame f's samples
    occupy untrimmed positions [f hop, f hop + N), output index = position -
    N / 2; every other output sample stays 0."""
    N, hop, F = 20, 5, 12
    bins = N // 2 + 1
    x = np.full((2 * bins, F), -200.0, np.float32)
    x[bins:] = 0.0
    x[0, 6] = 0.0  # frame 6: DC bin of magnitude 1
    out = R.istft(x, N, hop)
    nz = np.nonzero(out)[0]
    assert nz.min() == 6 * hop + 1 - N // 2 and nz.max() == 6 * hop + N - 1 - N // 2  # w[0] = 0
    assert np.all(out[nz] > 0)


def test_combine_oracle_special_cases():
    g = configs.rng(91)
    a, b, c = (g.standard_normal(4096).astype(np.float32) for _ in range(3))
    third = np.float32(0.3333333333333333)
    # association ((a + b) + c), then the f32 multiply by the rounded 1/3
    ref = ((a.astype(np.float64) + b + c) / 3.0)
    got = R.resblock_average(a, b, c)
    assert np.max(np.abs(got - ref)) <= 4e-7 * np.max(np.abs(ref)) * 4
    # the product by f32(1/3) is not the division by 3: some inputs differ by an ulp
    ints = np.arange(1, 4096, dtype=np.float32) * np.float32(1.1)
    z = np.zeros_like(ints)
    mul = R.resblock_average(ints, z, z)
    assert np.array_equal(mul, ints * third)
    assert np.any(mul != ints / np.float32(3.0))
    # the sum is associated left to right: big + (-big) + small keeps small
    big = np.full(4, 3e7, np.float32)
    small = np.full(4, 1.0, np.float32)
    assert np.all(R.combine(big, -big, small) == 1.0)
    assert np.all(R.combine(small, big, -big) == 0.0)
    # leaky ReLU: positives untouched, negatives times slope, zeros stay zero
    v = np.array([2.0, -2.0, 0.0, -0.0, 1e-30, -1e30], np.float32)
    lr = R.combine(v, lrelu_slope=0.01)
    assert np.array_equal(lr, np.array([2.0, np.float32(-2.0) * np.float32(0.01), 0.0, 0.0, 1e-30,
                                        np.float32(-1e30) * np.float32(0.01)], np.float32))
    # scale alone
    assert np.array_equal(R.combine(a, scale=0.25), a * np.float32(0.25))


def test_snake_oracle():
    """snake(x) = x + sin^2(alpha x) / (alpha + 1e-9) against float64, plus
    what the formula fixes: alpha = 0 gives x exactly (sin(0) = 0), the
    periodic part repeats with period pi / alpha, and the added term lies in
    [0, 1 / (alpha + 1e-9)]; the channel of row r is r % C."""
    g = configs.rng(95)
    C, T = 3, 257
    x = (g.standard_normal((2, C, T)) * 3).astype(np.float32)
    alpha = np.array([0.7, 1.3, 0.0], np.float32)
    got = R.snake(x, alpha)
    a64 = alpha.astype(np.float64)[None, :, None]
    ref = x + np.sin(a64 * x) ** 2 / (a64 + 1e-9)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1)) < 2e-6
    assert np.array_equal(got[:, 2], x[:, 2])
    extra = got[:, :2].astype(np.float64) - x[:, :2]
    assert np.all(extra >= -1e-6) and np.all(extra <= 1 / alpha[:2, None] + 1e-5)
    # period pi / alpha of the added term (channel 0), up to f32 rounding of x + period
    xp = (x[:, 0] + np.float32(np.pi / 0.7)).astype(np.float32)
    per = R.snake(xp[:, None, :], alpha[:1]).astype(np.float64)[:, 0] - xp
    assert np.max(np.abs(per - extra[:, 0])) < 1e-4
