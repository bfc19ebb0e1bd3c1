"""Randomised shape sweep over the fused kernels (seeded, so every run
checks the same cases): LayerNorm, residual add + LayerNorm, rotary,
AdaIN+Snake (f32 and f16 activations), the Q8_0 gather and the Kokoro tail,
each against the oracle at the bar of its output dtype. The fixed-shape
tests pin the edges; this sweeps the space between them (odd widths, row
counts that leave partial workgroups, every kernel-variant boundary that a
random size happens to land near)."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_F16, RTOL_F32, assert_bitexact, assert_close, rel_err, say

pytestmark = pytest.mark.gpu

N_CASES = 12


def _cases(seed):
    return [np.random.default_rng(seed * 1000 + i) for i in range(N_CASES)]


@pytest.mark.parametrize("i", range(N_CASES))
def test_layernorm_random(i):
    g = _cases(1)[i]
    rows = int(g.integers(1, 3000))
    cols = int(g.choice([int(g.integers(1, 64)), int(g.integers(64, 4096)), 512, 1024, 2048, 2049]))
    unit = bool(g.integers(0, 2))
    say("layernorm random", rows, cols, unit)
    x = (g.standard_normal((rows, cols)) * 2 + g.standard_normal()).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    b = (0.1 * g.standard_normal(cols)).astype(np.float32)
    y = abi.layernorm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(),
                      unit_offset=unit).cpu().numpy()
    assert_close(y, R.layernorm_twopass(x, w, b, unit_offset=unit), RTOL_F32, f"LN {rows}x{cols}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_rotary_random(i):
    g = _cases(2)[i]
    B, Hq, Hk = int(g.integers(1, 3)), int(g.integers(1, 9)), int(g.integers(1, 5))
    T = int(g.integers(1, 700))
    Dh = int(g.choice([16, 32, 64, 128]))
    rot = int(g.choice([r for r in (8, 16, 32, 64, 128) if r <= Dh]))
    pos0 = int(g.integers(0, 300))
    say("rotary random", B, Hq, Hk, T, Dh, rot, pos0)
    q = g.standard_normal((B, Hq, T, Dh)).astype(np.float32)
    k = g.standard_normal((B, Hk, T, Dh)).astype(np.float32)
    qo, ko = abi.rotary(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), rot, 10000.0, pos0)
    assert_close(qo.cpu().numpy(), R.rotary(q, rot, 10000.0, pos0), RTOL_F32, "q")
    assert_close(ko.cpu().numpy(), R.rotary(k, rot, 10000.0, pos0), RTOL_F32, "k")


@pytest.mark.parametrize("i", range(N_CASES))
def test_adain_snake_random(i):
    g = _cases(3)[i]
    B, C = int(g.integers(1, 3)), int(g.integers(1, 40))
    T = int(g.choice([int(g.integers(1, 300)), int(g.integers(300, 20000)), int(g.integers(20000, 130000))]))
    if B * C * T > 6_000_000:
        C = max(1, 6_000_000 // (B * T))
    say("adain+snake random", B, C, T)
    x = (g.standard_normal((B, C, T)) * 1.5 + 0.3).astype(np.float32)
    gamma = (0.1 * g.standard_normal((B, C))).astype(np.float32)
    beta = (0.1 * g.standard_normal(C)).astype(np.float32)
    alpha = g.uniform(0.3, 1.7, C).astype(np.float32)
    p = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    out = abi.adain_snake(p(x), p(gamma), p(beta), p(alpha)).cpu().numpy()
    # the reference's sequential f32 row sums drift from the exact statistics on long rows (up to ~2e-5 of
    # the output at T ~ 60k); the bar is the float64 form, and the oracle within its own measured drift
    f64 = CF.adain_snake(x, gamma, beta, alpha)
    orc = R.adain_snake(x, gamma, beta, alpha)
    drift = rel_err(orc, f64)
    assert_close(out, f64, RTOL_F32, f"f32 {B}x{C}x{T} vs f64")
    assert_close(out, orc, RTOL_F32 + drift, f"f32 {B}x{C}x{T} vs oracle (its drift {drift:.1e})")
    x16 = x.astype(np.float16)
    out16 = abi.adain_snake(torch.from_numpy(x16).cuda(), p(gamma), p(beta), p(alpha)).float().cpu().numpy()
    assert_close(out16, CF.adain_snake(x16.astype(np.float32), gamma, beta, alpha), RTOL_F16, f"f16 {B}x{C}x{T}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_q8_gather_random(i):
    g = _cases(4)[i]
    vocab = int(g.integers(1, 5000))
    d = 32 * int(g.integers(1, 40))
    n = int(g.integers(1, 3000))
    say("q8_0 gather random", vocab, d, n)
    nb = d // 32
    blocks = np.zeros((vocab, nb, 34), np.uint8)
    blocks[:, :, :2] = np.frombuffer(
        g.uniform(1e-3, 2e-2, vocab * nb).astype(np.float16).tobytes(), np.uint8).reshape(vocab, nb, 2)
    blocks[:, :, 2:] = g.integers(0, 256, (vocab, nb, 32), dtype=np.uint8)
    ids = g.integers(0, vocab, n).astype(np.int64)
    out = abi.q8_0_embed_gather(torch.from_numpy(blocks.ravel()).cuda(), vocab, d,
                                torch.from_numpy(ids).cuda()).cpu().numpy()
    ref, bad = R.q8_0_embedding(blocks.ravel(), vocab, d, ids)
    assert bad == 0
    assert_bitexact(out, ref.reshape(n, d), f"gather {vocab}x{d} n={n}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_kokoro_tail_random(i):
    g = _cases(5)[i]
    n = int(g.integers(1, 400000))
    off = int(g.integers(0, 4))
    say("resblock average random", n, off)
    r = [g.standard_normal(n + off).astype(np.float32) for _ in range(3)]
    dev = [torch.from_numpy(a).cuda()[off:] for a in r]
    slope = 0.01 if g.integers(0, 2) else None
    out = abi.resblock_average_f32(*dev, leaky_slope=slope).cpu().numpy()
    assert_bitexact(out, R.resblock_average(*(a[off:] for a in r), lrelu_slope=slope), "resblock average")
    n_frames = int(g.integers(2, 20000))
    say("istft random", n_frames)
    x = (g.standard_normal((22, n_frames)) * 0.7).astype(np.float32)
    got = abi.istft_f32(torch.from_numpy(x).cuda()).cpu().numpy()
    assert_close(got, R.istft(x, 20, 5), RTOL_F32, f"istft {n_frames}")


def _conv_f64(x, w, b, pad, dil):
    """Exact (float64) conv1d of the f32 input and f16 weights, plus bias."""
    B, C_in, T = x.shape
    C_out, _, K = w.shape
    T_out = T + 2 * pad - dil * (K - 1)
    xp = np.zeros((B, C_in, T + 2 * pad))
    xp[:, :, pad:pad + T] = x
    out = np.zeros((B, C_out, T_out)) + (0 if b is None else b.astype(np.float64)[None, :, None])
    w64 = w.astype(np.float64)
    for k in range(K):
        seg = xp[:, :, k * dil:k * dil + T_out]
        out += np.matmul(w64[:, :, k][None], seg)
    return out


def _conv_shape(g, square=False):
    while True:
        B = int(g.integers(1, 3))
        C_in = 16 * int(g.integers(1, 17))
        C_out = C_in if square else int(g.integers(1, 261))
        K = int(g.choice([1, 2, 3, 5, 7, 11]))
        dil = int(g.choice([d for d in (1, 2, 3, 5) if (K - 1) * d <= 64]))
        T = int(g.integers(1, 2500))
        pad = int(g.integers(0, (K - 1) * dil + 1))
        T_out = T + 2 * pad - dil * (K - 1)
        if T_out >= 1 and B * C_in * C_out * K * T_out <= 300_000_000:
            return B, C_in, C_out, K, dil, T, pad, T_out


@pytest.mark.parametrize("i", range(N_CASES))
def test_conv1d_random(i):
    g = _cases(6)[i]
    B, C_in, C_out, K, dil, T, pad, T_out = _conv_shape(g)
    res = bool(g.integers(0, 2))
    say("conv1d random", B, C_in, C_out, K, dil, T, pad, res)
    x = g.standard_normal((B, C_in, T)).astype(np.float32)
    w = (g.standard_normal((C_out, C_in, K)) * 0.1).astype(np.float16)
    b = g.standard_normal(C_out).astype(np.float16)
    r = g.standard_normal((B, C_out, T_out)).astype(np.float32) if res else None
    wp = abi.conv1d_pack_f16(torch.from_numpy(w).cuda())
    out = abi.conv1d_f16w_packed(torch.from_numpy(x).cuda(), wp, torch.from_numpy(b).cuda(),
                                 torch.from_numpy(r).cuda() if res else None, padding=pad, dilation=dil)
    ref = R.conv1d_f32io(x, w.view(np.uint16), b.view(np.uint16), 1, pad, dil, nthreads=16)
    ex = _conv_f64(x, w, b, pad, dil)
    if res:
        ref = ref + r
        ex = ex + r
    # long random dot products (C_in K up to 2816 terms): the reference's sequential f32 sums drift from the
    # exact result by up to ~1.5e-5 here; the GPU must be as close to exact as 1e-5 or twice that drift
    drift = rel_err(ref, ex)
    got = out.cpu().numpy()
    e = assert_close(got, ex, max(RTOL_F32, 2 * drift), f"conv1d random vs f64 (oracle drift {drift:.1e})")
    assert_close(got, ref, RTOL_F32 + 2 * drift, "conv1d random vs oracle")
    print(f"[conv random] gpu vs f64 {e:.2e}, oracle vs f64 {drift:.2e}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_adain_snake_conv1d_random(i):
    """The fused stage, with the AdaIN+Snake bar carried through the conv
    (sum_k |w| 1e-5 max(|y|, 1)) on top of the conv's own bar."""
    g = _cases(7)[i]
    B, C, _, K, dil, T, pad, T_out = _conv_shape(g, square=True)
    with_res = bool(g.integers(0, 2))
    say("adain_snake_conv1d random", B, C, K, dil, T, pad, with_res)
    x = (g.standard_normal((B, C, T)) * 1.5 + 0.3).astype(np.float32)
    gam = (g.standard_normal((B, C)) * 0.1).astype(np.float32)
    bet = (g.standard_normal((B, C)) * 0.1).astype(np.float32)
    alp = g.uniform(0.5, 1.5, C).astype(np.float32)
    w = (g.standard_normal((C, C, K)) * 0.05).astype(np.float16)
    b = g.standard_normal(C).astype(np.float16)
    res = g.standard_normal((B, C, T_out)).astype(np.float32)
    wp = abi.conv1d_pack_f16(torch.from_numpy(w).cuda())
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    out = abi.adain_snake_conv1d(dt(x), dt(gam), dt(bet), dt(alp), wp, dt(b), dt(res) if with_res else None,
                                 padding=pad, dilation=dil)
    y = R.adain_snake(x, gam, bet, alp)
    ref = R.conv1d_f32io(y, w.view(np.uint16), b.view(np.uint16), 1, pad, dil, nthreads=16)
    if with_res:
        ref = ref + res
    wabs = np.abs(w.astype(np.float32)).astype(np.float16)
    carried = R.conv1d_f32io(np.maximum(np.abs(y), 1.0).astype(np.float32), wabs.view(np.uint16), None, 1, pad, dil,
                             nthreads=16).astype(np.float64) * RTOL_F32 * 1.01
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
    bound = carried + RTOL_F32 * np.maximum(np.abs(ref), 1.0)
    assert np.all(err <= bound), f"max excess {float(np.max(err - bound)):.3e}"


@pytest.mark.parametrize("i", range(N_CASES))
def test_gemv_q8_random(i):
    """Repacked-Q8 GEMV (+ bias), both weight layouts, at random K (a multiple
    of 32) and N (a multiple of 16), within the f32 accumulation bound."""
    from .test_gpu_gemv import _TD, _bound, _check, _dev_w, _run, _weight, _x

    g = _cases(8)[i]
    K = 32 * int(g.integers(1, 130))
    N = 16 * int(g.integers(1, 300))
    xd, od = str(g.choice(["f16", "f32"])), str(g.choice(["f16", "f32"]))
    layout = str(g.choice(["ref", "t4"]))
    with_bias = bool(g.integers(0, 2))
    say("gemv_q8 random", layout, K, N, xd, od, with_bias)
    qs, sc, W = _weight(g, K, N)
    x, xt = _x(g, K, xd)
    bias = g.standard_normal(N).astype(np.float32) if with_bias else None
    q_t, s_t = _dev_w(qs, sc)
    out = _run(layout, "gemv_q8", xt, q_t, s_t, torch.from_numpy(bias).cuda() if with_bias else None,
               out_dtype=_TD[od])
    ref = R.gemv_q8(x, qs, sc.view(np.uint16), bias).astype(np.float64)
    _check(out, ref, _bound(x, W), od, f"gemv_q8 random K={K} N={N}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_attention_decode_random(i):
    """Decode attention at random head counts (grouped-query included), head
    dims, positions and both K/V layouts, one-launch and split forms."""
    from .test_gpu_attention import _check as attn_check
    from .test_gpu_attention import _inputs as attn_inputs

    g = _cases(9)[i]
    nkv = int(g.integers(1, 9))
    nq = nkv * int(g.choice([1, 2, 4]))
    hd = int(g.choice([16, 32, 36, 52, 64, 80, 128]))
    kv_len = int(g.integers(1, 3000))
    layout = str(g.choice(["cache", "enc"]))
    splits = None if g.integers(0, 2) else int(g.integers(1, 64))
    say("attention random", nq, nkv, hd, kv_len, layout, splits)
    q, k, v, skh, sks = attn_inputs(nq, nkv, hd, kv_len, layout, int(g.integers(0, 1 << 30)))
    scale = float(1.0 / np.sqrt(hd))
    T = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    out = abi.attention_decode(T(q), T(k), T(v), kv_len, n_kv_heads=nkv, sm_scale=scale, stride_kv_head=skh,
                               stride_kv_seq=sks, n_splits=splits)
    attn_check(out, q, k, v, kv_len, nkv, scale, skh, sks, f"attention random {nq}/{nkv} hd={hd} L={kv_len}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_residual_add_layernorm_random(i):
    """Residual add + LayerNorm (+ GELU / SiLU) in the dtype profiles the
    reference uses (bf16 everywhere; f16 projection + f32 residual -> f32 h
    and f16 norm; f32), at random widths and row counts: h bit-exact, the
    norm at the bar of its dtype against the float64 form on that h."""
    from oracle import closed_form as CF_

    from ._util import RTOL_BF16

    g = _cases(10)[i]
    rows = int(g.integers(1, 2000))
    cols = int(g.choice([int(g.integers(1, 128)), int(g.integers(128, 4097)), 640, 1024]))
    prof = str(g.choice(["bf16", "f16f32", "f32"]))
    act = str(g.choice(["none", "gelu", "silu"]))
    say("resadd+ln random", rows, cols, prof, act)
    x = g.standard_normal((rows, cols)).astype(np.float32)
    r = g.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    b = (0.1 * g.standard_normal(cols)).astype(np.float32)
    if prof == "bf16":
        xt, rt = torch.from_numpy(x).bfloat16().cuda(), torch.from_numpy(r).bfloat16().cuda()
        h, y = abi.residual_add_layernorm(xt, rt, torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(), act=act)
        h_ref = (xt.float() + rt.float()).bfloat16()
        tol = RTOL_BF16
    elif prof == "f16f32":
        xt, rt = torch.from_numpy(x).half().cuda(), torch.from_numpy(r).cuda()
        h, y = abi.residual_add_layernorm(xt, rt, torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(), act=act,
                                          h_dtype=torch.float32, out_dtype=torch.float16)
        h_ref = xt.float() + rt
        tol = RTOL_F16
    else:
        xt, rt = torch.from_numpy(x).cuda(), torch.from_numpy(r).cuda()
        h, y = abi.residual_add_layernorm(xt, rt, torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(), act=act)
        h_ref = xt + rt
        tol = RTOL_F32
    assert torch.equal(h.cpu(), h_ref.cpu()), "h"
    ref = CF_.layernorm(h_ref.float().cpu().numpy().astype(np.float64), w, b)
    if act == "gelu":
        ref = CF_.gelu_erf(ref)
    elif act == "silu":
        ref = ref / (1 + np.exp(-ref))
    assert_close(y.float().cpu().numpy(), ref, tol, f"norm {prof} {act}")


@pytest.mark.parametrize("i", range(N_CASES))
def test_rope_qk_cache_random(i):
    """Decode-step RoPE + K/V cache append (f16), random heads, head dims,
    rotary dims, cache lengths and positions: bit-exact with the oracle."""
    from .test_gpu_decode import _bits, _f16

    g = _cases(11)[i]
    Hk = int(g.integers(1, 9))
    Hq = Hk * int(g.choice([1, 2, 4]))
    Dh = 2 * int(g.integers(1, 65))
    rot = 2 * int(g.integers(0, Dh // 2 + 1))
    L = int(g.integers(1, 600))
    pos = int(g.integers(0, L))
    with_v = bool(g.integers(0, 2))
    say("rope_qk_cache random", Hq, Hk, Dh, rot, L, pos, with_v)
    q = g.standard_normal((Hq, Dh)).astype(np.float16).view(np.uint16)
    k = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16)
    v = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16) if with_v else None
    ck0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16)
    cv0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16) if with_v else None
    tab = R.rope_table(L, rot, 1e4) if rot else np.zeros((1, 2), np.float32)
    qd, kd, ckd = _f16(q), _f16(k), _f16(ck0)
    vd = _f16(v) if with_v else None
    cvd = _f16(cv0) if with_v else None
    abi.rope_qk_cache_append(qd, kd, vd, torch.from_numpy(tab).cuda(), ckd, cvd, pos, rot)
    qr, kr, ckr, cvr = R.rope_qk_cache_f16(q, k, v, tab, pos, rot, ck0, cv0)
    assert_bitexact(_bits(qd), qr, "q")
    assert_bitexact(_bits(kd), kr, "k")
    assert_bitexact(_bits(ckd), ckr, "cache_k")
    if with_v:
        assert_bitexact(_bits(cvd), cvr, "cache_v")


@pytest.mark.parametrize("i", range(N_CASES))
def test_conv_chain_random(i):
    """Chained ResBlock stages at random shapes (every conv kernel family,
    including rows that are not 16-byte aligned): stage output bit-identical
    to the unchained kernel, row statistics against float64 of that output,
    and the second stage with handed-over statistics against the unchained
    second stage."""
    from .test_gpu_conv_chain import _check_stats

    g = _cases(12)[i]
    B, C, _, K, dil, T, _, _ = _conv_shape(g, square=True)
    pad = (K - 1) * dil // 2
    if T + 2 * pad - dil * (K - 1) < 1:
        pad = (K - 1) * dil
    say("conv chain random", B, C, T, K, dil, pad)
    x = (g.standard_normal((B, C, T)) * 1.5 + 0.3).astype(np.float32)
    p = lambda *sh: torch.from_numpy((g.standard_normal(sh) * 0.1).astype(np.float32)).cuda()  # noqa: E731
    g1, b1, g2, b2 = p(B, C), p(B, C), p(B, C), p(B, C)
    a1 = torch.from_numpy(g.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    a2 = torch.from_numpy(g.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    w1 = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).cuda())
    w2 = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).cuda())
    bb = torch.from_numpy(g.standard_normal(C).astype(np.float16)).cuda()
    xt = torch.from_numpy(x).cuda()
    h, s_h = abi.adain_snake_conv1d_chain(xt, g1, b1, a1, w1, bb, padding=pad, dilation=dil)
    h_ref = abi.adain_snake_conv1d(xt, g1, b1, a1, w1, bb, padding=pad, dilation=dil)
    assert_bitexact(h.cpu().numpy(), h_ref.cpu().numpy(), "stage 1 output")
    _check_stats(h, s_h, 1e-5, "stage 1 statistics")
    y, _ = abi.adain_snake_conv1d_chain(h, g2, b2, a2, w2, bb, x_stats=s_h, want_stats=False, padding=pad,
                                        dilation=dil)
    y_ref = abi.adain_snake_conv1d(h_ref, g2, b2, a2, w2, bb, padding=pad, dilation=dil)
    assert_close(y.cpu().numpy(), y_ref.cpu().numpy(), RTOL_F32, "stage 2 with handed-over statistics")
