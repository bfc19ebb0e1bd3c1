"""LayerNorm family and fused residual-add + LN (+GELU) on the GPU.

f32: within 1e-5 of the f64 closed form and of the oracle's restatements of
candle's LayerNorm (src/parakeet/fast_conformer.rs:721-725) and the two-pass
Moonshine LayerNorms (src/moonshine/encoder.rs:68-76, decoder.rs:67-74).
bf16 (config 4a): h bit-exact, y within 1e-2 of the unfused bf16 chain and
within one bf16 rounding of the f64 closed form.
"""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_BF16, RTOL_F16, RTOL_F32, assert_bitexact, assert_close, dev_tensor, host, say

pytestmark = pytest.mark.gpu


def _ln(x, gamma=None, beta=None, **kw):
    out = abi.layernorm(dev_tensor(x), None if gamma is None else dev_tensor(gamma),
                        None if beta is None else dev_tensor(beta), **kw)
    torch.cuda.synchronize()
    return host(out)


def test_config0(dev):
    c = configs.c0()
    say("layernorm config0 f32 [1,125,1024]")
    got = _ln(c["x"], c["gamma"], c["beta"])
    assert_close(got, CF.layernorm(c["x"], c["gamma"], c["beta"]), RTOL_F32, "c0 vs f64")
    assert_close(got, R.layernorm_candle(c["x"], c["gamma"], c["beta"]), RTOL_F32, "c0 vs candle restatement")
    assert_close(got, R.layernorm_twopass(c["x"], c["gamma"], c["beta"]), RTOL_F32, "c0 vs two-pass")


@pytest.mark.parametrize("rows,cols", [(1, 4), (3, 64), (33, 288), (7, 1000), (5, 1001), (9, 2048), (4, 4096),
                                       (3, 5000), (2, 12345)])
def test_shapes_f32(dev, rows, cols):
    g = configs.rng(rows * 7 + cols)
    x = (g.standard_normal((rows, cols)) * 1.5 + 0.3).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    b = (0.1 * g.standard_normal(cols)).astype(np.float32)
    say("layernorm f32", rows, cols)
    assert_close(_ln(x, w, b), CF.layernorm(x, w, b), RTOL_F32, f"{rows}x{cols}")
    assert_close(_ln(x), CF.layernorm(x), RTOL_F32, f"{rows}x{cols} no affine")
    assert_close(_ln(x, w, unit_offset=True), CF.layernorm(x, w, unit_offset=True), RTOL_F32, "unit offset")


def test_golden(dev):
    from .golden import make_golden

    cases = make_golden.load_all()
    c = cases["ln_c0_rows16"]
    say("layernorm golden ln_c0_rows16")
    got = _ln(c["x"], c["gamma"], c["beta"])
    assert_close(got, c["out_candle"], RTOL_F32, "golden candle")
    assert_close(got, c["out_twopass"], RTOL_F32, "golden two-pass")
    c = cases["ln_unit_offset_8x288"]
    say("layernorm golden ln_unit_offset_8x288")
    assert_close(_ln(c["x"], c["gamma"], unit_offset=True), c["out"], RTOL_F32, "golden unit offset")


@pytest.mark.parametrize("xd,yd", [(torch.float32, torch.float16), (torch.float16, torch.float16),
                                   (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                   (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("cols", [576, 1024, 999])
def test_dtypes(dev, xd, yd, cols):
    g = configs.rng(cols)
    x = torch.from_numpy(g.standard_normal((37, cols)).astype(np.float32)).to(xd)
    w = torch.from_numpy((1 + 0.1 * g.standard_normal(cols)).astype(np.float32))
    say("layernorm dtypes", xd, yd, cols)
    out = abi.layernorm(x.cuda(), w.cuda(), None, out_dtype=yd)
    torch.cuda.synchronize()
    ref = CF.layernorm(x.float().numpy(), w.numpy())
    tol = {torch.float32: RTOL_F32, torch.float16: RTOL_F16, torch.bfloat16: RTOL_BF16}[yd]
    assert_close(out.float().cpu().numpy(), ref, tol, f"{xd}->{yd}")
    # f16 parameters
    out16 = abi.layernorm(x.cuda(), w.half().cuda(), None, out_dtype=yd)
    torch.cuda.synchronize()
    assert_close(out16.float().cpu().numpy(), CF.layernorm(x.float().numpy(), w.half().float().numpy()), tol, "f16 w")


@pytest.mark.parametrize("act", ["gelu", "silu"])
def test_fused_activation_f32(dev, act):
    g = configs.rng(3)
    x = g.standard_normal((64, 512)).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(512)).astype(np.float32)
    b = (0.1 * g.standard_normal(512)).astype(np.float32)
    say("layernorm + act", act)
    ln = CF.layernorm(x, w, b)
    ref = CF.gelu_erf(ln) if act == "gelu" else CF.silu(ln)
    assert_close(_ln(x, w, b, act=act), ref, RTOL_F32, act)


def test_config4a_resadd_ln_gelu_bf16(dev):
    c = configs.c4a()
    say("resadd+ln+gelu config4a bf16 [32,750,1024]")
    x, res = dev_tensor(c["x"]), dev_tensor(c["res"])
    h, y = abi.residual_add_layernorm(x, res, dev_tensor(c["gamma"]), dev_tensor(c["beta"]), act="gelu")
    torch.cuda.synchronize()
    h, y = host(h), host(y)
    wb, bb = configs.f32_to_bf16_bits(c["gamma"]), configs.f32_to_bf16_bits(c["beta"])
    h_ref, y_ref = R.resadd_ln_gelu_bf16(c["x"], c["res"], wb, bb, nthreads=16)
    assert_bitexact(h, h_ref, "h = bf16(x + res)")
    yf = configs.bf16_bits_to_f32(y)
    assert_close(yf, configs.bf16_bits_to_f32(y_ref), RTOL_BF16, "y vs bf16 chain")
    # f64 closed form on the bf16 h: one final rounding (2^-8 relative) + f32 noise
    rows = slice(0, 2000)
    hf = configs.bf16_bits_to_f32(h[rows]).astype(np.float64)
    ref = CF.gelu_erf(CF.layernorm(hf, c["gamma"], c["beta"]))
    assert np.all(np.abs(yf[rows] - ref) <= 2.0 ** -8 * np.abs(ref) * 1.001 + 1e-5)


def test_resadd_variants(dev):
    g = configs.rng(9)
    rows, cols = 50, 768
    x = g.standard_normal((rows, cols)).astype(np.float32)
    r = g.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    say("resadd f32 with and without h, no act")
    h, y = abi.residual_add_layernorm(dev_tensor(x), dev_tensor(r), dev_tensor(w), None)
    _, y2 = abi.residual_add_layernorm(dev_tensor(x), dev_tensor(r), dev_tensor(w), None, write_h=False)
    torch.cuda.synchronize()
    assert_bitexact(host(h), x + r, "h f32")
    assert_close(host(y), CF.layernorm(x + r, w), RTOL_F32, "y f32")
    assert_bitexact(host(y2), host(y), "h not written")
    # moonshine decoder profile: f16 projection + f32 residual -> f32 h, f16 norm
    say("resadd f16/f32 profile")
    xh = torch.from_numpy(x).half()
    h, y = abi.residual_add_layernorm(xh.cuda(), dev_tensor(r), dev_tensor(w).half(), None, h_dtype=torch.float32,
                                      out_dtype=torch.float16)
    torch.cuda.synchronize()
    hx = xh.float().numpy() + r
    assert_bitexact(host(h), hx, "h f32 from f16 + f32")
    assert_close(y.float().cpu().numpy(), CF.layernorm(hx, torch.from_numpy(w).half().float().numpy()), RTOL_F16,
                 "f16 norm")
    # ragged width takes the generic kernel
    say("resadd bf16 ragged width 1001")
    xb = torch.from_numpy(g.standard_normal((9, 1001)).astype(np.float32)).bfloat16()
    rb = torch.from_numpy(g.standard_normal((9, 1001)).astype(np.float32)).bfloat16()
    h, y = abi.residual_add_layernorm(xb.cuda(), rb.cuda(), None, None, act="gelu")
    torch.cuda.synchronize()
    hr = (xb.float() + rb.float()).bfloat16()
    assert torch.equal(h.cpu().view(torch.int16), hr.view(torch.int16))
    ref = CF.gelu_erf(CF.layernorm(hr.float().numpy()))
    assert_close(y.float().cpu().numpy(), ref, RTOL_BF16, "ragged bf16")


@pytest.mark.parametrize("cols", [1024, 768, 512])
def test_resadd_bf16_statistics_paths(dev, cols):
    """bf16 h: the kernel takes one-pass statistics from the packed h words and falls back to the centred
    two-pass form when mean^2 > var. Rows from mean 0 to |mean| / std = 300 cross that test; every row is
    held to one bf16 rounding of the float64 LayerNorm + GELU of the same h."""
    g = configs.rng(cols + 17)
    ratios = np.array([0.0, 0.01, 0.5, 0.9, 1.0, 1.1, 2.0, 10.0, 30.0, 300.0])
    rows = 4 * len(ratios)
    std = np.repeat(np.array([1.0, 0.01, 3.0, 100.0]), len(ratios))
    mean = np.tile(ratios, 4) * std * np.where(np.arange(rows) % 2, 1.0, -1.0)
    x = (mean[:, None] + std[:, None] * g.standard_normal((rows, cols))).astype(np.float32)
    r = (0.25 * std[:, None] * g.standard_normal((rows, cols))).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    b = (0.1 * g.standard_normal(cols)).astype(np.float32)
    xb, rb = torch.from_numpy(x).bfloat16(), torch.from_numpy(r).bfloat16()
    say("resadd bf16 statistics paths", cols)
    h, y = abi.residual_add_layernorm(xb.cuda(), rb.cuda(), dev_tensor(w), dev_tensor(b), act="gelu")
    torch.cuda.synchronize()
    hr = (xb.float() + rb.float()).bfloat16()
    assert torch.equal(h.cpu().view(torch.int16), hr.view(torch.int16)), "h = bf16(x + res)"
    ref = CF.gelu_erf(CF.layernorm(hr.double().numpy(), w, b))
    yf = y.float().cpu().numpy()
    assert np.all(np.isfinite(yf))
    err = np.abs(yf - ref)
    bound = 2.0 ** -8 * np.abs(ref) * 1.001 + 1e-5
    assert np.all(err <= bound), f"worst row {int(np.argmax((err - bound).max(axis=1)))}"


def test_resadd_bf16_gelu_extreme_inputs(dev):
    """The LayerNorm epilogue's GELU (logistic form of Phi) on pre-activations of a few 1e6 in magnitude
    (gamma 1e6, whose squares overflow f32 inside the polynomial), near 0 (gamma 1e-6) and in between: within
    one bf16 rounding of float64, no NaN."""
    g = configs.rng(23)
    rows, cols = 8, 1024
    x = g.standard_normal((rows, cols)).astype(np.float32)
    r = g.standard_normal((rows, cols)).astype(np.float32)
    w = np.tile(np.array([1e6, -1e3, 30.0, 6.0, 1.0, 1e-3, 1e-6, 0.0], dtype=np.float32), cols // 8)
    b = np.tile(np.array([0.0, 1.0, -5.0, 0.5, -40.0, 0.0, 1e-7, -2.0], dtype=np.float32), cols // 8)
    xb, rb = torch.from_numpy(x).bfloat16(), torch.from_numpy(r).bfloat16()
    say("resadd bf16 gelu extreme inputs")
    _, y = abi.residual_add_layernorm(xb.cuda(), rb.cuda(), dev_tensor(w), dev_tensor(b), act="gelu")
    torch.cuda.synchronize()
    hr = (xb.float() + rb.float()).bfloat16()
    ref = CF.gelu_erf(CF.layernorm(hr.double().numpy(), w, b))
    yf = y.float().cpu().numpy()
    assert not np.any(np.isnan(yf))
    assert np.all(np.abs(yf - ref) <= 2.0 ** -8 * np.abs(ref) * 1.001 + 1e-5)


def test_strided_rows(dev):
    g = configs.rng(10)
    rows, cols, ld = 20, 256, 320
    xs = g.standard_normal((rows, ld)).astype(np.float32)
    say("layernorm strided rows ld=320")
    xt = dev_tensor(xs)
    y = torch.full((rows, ld), 7.0, device="cuda:0")
    abi.check(abi.lib().nsr_layernorm(xt.data_ptr(), 0, None, None, 0, y.data_ptr(), 0, rows, cols, ld, ld,
                                      1e-5, 0, 0, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    yh = host(y)
    assert_close(yh[:, :cols], CF.layernorm(xs[:, :cols]), RTOL_F32, "strided")
    assert np.all(yh[:, cols:] == 7.0), "wrote outside the rows"
