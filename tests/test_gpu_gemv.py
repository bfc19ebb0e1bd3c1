"""Repacked-Q8 GEMV family on the GPU vs the oracle's restatement of
gemv_q8 / gemv_q8_bias / gemv_q8_bias_glu / gemv_q8_resadd_ln
(kernels/moonshine_kernels.py:616-677, 1721-1819), over the reference's
repacked-Q8 layout ("ref") and over the t4 tiles nsr_q8_pack_t4 makes
("t4"; the packing itself is checked bit for bit against the oracle's
restatement).

The GPU adds the same f32 products in another order (split over K), so the
bar is the f32 accumulation error bound rather than bit equality: two f32
sums of the same K products each lie within gamma_K * sum|x_k w_k| of the
exact sum, so they differ by at most twice that. f16 outputs add one f16 ulp
(the two sums may round to neighbouring f16 values); every result also meets
the f16 tolerance of the parity bar. Repeated calls are bit-identical (every
sum is formed in a fixed order)."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import restated as R

from ._util import RTOL_F16, assert_bitexact, assert_close, say

pytestmark = pytest.mark.gpu

_TD = {"f16": torch.float16, "f32": torch.float32}


def _weight(g, K, NW):
    qs = g.integers(0, 2 ** 32, size=(K, NW // 4), dtype=np.uint64).astype(np.uint32)
    sc = (g.standard_normal((K // 32, NW)) * 0.02).astype(np.float16)
    W = qs.view(np.int8).reshape(K, NW).astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=0)
    return qs, sc, W


def _dev_w(qs, sc):
    return (torch.from_numpy(qs.view(np.int32)).cuda(), torch.from_numpy(sc).cuda())


def _run(layout, fn, xt, q_t, s_t, *args, glu=False, **kw):
    """Call the reference-layout entry point, or pack to t4 and call its twin."""
    if layout == "ref":
        return getattr(abi, fn)(xt, q_t, s_t, *args, **kw)
    w = abi.Q8T4(q_t, s_t, glu=glu)
    return getattr(abi, fn.replace("gemv_q8", "gemv_q8_t4"))(xt, w, *args, **kw)


def _bound(x, W):
    K = x.shape[0]
    u = 2.0 ** -24
    return (K + 2) * u / (1 - (K + 2) * u) * (np.abs(x.astype(np.float64)) @ np.abs(W))


def _f16_ulp(v):
    return np.spacing(np.abs(v).astype(np.float16)).astype(np.float64)


def _x(g, K, xd):
    x16 = g.standard_normal(K).astype(np.float16)
    xt = torch.from_numpy(x16).cuda().to(_TD[xd])
    return x16.astype(np.float32), xt


def _check(got_t, ref, e, odt, what):
    got = got_t.float().cpu().numpy().astype(np.float64)
    if odt == "f16":
        bound = 2 * e + _f16_ulp(np.abs(ref) + 2 * e) + 1e-7
        assert_close(got, ref.astype(np.float16).astype(np.float64), RTOL_F16, what)
    else:
        bound = 2 * e + np.abs(ref) * 2.0 ** -22
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{what}: {bad.sum()} outside the bound, first {np.flatnonzero(bad)[:5]}"


@pytest.mark.parametrize("layout", ["ref", "t4"])
@pytest.mark.parametrize("K,N,xd,od,with_bias", [
    (288, 288, "f16", "f16", True),      # Moonshine tiny decoder dim (kernel_configs.py)
    (416, 416, "f16", "f16", False),     # Moonshine base decoder dim
    (640, 640, "f16", "f16", True),      # bench decoder projection
    (2560, 640, "f16", "f16", True),     # MLP fc2 (intermediate -> dim)
    (640, 1920, "f16", "f32", False),    # fused q|k|v projection
    (288, 32768, "f16", "f32", False),   # vocabulary projection
    (4096, 4096, "f16", "f16", False),   # many K chunks per tile
    (96, 272, "f32", "f16", True),       # a 16-column second tile
    (32, 16, "f32", "f32", True),        # smallest legal shape, one K chunk
])
def test_gemv_q8(dev, layout, K, N, xd, od, with_bias):
    say("gemv_q8", layout, K, N, xd, od, with_bias)
    g = configs.rng(K * 3 + N)
    qs, sc, W = _weight(g, K, N)
    x, xt = _x(g, K, xd)
    bias = g.standard_normal(N).astype(np.float32) if with_bias else None
    bt = torch.from_numpy(bias).cuda() if with_bias else None
    q_t, s_t = _dev_w(qs, sc)
    out = _run(layout, "gemv_q8", xt, q_t, s_t, bt, out_dtype=_TD[od])
    out2 = _run(layout, "gemv_q8", xt, q_t, s_t, bt, out_dtype=_TD[od])
    torch.cuda.synchronize()
    ref = R.gemv_q8(x, qs, sc.view(np.uint16), bias).astype(np.float64)
    _check(out, ref, _bound(x, W), od, f"gemv_q8 K={K} N={N}")
    assert_bitexact(out2.cpu().numpy(), out.cpu().numpy(), "repeat call")


@pytest.mark.parametrize("layout", ["ref", "t4"])
@pytest.mark.parametrize("K,N,xd,od", [
    (640, 2560, "f16", "f16"),   # Moonshine decoder fc1 + GLU (dim 640, intermediate 2560)
    (288, 1152, "f16", "f16"),
    (96, 144, "f32", "f32"),     # a 16-column second tile
    (32, 16, "f16", "f32"),
])
def test_gemv_q8_bias_glu(dev, layout, K, N, xd, od):
    say("gemv_q8_bias_glu", layout, K, N, xd, od)
    g = configs.rng(K * 5 + N)
    qs, sc, W = _weight(g, K, 2 * N)
    x, xt = _x(g, K, xd)
    bias = g.standard_normal(2 * N).astype(np.float32)
    q_t, s_t = _dev_w(qs, sc)
    out = _run(layout, "gemv_q8_bias_glu", xt, q_t, s_t, torch.from_numpy(bias).cuda(), out_dtype=_TD[od],
               glu=True)
    torch.cuda.synchronize()
    ref = R.gemv_q8(x, qs, sc.view(np.uint16), bias, glu=True).astype(np.float64)
    pre = x.astype(np.float64) @ W + bias
    e2 = 2 * _bound(x, W)
    xa, ga = pre[:N], pre[N:]
    sil = ga / (1 + np.exp(-ga))
    # an error d in the gate moves silu by at most 1.1 d; silu itself is
    # computed with the hardware exp2 / reciprocal (a few f32 ulps)
    e = 1.1 * e2[N:] * np.abs(xa) + np.abs(sil) * e2[:N] + np.abs(ref) * 2.0 ** -19 + 2.0 ** -30
    _check(out, ref, e / 2, od, f"gemv_q8_bias_glu K={K} N={N}")


@pytest.mark.parametrize("layout", ["ref", "t4"])
@pytest.mark.parametrize("K,dim,xd,wd,nd,in_place", [
    (2560, 640, "f16", "f16", "f16", False),  # decoder fc2 + residual + next LN (dim 640)
    (640, 640, "f16", "f16", "f16", True),    # attention out-projection, residual updated in place
    (288, 288, "f16", "f16", "f16", False),   # one tile
    (1152, 288, "f32", "f32", "f32", False),
    (32, 16, "f16", "f16", "f16", False),
])
def test_gemv_q8_resadd_ln(dev, layout, K, dim, xd, wd, nd, in_place):
    say("gemv_q8_resadd_ln", layout, K, dim, xd, wd, nd, in_place)
    g = configs.rng(K * 7 + dim)
    qs, sc, W = _weight(g, K, dim)
    x, xt = _x(g, K, xd)
    res = g.standard_normal(dim).astype(np.float32)
    w16 = (1 + 0.1 * g.standard_normal(dim)).astype(np.float16)
    q_t, s_t = _dev_w(qs, sc)
    res_t = torch.from_numpy(res).cuda()
    w_t = torch.from_numpy(w16).cuda().to(_TD[wd])
    h, norm = _run(layout, "gemv_q8_resadd_ln", xt, q_t, s_t, res_t, w_t, eps=1e-5,
                   out_f32=res_t if in_place else None, norm_dtype=_TD[nd])
    torch.cuda.synchronize()
    h_ref, _ = R.gemv_q8_resadd_ln(x, qs, sc.view(np.uint16), res, w16.view(np.uint16), 1e-5)
    proj = x.astype(np.float64) @ W
    e2 = 2 * _bound(x, W)
    hg = h.cpu().numpy().astype(np.float64)
    bound = e2 + _f16_ulp(np.abs(proj) + e2) + np.abs(h_ref) * 2.0 ** -23
    assert np.all(np.abs(hg - h_ref) <= bound), "h outside the accumulation bound"
    assert_close(hg, h_ref, RTOL_F16, "h")
    # the LN stage, checked exactly against the GPU's own h
    mu = hg.mean()
    n64 = (hg - mu) / np.sqrt(((hg - mu) ** 2).mean() + 1e-5) * w16.astype(np.float64)
    ng = norm.float().cpu().numpy().astype(np.float64)
    tol = (_f16_ulp(n64) if nd == "f16" else np.abs(n64) * 2.0 ** -20) + 1e-6
    assert np.all(np.abs(ng - n64) <= tol), float(np.max(np.abs(ng - n64) - tol))


@pytest.mark.parametrize("K,NW,glu", [(640, 5120, True), (2560, 640, False), (32, 16, False), (96, 288, True)])
def test_q8_pack_t4_bitexact(dev, K, NW, glu):
    say("q8_pack_t4", K, NW, glu)
    g = configs.rng(K + NW + glu)
    qs, sc, _ = _weight(g, K, NW)
    q_t, s_t = _dev_w(qs, sc)
    w = abi.Q8T4(q_t, s_t, glu=glu)
    torch.cuda.synchronize()
    tq, ts = R.q8_pack_t4(qs, sc.view(np.uint16), glu=glu)
    assert_bitexact(w.qs.cpu().numpy().view(np.uint32), tq, "t4 words")
    assert_bitexact(w.scales.cpu().numpy().view(np.uint16), ts, "t4 scales")


def test_gemv_q8_streams_and_repeats_agree(dev):
    """The same call on two streams, and again after other shapes ran, gives
    bit-identical results on both layouts."""
    g = configs.rng(77)
    K, N = 2560, 640
    qs, sc, _ = _weight(g, K, N)
    x, xt = _x(g, K, "f16")
    q_t, s_t = _dev_w(qs, sc)
    for layout in ("ref", "t4"):
        say("gemv_q8 streams", layout, K, N)
        base = _run(layout, "gemv_q8", xt, q_t, s_t)
        torch.cuda.synchronize()
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        outs = []
        for s in (s1, s2, s1):
            with torch.cuda.stream(s):
                outs.append(_run(layout, "gemv_q8", xt, q_t, s_t, stream=s))
        qs2, sc2, _ = _weight(g, 640, 5120)
        q2, s2t = _dev_w(qs2, sc2)
        _, x2 = _x(g, 640, "f16")
        _run(layout, "gemv_q8", x2, q2, s2t)
        again = _run(layout, "gemv_q8", xt, q_t, s_t)
        torch.cuda.synchronize()
        for o in outs + [again]:
            assert_bitexact(o.cpu().numpy(), base.cpu().numpy(), f"{layout}: same result on every stream and call")
