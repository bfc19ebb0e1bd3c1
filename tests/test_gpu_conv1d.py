"""Kokoro resblock conv1d on MFMA vs the oracle's restatement of
conv1d_f32io (kernels/kokoro_kernels.py:773-816), including the reference's
own GPU self-test shapes and inputs (src/kokoro/gpu_decoder.rs:64-76,
401-456: x[i] = 2 sin(0.001 i), w[i] = f16(0.1 cos(1e-4 i)), bias[i] =
f16(0.001 i)), and the fused AdaIN1d + Snake -> conv stage vs the oracle's
adain_snake followed by conv1d_f32io.

The GPU sums the same products in another order (and splits each f32
activation into two f16 halves, exact to 2^-22 relative), so the bar for the
conv is the fp32 parity tolerance: |gpu - ref| <= 1e-5 * max(|ref|, 1). The
fused stage composes two fp32 ops: its bar is the AdaIN+Snake tolerance
(1e-5 * max(|y|, 1) per activation) carried through the conv,
sum |w| * 1e-5 * max(|y|, 1), plus the conv's own tolerance."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import restated as R

from ._util import RTOL_F32, assert_close, say

pytestmark = pytest.mark.gpu


def _ref_inputs(C_in, C_out, T, K):
    i = np.arange(C_in * T, dtype=np.float32)
    x = (np.sin(i * np.float32(0.001)) * np.float32(2.0)).astype(np.float32).reshape(1, C_in, T)
    j = np.arange(C_out * C_in * K, dtype=np.float32)
    w = (np.cos(j * np.float32(0.0001)) * np.float32(0.1)).astype(np.float16).reshape(C_out, C_in, K)
    b = (np.arange(C_out, dtype=np.float32) * np.float32(0.001)).astype(np.float16)
    return x, w, b


@pytest.mark.parametrize("C,T,K,dil,pad", [
    (256, 1880, 3, 1, 1), (256, 1880, 7, 3, 9), (256, 1880, 11, 5, 25),        # the reference's stage-0 cases
    (128, 11281, 3, 1, 1), (128, 11281, 3, 3, 3), (128, 11281, 3, 5, 5),       # stage-1 cases
    (128, 11281, 7, 1, 3), (128, 11281, 7, 3, 9), (128, 11281, 7, 5, 15),
    (128, 11281, 11, 1, 5), (128, 11281, 11, 3, 15), (128, 11281, 11, 5, 25)])
def test_conv1d_f32io_reference_self_test_shapes(dev, C, T, K, dil, pad):
    say("conv1d_f32io", C, T, K, dil, pad)
    x, w, b = _ref_inputs(C, C, T, K)
    out = abi.conv1d_f32io(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(),
                           padding=pad, dilation=dil)
    torch.cuda.synchronize()
    ref = R.conv1d_f32io(x, w.view(np.uint16), b.view(np.uint16), 1, pad, dil, nthreads=16)
    assert_close(out.cpu().numpy(), ref, RTOL_F32, f"conv1d C={C} K={K} dil={dil}")


@pytest.mark.parametrize("B,C_in,C_out,T,K,dil,pad,res", [
    (2, 32, 48, 300, 3, 1, 1, False),    # C_out not a multiple of 128, several batches
    (1, 16, 16, 5, 3, 1, 1, True),       # shorter than one tile, residual
    (3, 144, 200, 257, 5, 2, 0, True),   # a 16-channel last chunk, valid padding (T_out < T_in)
    (1, 512, 128, 130, 1, 1, 0, False),  # 1x1 conv, four input chunks
    # resident-weight kernel (C_in, C_out <= 128, K <= 3, T_out % 4 == 0):
    (2, 64, 96, 1000, 3, 2, 2, True),    # residual, two batches
    (1, 128, 128, 4096, 3, 5, 5, False), # 74 staged columns (the wider staging variant)
    (1, 32, 32, 9, 2, 1, 0, True),       # K = 2, a single tile
    # streamed-weight kernel (16-byte aligned rows, other shapes):
    (2, 144, 200, 1000, 5, 2, 4, True),  # two input chunks (the last of 16 channels), two output blocks, residual
    (1, 512, 128, 132, 1, 1, 0, False),  # 1x1 conv, four input chunks
])
def test_conv1d_packed_edges(dev, B, C_in, C_out, T, K, dil, pad, res):
    say("conv1d packed", B, C_in, C_out, T, K, dil, pad, res)
    g = configs.rng(B * 7 + C_in + K)
    x = g.standard_normal((B, C_in, T)).astype(np.float32)
    w = (g.standard_normal((C_out, C_in, K)) * 0.1).astype(np.float16)
    b = g.standard_normal(C_out).astype(np.float16)
    wt = torch.from_numpy(w).cuda()
    wp = abi.conv1d_pack_f16(wt)
    T_out = T + 2 * pad - dil * (K - 1)
    r = g.standard_normal((B, C_out, T_out)).astype(np.float32) if res else None
    out = abi.conv1d_f16w_packed(torch.from_numpy(x).cuda(), wp, torch.from_numpy(b).cuda(),
                                 torch.from_numpy(r).cuda() if res else None, padding=pad, dilation=dil)
    torch.cuda.synchronize()
    assert np.array_equal(wp.cpu().numpy(), np.ascontiguousarray(w.transpose(0, 2, 1))), "packed layout"
    ref = R.conv1d_f32io(x, w.view(np.uint16), b.view(np.uint16), 1, pad, dil, nthreads=16)
    if res:
        ref = ref + r
    assert_close(out.cpu().numpy(), ref, RTOL_F32, "conv1d packed")


@pytest.mark.parametrize("B,C,T,K,dil,pdt,per_batch,with_res", [
    (1, 128, 4800, 3, 1, "f32", False, True),
    (2, 128, 3000, 11, 5, "f16", True, True),
    (1, 256, 1880, 7, 3, "f16", False, True),
    (3, 128, 2048, 3, 1, "f16", True, False),   # no residual; the batch index changes between tiles
    (1, 128, 1024, 3, 5, "f32", False, True),   # 74 staged columns
])
def test_adain_snake_conv1d_fused(dev, B, C, T, K, dil, pdt, per_batch, with_res):
    """One ResBlock stage: conv1d(snake(AdaIN(x))) + bias (+ residual), fused,
    vs the oracle's adain_snake then conv1d_f32io (f64-pinned pieces)."""
    say("adain_snake_conv1d", B, C, T, K, dil, pdt, per_batch, with_res)
    g = configs.rng(B + C + K)
    x = (g.standard_normal((B, C, T)) * 1.5 + 0.3).astype(np.float32)
    tdt = np.float32 if pdt == "f32" else np.float16
    gam = (g.standard_normal((B, C) if per_batch else C) * 0.1).astype(tdt)
    bet = (g.standard_normal((B, C) if per_batch else C) * 0.1).astype(tdt)
    alp = g.uniform(0.5, 1.5, C).astype(tdt)
    w = (g.standard_normal((C, C, K)) * 0.05).astype(np.float16)
    b = g.standard_normal(C).astype(np.float16)
    pad = (K - 1) * dil // 2
    res = g.standard_normal((B, C, T)).astype(np.float32)
    wp = abi.conv1d_pack_f16(torch.from_numpy(w).cuda())
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    out = abi.adain_snake_conv1d(dt(x), dt(gam), dt(bet), dt(alp), wp, dt(b), dt(res) if with_res else None,
                                 padding=pad, dilation=dil)
    torch.cuda.synchronize()
    y = R.adain_snake(x, gam.astype(np.float32), bet.astype(np.float32), alp.astype(np.float32))
    ref = R.conv1d_f32io(y, w.view(np.uint16), b.view(np.uint16), 1, pad, dil, nthreads=16)
    if with_res:
        ref = ref + res
    # the AdaIN+Snake bar carried through the conv: sum_k |w| * 1e-5 * max(|y|, 1)
    wabs = np.abs(w.astype(np.float32)).astype(np.float16)
    carried = R.conv1d_f32io(np.maximum(np.abs(y), 1.0).astype(np.float32), wabs.view(np.uint16), None, 1, pad, dil,
                             nthreads=16).astype(np.float64) * RTOL_F32 * 1.01
    got = out.cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    bound = carried + RTOL_F32 * np.maximum(np.abs(ref), 1.0)
    assert np.all(err <= bound), f"max excess {float(np.max(err - bound)):.3e}"
    print(f"[fused conv] max scaled error {float(np.max(err / np.maximum(np.abs(ref), 1.0))):.3e}, "
          f"max err / bound {float(np.max(err / bound)):.3f}")
