"""SiLU / GELU(erf), GLU-SiLU and residual add on the GPU vs the oracle
(candle silu/gelu_erf, DecoderMLP GLU src/moonshine/decoder.rs:406-409,
FastAddOp src/fast_ops.rs:32-34)."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_BF16, RTOL_F16, RTOL_F32, assert_bitexact, assert_close, dev_tensor, host, say

pytestmark = pytest.mark.gpu

TOL = {torch.float32: RTOL_F32, torch.float16: RTOL_F16, torch.bfloat16: RTOL_BF16}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 7, 8, 1000, 4096 * 416 + 3])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_activation(dev, dtype, n, act):
    g = configs.rng(n)
    x = torch.from_numpy((g.standard_normal(n) * 4).astype(np.float32)).to(dtype)
    say("activation", act, dtype, n)
    y = abi.activation(x.cuda(), act)
    torch.cuda.synchronize()
    xf = x.float().numpy()
    ref = CF.silu(xf) if act == "silu" else CF.gelu_erf(xf)
    assert_close(y.float().cpu().numpy(), ref, TOL[dtype], f"{act} {dtype} n={n}")
    if dtype == torch.float32:
        orc = R.silu(xf) if act == "silu" else R.gelu_erf(xf)
        assert_close(y.cpu().numpy(), orc, RTOL_F32, "vs oracle")


def test_activation_unaligned_view(dev):
    g = configs.rng(1)
    x = torch.from_numpy(g.standard_normal(1001).astype(np.float32)).cuda()[1:]
    say("activation unaligned view")
    y = abi.activation(x, "silu")
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), CF.silu(x.cpu().numpy()), RTOL_F32, "unaligned")


def test_golden_activations(dev):
    from .golden import make_golden

    c = make_golden.load_all()["act_f32_1000"]
    say("activation golden")
    x = dev_tensor(c["x"])
    ys, yg = abi.activation(x, "silu"), abi.activation(x, "gelu")
    torch.cuda.synchronize()
    assert_close(host(ys), c["out_silu"], RTOL_F32, "golden silu")
    assert_close(host(yg), c["out_gelu"], RTOL_F32, "golden gelu")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [5, 64, 1536, 100003])
def test_glu_silu(dev, dtype, n):
    g = configs.rng(n + 3)
    fc1 = torch.from_numpy(g.standard_normal(2 * n).astype(np.float32)).to(dtype)
    say("glu_silu", dtype, n)
    out = abi.glu_silu(fc1.cuda())
    torch.cuda.synchronize()
    f = fc1.float().numpy()
    assert_close(out.float().cpu().numpy(), CF.silu(f[n:]) * f[:n], TOL[dtype], f"glu {dtype} {n}")
    if dtype == torch.float32:
        assert_close(out.cpu().numpy(), R.glu_silu(f), RTOL_F32, "glu vs oracle")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [3, 4096, 24576000 // 64 + 5])
def test_residual_add(dev, dtype, n):
    g = configs.rng(n + 9)
    a = torch.from_numpy(g.standard_normal(n).astype(np.float32)).to(dtype)
    b = torch.from_numpy(g.standard_normal(n).astype(np.float32)).to(dtype)
    say("residual_add", dtype, n)
    out = abi.residual_add(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    ref = (a.float() + b.float()).to(dtype)  # one rounding of the exact f32 sum
    assert torch.equal(out.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if dtype != torch.float32 else torch.int32))
    if dtype == torch.float32:
        assert_bitexact(out.cpu().numpy(), R.fast_add(a.numpy(), b.numpy()), "vs FastAddOp")
