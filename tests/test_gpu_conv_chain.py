"""Row statistics handed along the Kokoro ResBlock chain
(nsr_conv1d_f16w_packed_stats, nsr_adain_snake_conv1d_chain_f32): the
conv's epilogue emits (count, mean, M2) per row and 32-column block, a
merge kernel combines them (Chan's pairwise formula), and the next fused
AdaIN+Snake conv takes them instead of re-reading its input.

Checks: the output itself is bit-identical to the conv without statistics;
the statistics match the float64 mean and 1 / sqrt(var + eps) of that
output within 1e-5 (relative, and for the mean relative to the row's
spread); a two-stage chain that hands the statistics along matches the
stages run separately (each re-reading its input) within the fp32 bar.
Shapes cover the resident-weight and streamed-weight kernels, partial
32-column blocks, C_out beyond one 128-channel block, batches, residuals,
and rows that are not 16-byte aligned (the fallback kernel, whose output the
row-statistics kernel re-reads)."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs

from ._util import RTOL_F32, assert_bitexact, assert_close, say

pytestmark = pytest.mark.gpu


def _check_stats(out, st, eps, what):
    o = out.cpu().numpy().astype(np.float64)
    B, C, T = o.shape
    rows = o.reshape(B * C, T)
    mean = rows.mean(axis=1)
    var = rows.var(axis=1)
    rstd = 1.0 / np.sqrt(var + eps)
    s = st.cpu().numpy().astype(np.float64)
    spread = np.sqrt(var + eps)
    assert np.all(np.abs(s[:, 0] - mean) <= RTOL_F32 * np.maximum(np.abs(mean), spread)), what + ": mean"
    assert np.all(np.abs(s[:, 1] - rstd) <= RTOL_F32 * rstd), what + ": rstd"


@pytest.mark.parametrize("B,C_in,C_out,T,K,dil,pad,res", [
    (2, 64, 96, 1000, 3, 1, 1, False),     # resident weights, partial last 32-column block
    (1, 128, 128, 4096, 3, 5, 5, True),    # resident weights, residual
    (2, 144, 200, 1000, 5, 2, 4, True),    # streamed weights, two output blocks of channels
    (1, 128, 128, 2048, 11, 5, 25, False), # streamed weights, K = 11
    (1, 64, 64, 257, 3, 1, 1, False),      # rows not 16-byte aligned: fallback + statistics kernel
    (3, 32, 16, 36, 2, 1, 0, True),        # a single short tile
])
def test_conv_stats(B, C_in, C_out, T, K, dil, pad, res):
    say("conv1d packed stats", B, C_in, C_out, T, K, dil, pad, res)
    g = configs.rng(B * 11 + C_in + K + T)
    x = g.standard_normal((B, C_in, T)).astype(np.float32)
    w = (g.standard_normal((C_out, C_in, K)) * 0.1).astype(np.float16)
    b = g.standard_normal(C_out).astype(np.float16)
    T_out = T + 2 * pad - dil * (K - 1)
    r = torch.from_numpy((g.standard_normal((B, C_out, T_out)) + 0.5).astype(np.float32)).cuda() if res else None
    wp = abi.conv1d_pack_f16(torch.from_numpy(w).cuda())
    xt, bt = torch.from_numpy(x).cuda(), torch.from_numpy(b).cuda()
    out, st = abi.conv1d_f16w_packed_stats(xt, wp, bt, r, padding=pad, dilation=dil, eps=1e-5)
    plain = abi.conv1d_f16w_packed(xt, wp, bt, r, padding=pad, dilation=dil)
    assert_bitexact(out.cpu().numpy(), plain.cpu().numpy(), "output with and without statistics")
    _check_stats(out, st, 1e-5, f"conv stats {B}x{C_in}->{C_out} T={T} K={K}")


@pytest.mark.parametrize("B,C,T,K,dil", [(2, 128, 4096, 3, 1), (1, 128, 3000, 3, 3), (1, 192, 2048, 5, 2),
                                         (1, 128, 2048, 11, 5), (1, 64, 1001, 3, 1)])
def test_resblock_chain(B, C, T, K, dil):
    """conv1(snake(AdaIN1(x))) then conv2(snake(AdaIN2(.))) + x, with the
    statistics of conv1's output handed to stage 2 (and stage 2's output
    statistics checked), against the stages run separately."""
    say("resblock chain", B, C, T, K, dil)
    g = configs.rng(B + C + T + K)
    x = (g.standard_normal((B, C, T)) * 1.5 + 0.3).astype(np.float32)
    p = lambda *sh: torch.from_numpy((g.standard_normal(sh) * 0.1).astype(np.float32)).cuda()  # noqa: E731
    g1, b1, g2, b2 = p(B, C), p(B, C), p(B, C), p(B, C)
    a1 = torch.from_numpy(g.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    a2 = torch.from_numpy(g.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    w1 = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).cuda())
    w2 = abi.conv1d_pack_f16(torch.from_numpy((g.standard_normal((C, C, K)) * 0.05).astype(np.float16)).cuda())
    bb1 = torch.from_numpy(g.standard_normal(C).astype(np.float16)).cuda()
    bb2 = torch.from_numpy(g.standard_normal(C).astype(np.float16)).cuda()
    pad = (K - 1) * dil // 2
    xt = torch.from_numpy(x).cuda()
    # chained
    h, s_h = abi.adain_snake_conv1d_chain(xt, g1, b1, a1, w1, bb1, padding=pad, dilation=dil)
    y, s_y = abi.adain_snake_conv1d_chain(h, g2, b2, a2, w2, bb2, xt, x_stats=s_h, padding=pad, dilation=dil)
    # separate stages
    h_ref = abi.adain_snake_conv1d(xt, g1, b1, a1, w1, bb1, padding=pad, dilation=dil)
    y_ref = abi.adain_snake_conv1d(h_ref, g2, b2, a2, w2, bb2, xt, padding=pad, dilation=dil)
    assert_bitexact(h.cpu().numpy(), h_ref.cpu().numpy(), "stage 1 output")
    _check_stats(h, s_h, 1e-5, "stage 1 statistics")
    _check_stats(y, s_y, 1e-5, "stage 2 statistics")
    assert_close(y.cpu().numpy(), y_ref.cpu().numpy(), RTOL_F32, "stage 2 with handed-over statistics")
