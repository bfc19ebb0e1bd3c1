"""The conv's record path (NSR_WS_RECORDS in the workspace): a bandwidth-
bound pass writes the input as f16 hi / lo records (AdaIN + Snake included
in the fused entry points) and the weights in MFMA fragment order, then an
MFMA kernel with no per-element VALU work reads them. It adds the same
products in the same order as the one-launch kernels (per output tile:
input-channel chunks, then taps, then 16-channel steps, hi before lo), so
each entry point's output must match its one-launch form bit for bit; the
one-launch forms are checked against the oracle and float64 in
test_gpu_conv1d.py and test_gpu_conv_chain.py. The record path is taken from
K = 7 on; shapes: K = 7 / 8 / 9 / 11 at several dilations (an odd (K - 1)
dilation among them), a partial 128-channel input chunk (C_in = 144, 96),
two input chunks and two output blocks (C = 256, C_out = 200), batches,
residuals, statistics handed along; and the one-launch fallbacks: K = 3 and
5 (below the threshold), rows that are not 16-byte aligned, an odd C_out."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs

from ._util import assert_bitexact, assert_close, say

pytestmark = pytest.mark.gpu

SHAPES = [  # B, C_in, C_out, T, K, dil, res
    (1, 128, 128, 4096, 7, 1, False),
    (2, 128, 128, 2048, 11, 5, True),
    (1, 256, 256, 1880, 7, 3, True),
    (2, 144, 200, 1000, 7, 5, True),
    (1, 96, 96, 3000, 9, 5, False),
    (3, 128, 64, 512, 11, 1, False),
    (2, 64, 96, 1001, 8, 1, False),   # (K - 1) dilation = 7, odd
    (1, 128, 128, 4096, 3, 1, False),  # K < 7: the one-launch kernels both ways
    (2, 144, 200, 1000, 5, 2, True),
    (1, 64, 64, 601, 5, 2, False),    # T_out % 4 != 0: the one-launch kernels (no record path)
    (1, 128, 127, 1024, 7, 3, False),  # odd C_out: the one-launch kernels
]


def _inputs(B, C_in, C_out, T, K, dil, res):
    g = configs.rng(B * 7 + C_in + 3 * K + dil)
    x = torch.from_numpy((g.standard_normal((B, C_in, T)) * 1.3 + 0.2).astype(np.float32)).cuda()
    w = torch.from_numpy((g.standard_normal((C_out, C_in, K)) * 0.05).astype(np.float16)).cuda()
    b = torch.from_numpy(g.standard_normal(C_out).astype(np.float16)).cuda()
    pad = (K - 1) * dil // 2
    T_out = T + 2 * pad - dil * (K - 1)
    r = torch.from_numpy(g.standard_normal((B, C_out, T_out)).astype(np.float32)).cuda() if res else None
    gam = torch.from_numpy((g.standard_normal((B, C_in)) * 0.1).astype(np.float32)).cuda()
    bet = torch.from_numpy((g.standard_normal((B, C_in)) * 0.1).astype(np.float32)).cuda()
    alp = torch.from_numpy(g.uniform(0.5, 1.5, C_in).astype(np.float32)).cuda()
    return x, w, b, r, gam, bet, alp, pad


@pytest.mark.parametrize("B,C_in,C_out,T,K,dil,res", SHAPES)
def test_records_match_one_launch(B, C_in, C_out, T, K, dil, res):
    say("conv records", B, C_in, C_out, T, K, dil, res)
    x, w, b, r, gam, bet, alp, pad = _inputs(B, C_in, C_out, T, K, dil, res)
    if not res:  # conv1d_f32io has no residual
        o1 = abi.conv1d_f32io(x, w, b, padding=pad, dilation=dil, records=True)
        o0 = abi.conv1d_f32io(x, w, b, padding=pad, dilation=dil, records=False)
        assert_bitexact(o1.cpu().numpy(), o0.cpu().numpy(), "conv1d_f32io")
    wp = abi.conv1d_pack_f16(w)
    f1 = abi.adain_snake_conv1d(x, gam, bet, alp, wp, b, r, padding=pad, dilation=dil, records=True)
    f0 = abi.adain_snake_conv1d(x, gam, bet, alp, wp, b, r, padding=pad, dilation=dil, records=False)
    assert_bitexact(f1.cpu().numpy(), f0.cpu().numpy(), "adain_snake_conv1d")
    c1, s1 = abi.adain_snake_conv1d_chain(x, gam, bet, alp, wp, b, r, padding=pad, dilation=dil, records=True)
    c0, s0 = abi.adain_snake_conv1d_chain(x, gam, bet, alp, wp, b, r, padding=pad, dilation=dil, records=False)
    assert_bitexact(c1.cpu().numpy(), c0.cpu().numpy(), "adain_snake_conv1d_chain output")
    if T % 4 == 0:
        assert_bitexact(s1.cpu().numpy(), s0.cpu().numpy(), "adain_snake_conv1d_chain statistics")
    else:
        # rows not 16-byte aligned on input: the one-launch path takes the statistics from a pass over its
        # output instead of per-32-column partials, another summation order
        assert_close(s1.cpu().numpy(), s0.cpu().numpy(), 1e-5, "adain_snake_conv1d_chain statistics")
    p1, q1 = abi.conv1d_f16w_packed_stats(x, wp, b, r, padding=pad, dilation=dil, records=True)
    p0 = abi.conv1d_f16w_packed(x, wp, b, r, padding=pad, dilation=dil)
    assert_bitexact(p1.cpu().numpy(), p0.cpu().numpy(), "conv1d_f16w_packed_stats vs conv1d_f16w_packed")


def test_records_repeated_calls_and_workspace_reuse():
    """Two calls in a row on one workspace (the second smaller) give the one-launch results."""
    for shape in [(2, 128, 128, 2048, 11, 5, False), (1, 128, 128, 1024, 7, 3, False)]:
        B, C_in, C_out, T, K, dil, res = shape
        x, w, b, r, gam, bet, alp, pad = _inputs(*shape)
        ws = abi.conv_workspace(2, 128, 128, 2048, 11, 25, 5, abi.WS_PACKED_WEIGHTS | abi.WS_RECORDS)
        o1 = abi.conv1d_f32io(x, w, b, padding=pad, dilation=dil, workspace=ws)
        o0 = abi.conv1d_f32io(x, w, b, padding=pad, dilation=dil, records=False)
        assert_bitexact(o1.cpu().numpy(), o0.cpu().numpy(), f"reused workspace {shape}")
