"""Partial interleaved rotary on the GPU vs apply_rotary_pos_emb
(src/moonshine/decoder.rs:85-183).

With the host-built RoPE table (src/moonshine/gpu_decoder.rs:326-340) the
kernel repeats the reference's f32 op sequence and is bit-exact against the
oracle; with in-kernel sin/cos it is within 1e-5.
"""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_F32, assert_bitexact, assert_close, dev_tensor, host, say

pytestmark = pytest.mark.gpu


def _rot(q, k, rot, theta, pos0, table):
    tab = None
    if table:
        tab = abi.rope_table(pos0 + q.shape[2], rot, theta).cuda()
    qo, ko = abi.rotary(dev_tensor(q), None if k is None else dev_tensor(k), rot, theta, pos0, table=tab)
    torch.cuda.synchronize()
    return host(qo), None if ko is None else host(ko)


@pytest.mark.parametrize("table", [True, False])
def test_config1(dev, table):
    c = configs.c1()
    say("rotary config1 [1,8,1024,64] rot32 table=", table)
    qo, ko = _rot(c["q"], c["k"], 32, 10000.0, 0, table)
    rq = R.rotary(c["q"], 32, 10000.0, 0, nthreads=8)
    rk = R.rotary(c["k"], 32, 10000.0, 0, nthreads=8)
    if table:
        assert_bitexact(qo, rq, "q (table)")
        assert_bitexact(ko, rk, "k (table)")
    else:
        assert_close(qo, rq, RTOL_F32, "q (in-kernel sincos)")
        assert_close(ko, rk, RTOL_F32, "k (in-kernel sincos)")
    assert_close(qo, CF.rotary(c["q"], 32, 10000.0, 0), RTOL_F32, "q vs complex rotation")
    assert_bitexact(qo[..., 32:], c["q"][..., 32:], "pass-through")


@pytest.mark.parametrize("table", [True, False])
@pytest.mark.parametrize("B,Hq,Hk,T,Dh,rot,theta,pos0", [
    (2, 4, 2, 37, 64, 32, 10000.0, 0),        # GQA, ragged T
    (1, 3, 3, 5, 64, 64, 10000.0, 1000),      # full rotation, offset positions
    (1, 2, 1, 8, 128, 64, 500000.0, 4090),    # long-context theta
    (3, 1, 1, 1, 36, 4, 10.0, 7),             # one position, tiny rot
    (1, 8, 8, 513, 64, 0, 10000.0, 0),        # rot 0: pure copy
])
def test_shapes(dev, table, B, Hq, Hk, T, Dh, rot, theta, pos0):
    g = configs.rng(B * 100 + T)
    q = g.standard_normal((B, Hq, T, Dh)).astype(np.float32)
    k = g.standard_normal((B, Hk, T, Dh)).astype(np.float32)
    say("rotary", B, Hq, Hk, T, Dh, rot, theta, pos0, "table=", table)
    qo, ko = _rot(q, k, rot, theta, pos0, table and rot > 0)
    for got, x, nm in ((qo, q, "q"), (ko, k, "k")):
        ref = R.rotary(x, rot, theta, pos0)
        if table and rot > 0:
            assert_bitexact(got, ref, nm)
        else:
            assert_close(got, ref, RTOL_F32, nm)
        assert_close(got, CF.rotary(x, rot, theta, pos0), RTOL_F32, nm + " closed form")


def test_q_only_and_in_place(dev):
    c = configs.c1(T=64)
    say("rotary q only, in place")
    qt = dev_tensor(c["q"])
    abi.rotary(qt, None, 32, 10000.0, 3, q_out=qt)
    torch.cuda.synchronize()
    assert_close(host(qt), R.rotary(c["q"], 32, 10000.0, 3), RTOL_F32, "in place")


def test_golden(dev):
    from .golden import make_golden

    c = make_golden.load_all()["rope_b1h2t16_pos5"]
    say("rotary golden")
    rot, theta, pos0 = int(c["rot"]), float(c["theta"]), int(c["pos0"])
    assert_bitexact(abi.rope_table(pos0 + 16, rot, theta).numpy(), c["table"], "table")
    qo, _ = _rot(c["q"], None, rot, theta, pos0, True)
    assert_bitexact(qo, c["out"], "golden table path")
    qo, _ = _rot(c["q"], None, rot, theta, pos0, False)
    assert_close(qo, c["out"], RTOL_F32, "golden in-kernel path")


def test_norm_preserved_at_large_positions(dev):
    """Size-independent property at long positions: each rotated pair keeps
    its norm, and position p of a sequence equals position 0 of a sequence
    starting at pos0 = p."""
    g = configs.rng(77)
    q = g.standard_normal((1, 4, 300, 64)).astype(np.float32)
    say("rotary pos0 shift property")
    a, _ = _rot(q, None, 32, 10000.0, 2000, False)
    b, _ = _rot(q[:, :, 100:101], None, 32, 10000.0, 2100, False)
    assert_bitexact(a[:, :, 100:101], b, "shift invariance")
    n_in = q[..., :32:2] ** 2 + q[..., 1:32:2] ** 2
    n_out = a[..., :32:2].astype(np.float64) ** 2 + a[..., 1:32:2] ** 2
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-3)) < 1e-5
