"""Decode-step RoPE + KV-cache append on the GPU (one launch) vs the oracle's
restatement of rope_qk_cache_fused + kv_cache_append
(kernels/moonshine_kernels.py:1372-1454, :865-883; dispatched together by
src/moonshine/gpu_decoder_metal.rs:144-156). f16 results are bit-exact with
the oracle (each value is the f16 rounding of the same f32 expression); the
f32 variant is bit-exact with numpy's IEEE f32 arithmetic."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import restated as R

from ._util import assert_bitexact, say

pytestmark = pytest.mark.gpu


def _f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16).cuda()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("Hq,Hk,Dh,rot,L,pos,with_v", [
    (10, 10, 64, 32, 448, 0, True),      # Moonshine decoder (kernel_configs.py:102-104), first token
    (10, 10, 64, 32, 448, 137, True),
    (10, 10, 64, 32, 448, 447, True),    # last cache row
    (10, 10, 64, 32, 448, 200, False),   # k only: exactly enc_rope_qk_cache_fused
    (8, 2, 64, 32, 100, 63, True),       # grouped KV heads
    (4, 4, 128, 128, 64, 5, True),       # full rotation, no pass-through dims
    (3, 3, 16, 0, 8, 7, True),           # no rotation: plain K/V append
    (1, 1, 6, 2, 3, 2, True),            # tiny, odd pair counts
])
def test_rope_qk_cache_f16_bitexact(dev, Hq, Hk, Dh, rot, L, pos, with_v):
    g = configs.rng(Hq * 7 + Dh + pos)
    q = g.standard_normal((Hq, Dh)).astype(np.float16).view(np.uint16)
    k = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16)
    v = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16) if with_v else None
    ck0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16)
    cv0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16) if with_v else None
    tab = R.rope_table(max(L, 1), rot, 1e4) if rot else np.zeros((1, 2), np.float32)
    say("rope_qk_cache f16", Hq, Hk, Dh, rot, L, pos, with_v)
    qd, kd, ckd = _f16(q), _f16(k), _f16(ck0)
    vd = _f16(v) if with_v else None
    cvd = _f16(cv0) if with_v else None
    tabd = torch.from_numpy(tab).cuda()
    abi.rope_qk_cache_append(qd, kd, vd, tabd, ckd, cvd, pos, rot)
    torch.cuda.synchronize()
    qr, kr, ckr, cvr = R.rope_qk_cache_f16(q, k, v, tab, pos, rot, ck0, cv0)
    assert_bitexact(_bits(qd), qr, "q")
    assert_bitexact(_bits(kd), kr, "k")
    assert_bitexact(_bits(ckd), ckr, "cache_k")
    if with_v:
        assert_bitexact(_bits(cvd), cvr, "cache_v")


def test_rope_qk_cache_f32(dev):
    g = configs.rng(41)
    Hq, Hk, Dh, rot, L, pos = 6, 3, 64, 32, 20, 11
    q = g.standard_normal((Hq, Dh)).astype(np.float32)
    k = g.standard_normal((Hk, Dh)).astype(np.float32)
    v = g.standard_normal((Hk, Dh)).astype(np.float32)
    ck = np.zeros((Hk, L, Dh), np.float32)
    cv = np.zeros((Hk, L, Dh), np.float32)
    tab = R.rope_table(L, rot, 1e4)
    say("rope_qk_cache f32")
    qd, kd, vd, ckd, cvd = (torch.from_numpy(a.copy()).cuda() for a in (q, k, v, ck, cv))
    abi.rope_qk_cache_append(qd, kd, vd, torch.from_numpy(tab).cuda(), ckd, cvd, pos, rot)
    torch.cuda.synchronize()
    c, s = tab[pos, :rot // 2], tab[pos, rot // 2:]
    for x, xd in ((q, qd), (k, kd)):
        e = x.copy()
        e[:, 0:rot:2] = x[:, 0:rot:2] * c - x[:, 1:rot:2] * s   # numpy f32: separately rounded products
        e[:, 1:rot:2] = x[:, 1:rot:2] * c + x[:, 0:rot:2] * s
        assert_bitexact(xd.cpu().numpy(), e, "rotated")
        if x is k:
            ek = e
    assert_bitexact(ckd.cpu().numpy()[:, pos], ek, "cache_k")
    assert_bitexact(cvd.cpu().numpy()[:, pos], v, "cache_v")
    assert not np.any(ckd.cpu().numpy()[:, :pos]) and not np.any(cvd.cpu().numpy()[:, pos + 1:])


def test_kv_cache_append_alone(dev):
    g = configs.rng(42)
    Hk, Dh, L = 10, 64, 33
    v = g.standard_normal((Hk, Dh)).astype(np.float16).view(np.uint16)
    c0 = g.standard_normal((Hk, L, Dh)).astype(np.float16).view(np.uint16)
    say("kv_cache_append")
    cd = _f16(c0)
    for pos in (0, 17, 32):
        abi.kv_cache_append(_f16(v), cd, pos)
    torch.cuda.synchronize()
    exp = c0.copy()
    exp[:, [0, 17, 32]] = v[:, None, :]
    assert_bitexact(_bits(cd), exp, "cache after three appends")
