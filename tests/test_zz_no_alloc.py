"""The entry point that allocates nothing, nsr_attention_splitkv_f16_noalloc,
against nsr_attention_splitkv_f16 with a caller-allocated partial buffer:
the same kernels over the same inputs, so the outputs must agree bit for bit.
Two calls in a row on the library's fixed scratch, the second smaller than
the first (the scratch keeps the first call's partials, which the second must
not read), then a call needing more than the fixed scratch, which must be
rejected before any launch. Called through the C ABI (ctypes)."""
import math

import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs

from ._util import assert_bitexact, say

pytestmark = pytest.mark.gpu


def _inputs(nq, nkv, hd, kv_len, seed):
    """encoder K/V layout [kv_len, heads, head_dim] (the cross-attention the
    split form serves), f16"""
    g = configs.rng(seed)
    q = torch.from_numpy((g.standard_normal((nq, hd)) * 0.8).astype(np.float16)).cuda()
    k = torch.from_numpy(g.standard_normal((kv_len, nkv, hd)).astype(np.float16)).cuda()
    v = torch.from_numpy(g.standard_normal((kv_len, nkv, hd)).astype(np.float16)).cuda()
    return q, k, v


def _call(noalloc, q, k, v, kv_len, nq, nkv, hd, splits):
    L = abi.lib()
    out = torch.empty((nq, hd), dtype=torch.float16, device="cuda")
    scale = 1.0 / math.sqrt(hd)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = L.nsr_attention_splitkv_f16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), kv_len, hd,
                                                 nkv, nq, scale, hd, nkv * hd, splits, stream)
    else:
        part = torch.empty(nq * splits * (hd + 2), dtype=torch.float32, device="cuda")
        st = L.nsr_attention_splitkv_f16(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), part.data_ptr(),
                                         kv_len, hd, nkv, nq, scale, hd, nkv * hd, splits, stream)
    abi.check(st)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_caller_buffer_two_calls(dev):
    # first call: Moonshine cross-attention over 30 s of encoder K/V, 32 splits (10 heads x 64)
    # second call: smaller in every dimension, so the scratch still holds partials of the first
    for nq, nkv, hd, kv_len, splits, seed in ((10, 10, 64, 1500, 32, 71), (4, 2, 36, 129, 5, 72)):
        say("attention_splitkv_noalloc", nq, nkv, hd, kv_len, splits)
        q, k, v = _inputs(nq, nkv, hd, kv_len, seed)
        ref = _call(False, q, k, v, kv_len, nq, nkv, hd, splits)
        got = _call(True, q, k, v, kv_len, nq, nkv, hd, splits)
        assert_bitexact(got, ref, f"noalloc vs caller buffer {nq}x{hd} kv {kv_len} splits {splits}")


def test_noalloc_rejects_more_than_the_scratch(dev):
    # 64 heads x 32 splits x (128 + 2) floats = 266240 > 262144
    nq, nkv, hd, kv_len, splits = 64, 64, 128, 64, 32
    say("attention_splitkv_noalloc over the scratch limit")
    q, k, v = _inputs(nq, nkv, hd, kv_len, 73)
    with pytest.raises(abi.NsrError) as ei:
        _call(True, q, k, v, kv_len, nq, nkv, hd, splits)
    assert ei.value.status == abi.NSR_ERR_UNSUPPORTED
    assert "fixed scratch" in str(ei.value)
    # at the limit it runs: 64 heads x 31 splits x 130 = 257920 floats
    ref = _call(False, q, k, v, kv_len, nq, nkv, hd, 31)
    got = _call(True, q, k, v, kv_len, nq, nkv, hd, 31)
    assert_bitexact(got, ref, "noalloc at 257920 floats")
