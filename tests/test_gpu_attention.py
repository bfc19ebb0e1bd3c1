"""Decode attention (one query position per head, f16 in and out) on the GPU
vs the oracle's restatement of attention_decode_1d_masked
(kernels/moonshine_kernels.py:1579-1625) and the float64 softmax closed form,
for the decoder's two layouts: the self-attention KV cache [heads,
max_kv_len, head_dim] (nsr_attention_decode_f16, as enc_attention_decode,
src/triton_kernels.rs:900-923) and the encoder K/V [kv_len, heads, head_dim]
with a caller-chosen split count (nsr_attention_splitkv_f16, as
enc_attention_splitkv, :925-973, which the decoder calls with
min(32, kv_len) splits). The GPU sums in another order and splits the
positions, so the bar is the f16 output tolerance: |gpu - ref| <= 2e-3 *
max(|ref|, 1) (an f16 ulp at 1 is 9.8e-4)."""
import math

import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import restated as R

from ._util import RTOL_F16, assert_close, say
from .test_oracle import _attn_f64

pytestmark = pytest.mark.gpu


def _inputs(nq, nkv, hd, kv_len, layout, seed):
    g = configs.rng(seed)
    q = (g.standard_normal((nq, hd)) * 0.8).astype(np.float16)
    if layout == "cache":
        mx = kv_len + 7
        k = g.standard_normal((nkv, mx, hd)).astype(np.float16)
        v = g.standard_normal((nkv, mx, hd)).astype(np.float16)
        return q, k, v, mx * hd, hd
    k = g.standard_normal((kv_len, nkv, hd)).astype(np.float16)
    v = g.standard_normal((kv_len, nkv, hd)).astype(np.float16)
    return q, k, v, hd, nkv * hd


def _check(out, q, k, v, kv_len, nkv, scale, skh, sks, what):
    got = out.cpu().numpy().astype(np.float64)
    ref = _attn_f64(q, k, v, kv_len, nkv, scale, skh, sks)
    assert_close(got, ref, RTOL_F16, what + " vs f64")
    orc = R.attention_decode(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), kv_len, nkv, scale, skh, sks)
    assert_close(got, orc.astype(np.float16).astype(np.float64), RTOL_F16, what + " vs oracle")


@pytest.mark.parametrize("nq,nkv,hd,kv_len", [
    (10, 10, 64, 1), (10, 10, 64, 7), (10, 10, 64, 64), (10, 10, 64, 65), (10, 10, 64, 448), (10, 10, 64, 1024),
    (8, 2, 64, 300),      # grouped-query heads
    (8, 8, 52, 200),      # head_dim not a multiple of 8 (Moonshine base)
    (8, 8, 36, 129),      # head_dim 36 (Moonshine tiny)
    (4, 4, 128, 777),     # the largest head_dim
    (2, 1, 4, 50000),     # a long row over 8 waves (run-time head_dim)
    (6, 3, 96, 513),      # run-time head_dim 96
])
def test_attention_decode_self_cache_layout(dev, nq, nkv, hd, kv_len):
    say("attention_decode cache", nq, nkv, hd, kv_len)
    q, k, v, skh, sks = _inputs(nq, nkv, hd, kv_len, "cache", nq * 1000 + kv_len + hd)
    scale = 1.0 / math.sqrt(hd)
    out = abi.attention_decode(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                               kv_len, nkv, scale, stride_kv_head=skh, stride_kv_seq=sks)
    torch.cuda.synchronize()
    _check(out, q, k, v, kv_len, nkv, scale, skh, sks, "attention_decode")


@pytest.mark.parametrize("nq,nkv,hd,kv_len,n_splits", [
    (10, 10, 64, 416, 32),   # the decoder's cross-attention split
    (10, 10, 64, 20, 20),    # min(32, kv_len) for a short encoder output
    (10, 10, 64, 5, 8),      # more splits than positions: empty splits
    (10, 10, 64, 1500, 1),   # one split, 24 chunks of 64 positions
    (8, 4, 52, 333, 7),
    (8, 8, 36, 100, 3),      # head_dim 36
    (4, 2, 44, 999, 9),      # run-time head_dim 44
    (10, 10, 64, 1500, 33),  # more than 32 splits: the reduce's 16-split rounds
    (8, 4, 52, 2000, 48),
])
def test_attention_splitkv_encoder_layout(dev, nq, nkv, hd, kv_len, n_splits):
    say("attention_splitkv encoder", nq, nkv, hd, kv_len, n_splits)
    q, k, v, skh, sks = _inputs(nq, nkv, hd, kv_len, "encoder", nq * 77 + kv_len + n_splits)
    scale = 1.0 / math.sqrt(hd)
    # the reference's partial buffer size: 3 * 128 floats per (head, split)
    partial = torch.full((nq * n_splits * 384,), float("nan"), dtype=torch.float32, device="cuda")
    out = abi.attention_decode(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                               kv_len, nkv, scale, stride_kv_head=skh, stride_kv_seq=sks, n_splits=n_splits,
                               partial=partial)
    torch.cuda.synchronize()
    _check(out, q, k, v, kv_len, nkv, scale, skh, sks, "attention_splitkv")


def test_attention_decode_streams_and_repeats(dev):
    """Same call on a side stream and repeated: identical bits (deterministic order)."""
    q, k, v, skh, sks = _inputs(10, 10, 64, 500, "cache", 5)
    qt, kt, vt = (torch.from_numpy(a).cuda() for a in (q, k, v))
    a = abi.attention_decode(qt, kt, vt, 500, 10, 0.125, stride_kv_head=skh, stride_kv_seq=sks)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = abi.attention_decode(qt, kt, vt, 500, 10, 0.125, stride_kv_head=skh, stride_kv_seq=sks, stream=s)
    s.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
