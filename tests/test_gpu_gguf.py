"""GGUF loader feeding the GPU directly: tensors of a GGUF file go to HBM as
stored (nsr_gguf_upload) and are used there with no host dequantisation:
the Q8_0 embedding table by the fused gather, nn::Linear Q8_0 weights
converted on the device to the GEMV layouts (nsr_q8_0_to_gemv_q8,
nsr_q8_0_to_t4). Byte work is checked bit for bit against the oracle's
restatements; the GEMV on converted weights against the f32 accumulation
bound of the oracle."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from nspeech_amd.gguf import GgufFile
from oracle import restated as R

from . import gguf_writer as W
from ._util import RTOL_F32, assert_bitexact, assert_close, say

pytestmark = pytest.mark.gpu


def _model_file(tmp_path, vocab=1000, dim=288, inter=1152):
    """A Moonshine-decoder-like GGUF: Q8_0 embedding [vocab, dim], fc1
    [2*inter, dim] and fc2 [dim, inter] Q8_0 weights, an f32 bias."""
    g = configs.rng(70)
    emb = R.q8_0_quantize((g.standard_normal((vocab, dim)) * 0.05).astype(np.float32))
    fc1 = R.q8_0_quantize((g.standard_normal((2 * inter, dim)) * 0.05).astype(np.float32))
    fc2 = R.q8_0_quantize((g.standard_normal((dim, inter)) * 0.05).astype(np.float32))
    b1 = g.standard_normal(2 * inter).astype(np.float32)
    img = W.gguf_bytes([("general.architecture", W.STRING, "moonshine")],
                       [("decoder.embed_tokens.weight", (vocab, dim), W.GGML_Q8_0, emb.tobytes()),
                        ("decoder.layers.0.mlp.fc1.weight", (2 * inter, dim), W.GGML_Q8_0, fc1.tobytes()),
                        ("decoder.layers.0.mlp.fc1.bias", (2 * inter,), W.GGML_F32, b1.tobytes()),
                        ("decoder.layers.0.mlp.fc2.weight", (dim, inter), W.GGML_Q8_0, fc2.tobytes())])
    path = tmp_path / "model.gguf"
    path.write_bytes(img)
    return path, dict(emb=emb, fc1=fc1, fc2=fc2, b1=b1, vocab=vocab, dim=dim, inter=inter)


def test_embedding_table_from_gguf(dev, tmp_path):
    path, m = _model_file(tmp_path)
    say("gguf embedding", m["vocab"], m["dim"])
    g = configs.rng(71)
    ids = g.integers(0, m["vocab"], 500).astype(np.int64)
    with GgufFile(path) as f:
        info = f.tensor("decoder.embed_tokens.weight")
        assert info.shape == (m["vocab"], m["dim"]) and info.type == 8
        table = f.upload("decoder.embed_tokens.weight")
        torch.cuda.synchronize()
    assert_bitexact(table.cpu().numpy(), m["emb"].reshape(-1), "uploaded bytes")
    ids_t = torch.from_numpy(ids).cuda()
    out = abi.q8_0_embed_gather(table, m["vocab"], m["dim"], ids_t)
    ref, n_bad = R.q8_0_embedding(m["emb"].reshape(-1), m["vocab"], m["dim"], ids)
    assert n_bad == 0
    assert_bitexact(out.cpu().numpy(), ref, "gather (dequantised rows)")
    out_s = abi.q8_0_embed_gather(table, m["vocab"], m["dim"], ids_t, act="silu")
    ref_s, _ = R.q8_0_embedding(m["emb"].reshape(-1), m["vocab"], m["dim"], ids, act=1)
    assert_close(out_s.cpu().numpy(), ref_s, RTOL_F32, "gather + silu")


@pytest.mark.parametrize("name,glu", [("decoder.layers.0.mlp.fc1.weight", True),
                                      ("decoder.layers.0.mlp.fc2.weight", False)])
def test_linear_weight_conversions_bitexact(dev, tmp_path, name, glu):
    path, m = _model_file(tmp_path)
    with GgufFile(path) as f:
        N, K = f.tensor(name).shape
        say("gguf convert", name, N, K, glu)
        blocks = f.upload(name)
        torch.cuda.synchronize()
    qs, sc = abi.q8_0_to_gemv_q8(blocks, N, K)
    w4 = abi.Q8T4.from_q8_0(blocks, N, K, glu=glu)
    torch.cuda.synchronize()
    rq, rs = R.q8_0_to_gemv_q8(m["fc1" if glu else "fc2"], N, K)
    assert_bitexact(qs.cpu().numpy().view(np.uint32), rq, "repacked words")
    assert_bitexact(sc.cpu().numpy().view(np.uint16), rs, "repacked scales")
    tq, ts = R.q8_pack_t4(rq, rs, glu=glu)
    assert_bitexact(w4.qs.cpu().numpy().view(np.uint32), tq, "t4 words")
    assert_bitexact(w4.scales.cpu().numpy().view(np.uint16), ts, "t4 scales")


def test_mlp_fc1_glu_straight_from_gguf(dev, tmp_path):
    """fc1 + bias + GLU-SiLU on t4 tiles converted on the device from the
    file's Q8_0 weight, against the oracle on the same weight."""
    path, m = _model_file(tmp_path)
    name = "decoder.layers.0.mlp.fc1.weight"
    g = configs.rng(72)
    x16 = g.standard_normal(m["dim"]).astype(np.float16)
    with GgufFile(path) as f:
        N, K = f.tensor(name).shape
        blocks = f.upload(name)
        bias = f.upload("decoder.layers.0.mlp.fc1.bias").view(torch.float32)
        torch.cuda.synchronize()
    say("gguf fc1 glu", N, K)
    w4 = abi.Q8T4.from_q8_0(blocks, N, K, glu=True)
    out = abi.gemv_q8_t4_bias_glu(torch.from_numpy(x16).cuda(), w4, bias, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rq, rs = R.q8_0_to_gemv_q8(m["fc1"], N, K)
    ref = R.gemv_q8(x16.astype(np.float32), rq, rs, m["b1"], glu=True).astype(np.float64)
    Wd = rq.view(np.int8).reshape(K, N).astype(np.float64) * np.repeat(rs.view(np.float16).astype(np.float64), 32, 0)
    u = 2.0 ** -24
    e = 2 * (K + 2) * u / (1 - (K + 2) * u) * (np.abs(x16.astype(np.float64)) @ np.abs(Wd))
    pre = x16.astype(np.float64) @ Wd + m["b1"]
    xa, ga = pre[: N // 2], pre[N // 2:]
    sil = ga / (1 + np.exp(-ga))
    bound = 1.1 * e[N // 2:] * np.abs(xa) + np.abs(sil) * e[: N // 2] + np.abs(ref) * 2.0 ** -19 + 2.0 ** -30
    got = out.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= bound)
