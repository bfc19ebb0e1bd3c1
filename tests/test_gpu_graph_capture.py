"""The decoder-step entry points under HIP graph capture. A decode step
(RoPE of q and k with the K/V cache append, self-attention over the cache,
the MLP's fc1 GEMV with bias and GLU on the attention output; the reference
dispatches these per layer per token, src/moonshine/gpu_decoder_metal.rs:
144-168) is captured with torch.cuda.graph on the stream the wrappers use
and replayed several times, with eager work in between. The entry points
allocate nothing, synchronise nothing and issue only kernel launches, so
each replay runs the same kernels on the same buffers and must equal the
eager step bit for bit."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs

from ._util import assert_bitexact, say

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().copy()


def test_decode_step_graph_replays_match_eager(dev):
    H, Dh, L, rot, pos = 10, 64, 448, 32, 300  # Moonshine decoder (kernel_configs.py:102-104)
    K, N = H * Dh, 2560
    say("decode step under graph capture: rope+cache, attention, fc1 GEMV + GLU; 3 replays")
    g = configs.rng(11)
    f16 = lambda *s: torch.from_numpy((g.standard_normal(s) * 0.5).astype(np.float16)).cuda()
    q0, k0, v = f16(H, Dh), f16(H, Dh), f16(H, Dh)
    ck, cv = f16(H, L, Dh), f16(H, L, Dh)
    ang = np.arange(L)[:, None] * (1.0 / 10000.0 ** (np.arange(rot // 2) * 2.0 / rot))[None, :]
    table = torch.from_numpy(np.concatenate([np.cos(ang), np.sin(ang)], 1).astype(np.float32)).cuda()
    qs = torch.from_numpy(g.integers(0, 2 ** 32, size=(K, 2 * N // 4), dtype=np.uint64).astype(np.uint32)
                          .view(np.int32)).cuda()
    sc = torch.from_numpy((g.standard_normal((K // 32, 2 * N)) * 0.02).astype(np.float16)).cuda()
    w = abi.Q8T4(qs, sc, glu=True)
    bias = torch.from_numpy(g.standard_normal(2 * N).astype(np.float32)).cuda()
    q, k = torch.empty_like(q0), torch.empty_like(k0)

    def step():
        q.copy_(q0)
        k.copy_(k0)
        abi.rope_qk_cache_append(q, k, v, table, ck, cv, pos, rot)
        o = abi.attention_decode(q, ck, cv, pos + 1, H, Dh ** -0.5, stride_kv_head=L * Dh, stride_kv_seq=Dh)
        y = abi.gemv_q8_t4_bias_glu(o.view(-1), w, bias)
        return o, y

    o_e, y_e = step()
    torch.cuda.synchronize()
    ref = [_bits(q), _bits(ck[:, pos]), _bits(cv[:, pos]), _bits(o_e), _bits(y_e)]

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_g, y_g = step()
    for r in range(3):
        q.zero_()  # eager work between replays on the same buffers
        ck[:, pos].zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = [_bits(q), _bits(ck[:, pos]), _bits(cv[:, pos]), _bits(o_g), _bits(y_g)]
        for name, a, b in zip(["q", "cache k row", "cache v row", "attention out", "fc1 GLU out"], got, ref):
            assert_bitexact(a, b, f"replay {r}: {name}")


def test_noalloc_splitkv_graph_replays_match_eager(dev):
    """nsr_attention_splitkv_f16_noalloc under capture (its fixed scratch is resolved when the library loads
    on the device, before any capture here, since the fixture called nsr_init): three replays, with eager
    work between them, against the caller-buffer entry point run eagerly."""
    import math

    L = abi.lib()
    nq, nkv, hd, kv_len, splits = 10, 10, 64, 1500, 32  # Moonshine cross-attention over 30 s of encoder K/V
    say("attention_splitkv_noalloc under graph capture; 3 replays")
    g = configs.rng(12)
    q = torch.from_numpy((g.standard_normal((nq, hd)) * 0.8).astype(np.float16)).cuda()
    k = torch.from_numpy(g.standard_normal((kv_len, nkv, hd)).astype(np.float16)).cuda()
    v = torch.from_numpy(g.standard_normal((kv_len, nkv, hd)).astype(np.float16)).cuda()
    scale = 1.0 / math.sqrt(hd)
    ref_out = torch.empty((nq, hd), dtype=torch.float16, device="cuda")
    part = torch.empty(nq * splits * (hd + 2), dtype=torch.float32, device="cuda")
    abi.check(L.nsr_attention_splitkv_f16(q.data_ptr(), k.data_ptr(), v.data_ptr(), ref_out.data_ptr(),
                                          part.data_ptr(), kv_len, hd, nkv, nq, scale, hd, nkv * hd, splits,
                                          torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = _bits(ref_out)

    out = torch.empty((nq, hd), dtype=torch.float16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        abi.check(L.nsr_attention_splitkv_f16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                                      kv_len, hd, nkv, nq, scale, hd, nkv * hd, splits,
                                                      torch.cuda.current_stream().cuda_stream))
    for r in range(3):
        out.zero_()  # eager work between replays on the same buffer
        # an eager noalloc call of another shape in between leaves other partials in the shared scratch
        small = torch.empty((4, 36), dtype=torch.float16, device="cuda")
        abi.check(L.nsr_attention_splitkv_f16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), small.data_ptr(),
                                                      129, 36, 2, 4, 1.0 / 6.0, 36, nkv * hd, 5,
                                                      torch.cuda.current_stream().cuda_stream))
        graph.replay()
        torch.cuda.synchronize()
        assert_bitexact(_bits(out), ref, f"replay {r}: noalloc split-KV attention")
