"""GGUF Q8_0 embedding gather-dequant on the GPU vs the oracle's
dequantize-whole-table + index_select (QEmbedding::forward,
src/parakeet/quantized_layers.rs:65-71). Bit-exact without activation;
SiLU epilogue within 1e-5."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_F32, assert_bitexact, assert_close, dev_tensor, host, say

pytestmark = pytest.mark.gpu


def _run(blocks, vocab, d, ids, act="none", ids_dtype=torch.int32, err=None):
    b = dev_tensor(blocks)
    i = torch.from_numpy(np.asarray(ids).astype(np.int64)).to("cuda:0").to(ids_dtype)
    out = abi.q8_0_embed_gather(b, vocab, d, i, act=act, err_flag=err)
    torch.cuda.synchronize()
    return host(out)


def test_config3_full_bitexact(dev):
    c = configs.c3()
    say("q8_0 config3 vocab=32768 d=416 n_ids=4096 act=none/silu")
    ids = c["ids"].astype(np.int64)
    ref0, bad = R.q8_0_embedding(c["blocks"], c["vocab"], c["d"], ids, act=0)
    assert bad == 0
    assert_bitexact(_run(c["blocks"], c["vocab"], c["d"], ids), ref0, "q8 config3 gather")
    ref1, _ = R.q8_0_embedding(c["blocks"], c["vocab"], c["d"], ids, act=1)
    got1 = _run(c["blocks"], c["vocab"], c["d"], ids, act="silu")
    assert_close(got1, ref1, RTOL_F32, "q8 config3 gather+silu vs oracle")
    dense = CF.q8_0_decode(c["blocks"], c["vocab"], c["d"])[ids]
    assert_close(got1, CF.silu(dense), RTOL_F32, "q8 config3 gather+silu vs f64")


@pytest.mark.parametrize("vocab,d", [(1, 32), (7, 32), (37, 64), (101, 416), (64, 4096)])
@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
def test_every_row_brute_force(dev, vocab, d, ids_dtype):
    g = configs.rng(vocab * 1000 + d)
    blocks = configs.make_q8_0_table(g, vocab, d)
    ids = np.concatenate([np.arange(vocab), np.arange(vocab)[::-1], g.integers(0, vocab, 13)])
    say("q8_0 brute force", vocab, d, ids_dtype)
    got = _run(blocks, vocab, d, ids, ids_dtype=ids_dtype)
    assert_bitexact(got, CF.q8_0_decode(blocks, vocab, d).astype(np.float32)[ids], "all rows")


def test_golden_fixtures(dev):
    from .golden import make_golden

    for name, case in make_golden.load_all().items():
        if not name.startswith("q8_"):
            continue
        say("q8_0 golden", name)
        vocab, d = int(case["vocab"]), int(case["d"])
        assert_bitexact(_run(case["blocks"], vocab, d, case["ids"]), case["out_none"], name)
        assert_close(_run(case["blocks"], vocab, d, case["ids"], act="silu"), case["out_silu"], RTOL_F32, name)


def test_out_of_range_ids_zero_row_and_flag(dev):
    g = configs.rng(5)
    vocab, d = 10, 64
    blocks = configs.make_q8_0_table(g, vocab, d)
    say("q8_0 out-of-range ids")
    err = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    got = _run(blocks, vocab, d, [3, 10, -1, 9], ids_dtype=torch.int64, err=err)
    assert int(err.item()) == 1
    dense = CF.q8_0_decode(blocks, vocab, d).astype(np.float32)
    assert_bitexact(got[[0, 3]], dense[[3, 9]], "valid rows")
    assert not got[1:3].any()
    err.zero_()
    _run(blocks, vocab, d, [0, 9], err=err)
    assert int(err.item()) == 0
    # u32 ids above vocab (no sign) are out of range too
    got = _run(blocks, vocab, d, [2**31 + 5], ids_dtype=torch.int32, err=err)
    assert int(err.item()) == 1 and not got.any()


def test_misaligned_output_is_rejected(dev):
    g = configs.rng(6)
    blocks = dev_tensor(configs.make_q8_0_table(g, 4, 32))
    ids = torch.zeros(2, dtype=torch.int32, device="cuda:0")
    out = torch.empty(2 * 32 + 1, dtype=torch.float32, device="cuda:0")[1:].view(2, 32)
    with pytest.raises(abi.NsrError):
        abi.q8_0_embed_gather(blocks, 4, 32, ids, out=out)
