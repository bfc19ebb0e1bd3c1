"""GGUF reader (libnspeech_rocm_host.so, include/nspeech_gguf.h) on the CPU:
hand-assembled images (every metadata type, versions 1-3, custom
alignment), round trips of Q8_0 / F32 / F16 tensors, and malformed files
(every truncation of a valid image, oversized lengths and counts, bad
offsets), each of which must fail with a message and never read out of
bounds. Also pins the oracle's Q8_0 quantiser and the GGUF-to-GEMV layout
restatement."""
import struct

import numpy as np
import pytest

from nspeech_amd import configs
from nspeech_amd.gguf import GgufError, GgufFile
from oracle import restated as R

from . import gguf_writer as W
from ._util import assert_bitexact


def test_hand_assembled_v3_file():
    """A v3 image written with struct.pack straight from the specification:
    one u32 and one string key, one Q8_0 tensor [2, 32] (candle shape) at
    offset 0 of a 32-aligned data section."""
    q8 = bytes(range(68))
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 2)
    kv = struct.pack("<Q", 4) + b"a.b0" + struct.pack("<II", 4, 7)
    kv += struct.pack("<Q", 4) + b"name" + struct.pack("<IQ", 8, 3) + b"xyz"
    ti = struct.pack("<Q", 1) + b"w" + struct.pack("<IQQIQ", 2, 32, 2, 8, 0)
    img = hdr + kv + ti
    img += b"\0" * ((-len(img)) % 32)
    data_off = len(img)
    img += q8
    with GgufFile(buffer=img) as g:
        assert g.version == 3 and g.alignment == 32 and g.data_offset == data_off
        assert g.metadata() == {"a.b0": 7, "name": "xyz"}
        (t,) = g.tensors()
        assert (t.name, t.type, t.shape, t.offset, t.nbytes) == ("w", 8, (2, 32), data_off, 68)
        assert g.tensor_bytes("w").tobytes() == q8


@pytest.mark.parametrize("version", [1, 2, 3])
def test_every_metadata_type_and_tensor_type_round_trip(version, tmp_path):
    g0 = configs.rng(50 + version)
    md = [("u8", W.U8, 250), ("i8", W.I8, -7), ("u16", W.U16, 65000), ("i16", W.I16, -30000),
          ("u32", W.U32, 4000000000), ("i32", W.I32, -2000000000), ("f32", W.F32, 0.5), ("bool", W.BOOL, 1),
          ("str", W.STRING, "héllo"), ("u64", W.U64, 2 ** 63 - 1), ("i64", W.I64, -2 ** 62), ("f64", W.F64, 1e-300),
          ("ints", W.ARRAY, (W.I32, [1, -2, 3])), ("strs", W.ARRAY, (W.STRING, ["a", "", "bc"])),
          ("floats", W.ARRAY, (W.F64, [0.25, -1.5])), ("empty", W.ARRAY, (W.U8, [])),
          ("nested", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.U8, [])]))]
    x = g0.standard_normal((3, 64)).astype(np.float32)
    q8 = R.q8_0_quantize(x)
    f16 = g0.standard_normal((5, 7)).astype(np.float16)
    f32 = g0.standard_normal(9).astype(np.float32)
    tensors = [("q", (3, 64), W.GGML_Q8_0, q8.tobytes()), ("h", (5, 7), W.GGML_F16, f16.tobytes()),
               ("v", (9,), W.GGML_F32, f32.tobytes()), ("z", (2, 0), W.GGML_F32, b"")]
    img = W.gguf_bytes(md, tensors, version=version, alignment=64 if version == 3 else None)
    path = tmp_path / "t.gguf"
    path.write_bytes(img)
    for g in (GgufFile(path), GgufFile(buffer=img)):
        with g:
            assert g.version == version
            assert g.alignment == (64 if version == 3 else 32)
            m = g.metadata()
            expect = {k: v for k, _, v in md}
            expect["bool"] = True
            expect["ints"], expect["strs"], expect["floats"], expect["empty"] = [1, -2, 3], ["a", "", "bc"], \
                [0.25, -1.5], []
            expect["nested"] = [None, None]
            if version == 3:
                expect["general.alignment"] = 64
            assert m == expect
            infos = {t.name: t for t in g.tensors()}
            assert [t.name for t in g.tensors()] == ["q", "h", "v", "z"]
            assert infos["q"].shape == (3, 64) and infos["q"].nbytes == 3 * 2 * 34 and infos["q"].type == 8
            assert infos["h"].shape == (5, 7) and infos["h"].nbytes == 70
            assert infos["v"].shape == (9,) and infos["v"].nbytes == 36
            assert infos["z"].nbytes == 0
            for t in infos.values():
                assert t.offset % g.alignment == 0
            assert_bitexact(g.tensor_bytes("q"), q8.reshape(-1), "q8_0 bytes")
            assert g.tensor_bytes("h").tobytes() == f16.tobytes()
            assert g.tensor_bytes("v").tobytes() == f32.tobytes()
            with pytest.raises(GgufError, match="cannot find tensor"):
                g.tensor("missing")


def _valid_image():
    x = configs.rng(60).standard_normal((2, 32)).astype(np.float32)
    return W.gguf_bytes([("k", W.STRING, "v"), ("a", W.ARRAY, (W.U16, [1, 2, 3]))],
                        [("w", (2, 32), W.GGML_Q8_0, R.q8_0_quantize(x).tobytes()),
                         ("b", (4,), W.GGML_F32, np.ones(4, np.float32).tobytes())])


def test_every_truncation_fails_cleanly():
    img = _valid_image()
    with GgufFile(buffer=img):
        pass
    for n in range(len(img)):
        with pytest.raises(GgufError):
            GgufFile(buffer=img[:n])


def _replace(img: bytes, old: bytes, new: bytes) -> bytes:
    assert img.count(old) == 1
    return img.replace(old, new)


@pytest.mark.parametrize("case", ["magic", "version", "string_len", "array_len", "n_dims", "ggml_type", "offset",
                                  "past_eof", "tensor_count", "kv_count", "bool", "alignment", "dup_tensor",
                                  "dup_key", "block", "value_type", "deep"])
def test_malformed_files_are_rejected(case):
    if case == "magic":
        img = b"GGUX" + _valid_image()[4:]
    elif case == "version":
        img = struct.pack("<II", 0x46554747, 4) + _valid_image()[8:]
    elif case == "string_len":   # key length larger than the file
        img = W.gguf_bytes([("k", W.U8, 1)])
        img = _replace(img, struct.pack("<Q", 1) + b"k", struct.pack("<Q", 2 ** 62) + b"k")
    elif case == "array_len":
        img = W.gguf_bytes([("a", W.ARRAY, (W.U32, [7]))])
        img = _replace(img, struct.pack("<IQ", W.U32, 1), struct.pack("<IQ", W.U32, 2 ** 60))
    elif case == "n_dims":
        img = W.gguf_bytes([], [("t", (1, 1, 1, 1, 1), W.GGML_F32, b"\0" * 4)])
    elif case == "ggml_type":
        img = W.gguf_bytes([], [("t", (4,), 77, b"\0" * 16)])
    elif case == "offset":       # tensor offset not aligned
        img = bytearray(W.gguf_bytes([], [("tensoroff", (4,), W.GGML_F32, b"\1" * 16)]))
        at = img.index(b"tensoroff") + 9 + 4 + 8 + 4   # name, n_dims, one dim, type -> offset field
        img[at:at + 8] = struct.pack("<Q", 4)
        img = bytes(img)
    elif case == "past_eof":
        img = W.gguf_bytes([], [("t", (4,), W.GGML_F32, b"\0" * 16)])[:-4]
    elif case == "tensor_count":
        img = _valid_image()
        img = img[:8] + struct.pack("<Q", 2 ** 40) + img[16:]
    elif case == "kv_count":
        img = _valid_image()
        img = img[:16] + struct.pack("<Q", 2 ** 40) + img[24:]
    elif case == "bool":
        img = W.gguf_bytes([("b", W.BOOL, 2)])
    elif case == "alignment":
        img = W.gguf_bytes([], [("t", (4,), W.GGML_F32, b"\0" * 16)], alignment=24)
    elif case == "dup_tensor":
        img = W.gguf_bytes([], [("t", (4,), W.GGML_F32, b"\0" * 16), ("t", (4,), W.GGML_F32, b"\0" * 16)])
    elif case == "dup_key":
        img = W.gguf_bytes([("k", W.U8, 1), ("k", W.U8, 2)])
    elif case == "block":        # Q8_0 innermost dimension not a multiple of 32
        img = W.gguf_bytes([], [("t", (2, 16), W.GGML_Q8_0, b"\0" * 34)])
    elif case == "value_type":
        img = bytearray(W.gguf_bytes([("kk", W.U8, 1)]))
        at = img.index(b"kk") + 2                        # the value type field after the key
        img[at:at + 4] = struct.pack("<I", 13)
        img = bytes(img)
    else:  # arrays nested deeper than the reader allows
        v = (W.U8, [1])
        for _ in range(5):
            v = (W.ARRAY, [v])
        img = W.gguf_bytes([("deep", W.ARRAY, v)])
    with pytest.raises(GgufError) as ei:
        GgufFile(buffer=img)
    assert str(ei.value).startswith("gguf:")


def test_missing_file_fails(tmp_path):
    with pytest.raises(GgufError, match="cannot open"):
        GgufFile(tmp_path / "nope.gguf")
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(GgufError, match="empty"):
        GgufFile(tmp_path / "empty.gguf")


# ------------------------------------------------ Q8_0 quantiser, layouts ---

def test_q8_0_quantize_follows_the_published_rounding():
    """Per 32 values: d = max|x|/127 stored as f16, q = round-half-away(x/d);
    the max-magnitude value maps to +-127, zero blocks give d = 0 and q = 0,
    exact multiples of d round-trip, and every dequantised value lies within
    d/2 (plus the f16 rounding of d times |q|) of the input."""
    g = configs.rng(61)
    x = (g.standard_normal((8, 128)) * 3).astype(np.float32)
    x[1, :32] = 0.0
    x[2, :32] = np.arange(32, dtype=np.float32) - 16.0          # multiples of d = 16/127
    x[3, 5] = 2.5 * np.max(np.abs(x[3, :32]))                   # a dominant value
    b = R.q8_0_quantize(x).reshape(8, 4, 34)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    q = b[:, :, 2:].view(np.int8).astype(np.float64)
    xb = x.reshape(8, 4, 32).astype(np.float64)
    assert np.all(d[1, 0] == 0) and np.all(q[1, 0] == 0)
    amax_idx = np.argmax(np.abs(xb), axis=2)
    qmax = np.abs(np.take_along_axis(q, amax_idx[:, :, None], 2))[:, :, 0]
    assert np.all(qmax[d > 0] == 127)
    d32 = (np.max(np.abs(x.reshape(8, 4, 32)), axis=2) / np.float32(127)).astype(np.float64)
    err = np.abs(q * d[:, :, None] - xb)
    assert np.all(err <= d32[:, :, None] / 2 * (1 + 1e-6) + np.abs(q) * np.abs(d - d32)[:, :, None] + 1e-30)
    deq = R.q8_0_dequantize(b.reshape(-1), 8, 128)
    assert_bitexact(np.asarray(deq, np.float32).reshape(8, 128),
                    (q * d[:, :, None]).astype(np.float32).reshape(8, 128), "oracle dequant of the quantiser's blocks")
    # a half-way case rounds away from zero: x/d = 2.5 exactly when max|x| = 127*d
    y = np.zeros((1, 32), np.float32)
    y[0, 0], y[0, 1], y[0, 2] = 127.0, 2.5, -2.5
    qy = R.q8_0_quantize(y).reshape(34)[2:].view(np.int8)
    assert (qy[0], qy[1], qy[2]) == (127, 3, -3)


def test_q8_0_to_gemv_q8_is_the_transpose_of_the_dequantised_weight():
    """The restated conversion moves bytes only: dequantising its output in
    the repacked layout gives exactly the transpose of the GGUF weight's
    dequantisation (both decoded here independently of the restatement)."""
    g = configs.rng(62)
    N, K = 48, 96
    blocks = R.q8_0_quantize(g.standard_normal((N, K)).astype(np.float32))
    qs, sc = R.q8_0_to_gemv_q8(blocks, N, K)
    b = blocks.reshape(N, K // 32, 34)
    Wg = b[:, :, 2:].view(np.int8).reshape(N, K).astype(np.float32) * np.repeat(
        b[:, :, 0:2].copy().view(np.float16).reshape(N, K // 32).astype(np.float32), 32, axis=1)
    Wr = qs.view(np.int8).reshape(K, N).astype(np.float32) * np.repeat(
        sc.view(np.float16).astype(np.float32), 32, axis=0)
    assert_bitexact(Wr, np.ascontiguousarray(Wg.T), "repacked dequant == transposed GGUF dequant")


def test_reader_under_address_sanitizer(tmp_path):
    """The same truncations and malformed images, parsed by the reader built
    with AddressSanitizer + UBSan (tests/host/test_gguf_asan.cpp): every
    read stays inside the image (an out-of-bounds access aborts the run)."""
    import subprocess
    from pathlib import Path

    exe = Path(__file__).resolve().parent / "host" / "_build" / "test_gguf_asan"
    if not exe.exists():
        pytest.fail(f"{exe} is not built: run `python -m nspeech_amd.build`")
    img = _valid_image()
    files = []
    for n in range(len(img) + 1):
        f = tmp_path / f"cut{n:04d}.gguf"
        f.write_bytes(img[:n])
        files.append(f)
    big = bytearray(img)
    big[8:16] = struct.pack("<Q", 2 ** 40)
    (tmp_path / "count.gguf").write_bytes(bytes(big))
    files.append(tmp_path / "count.gguf")
    out = subprocess.run([str(exe), *map(str, files)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = out.stdout.splitlines()
    assert len(lines) == len(files)
    assert lines[len(img)].startswith("ok ")                       # the whole image parses
    assert all(ln.startswith("err ") for k, ln in enumerate(lines) if k != len(img))
