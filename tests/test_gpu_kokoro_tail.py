"""The Kokoro generator's tail on the GPU: the multi-receptive-field average
of the three resblocks ((r0 + r1) + r2) * f32(1/3) with the optional leaky
ReLU(0.01) of the last stage (src/kokoro/decoder.rs:540-575 over
kernels/kokoro_kernels.py:942-969 and :109-122), the plain scale and leaky
ReLU, and the inverse STFT istft_fused (kernels/kokoro_kernels.py:1097-1183;
CPU istft src/kokoro/decoder.rs:1545-1632).

The element-wise kernels repeat the reference's f32 operation sequence, so
they are bit-exact against the oracle (vector and scalar-tail paths). The
iSTFT computes the same transform in another f32 order (symmetric iDFT,
exact basis angles, polynomial cos / sin of the phase), so the bar is the
f32 tolerance |gpu - ref| <= 1e-5 * max(|ref|, 1) against both the oracle
and the float64 irfft overlap-add, times the gain with which the window
normalisation amplifies rounding (1 at the reference's 75% overlap)."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import restated as R

from ._util import RTOL_F16, RTOL_F32, assert_bitexact, assert_close, say
from .test_oracle import _istft_f64

pytestmark = pytest.mark.gpu


def _vals(n, seed):
    g = configs.rng(seed)
    x = g.standard_normal(n).astype(np.float32) * 3
    if n >= 8:
        x[:8] = [0.0, -0.0, 1e-38, -1e-38, 3e38, -3e38, 1.0, -1.0]
    return x


@pytest.mark.parametrize("n", [1, 3, 4, 7, 1027, 65536 + 5, 128 * 2401])
@pytest.mark.parametrize("lrelu", [None, 0.01])
@pytest.mark.parametrize("offset", [0, 1])
def test_resblock_average(n, lrelu, offset):
    say("resblock_average", n, lrelu, offset)
    r = [_vals(n + offset, 10 + i + n) for i in range(3)]
    dev = [torch.from_numpy(a).cuda()[offset:] for a in r]  # offset 1: 4-byte aligned, scalar kernel
    out = torch.full((n + offset,), np.nan, dtype=torch.float32, device="cuda")[offset:]
    abi.resblock_average_f32(*dev, leaky_slope=lrelu, out=out)
    ref = R.resblock_average(*(a[offset:] for a in r), lrelu_slope=lrelu)
    assert_bitexact(out.cpu().numpy(), ref, f"resblock_average n={n}")


@pytest.mark.parametrize("n", [5, 4096, 300001])
def test_scale_and_leaky_relu(n):
    say("scale/leaky_relu", n)
    x = _vals(n, n)
    xd = torch.from_numpy(x).cuda()
    assert_bitexact(abi.scale_f32(xd, 0.3333333333333333).cpu().numpy(),
                    R.combine(x, scale=np.float32(0.3333333333333333)), "scale")
    assert_bitexact(abi.leaky_relu_f32(xd, 0.1).cpu().numpy(), R.combine(x, lrelu_slope=0.1), "leaky_relu")
    # in place
    abi.leaky_relu_f32(xd, 0.01, out=xd)
    assert_bitexact(xd.cpu().numpy(), R.combine(x, lrelu_slope=0.01), "leaky_relu in place")


def test_elementwise_empty():
    # zero elements at a valid address (the entry points reject null pointers whatever n is; torch reports
    # address 0 for an empty tensor, so the library is called directly)
    L = abi.lib()
    buf = torch.full((4,), 5.0, dtype=torch.float32, device="cuda")
    p = buf.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    abi.check(L.nsr_resblock_average_f32(p, p, p, p, 0, 1, 0.01, s))
    abi.check(L.nsr_scale_f32(p, p, 0, 2.0, s))
    abi.check(L.nsr_leaky_relu_f32(p, p, 0, 0.01, s))
    assert torch.all(buf.cpu() == 5.0)


def _cola_gain(n_fft, hop):
    """How much the window normalisation amplifies f32 rounding of the
    frames, relative to the 75%-overlap Hann case: max over positions of
    (sum_f w) / (sum_f w^2), divided by its value 2 / (3/2) there. It is 1
    for hop = n_fft / 4 and grows to 0.75 / w[1] (about 31 for n_fft 20)
    with no overlap, where samples near a frame's edge are divided by w^2."""
    w = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(n_fft) / n_fft)
    s1 = np.zeros(hop)
    s2 = np.zeros(hop)
    for n in range(n_fft):
        s1[n % hop] += w[n]
        s2[n % hop] += w[n] ** 2
    ok = s2 > 1e-8
    return max(1.0, float(np.max(s1[ok] / s2[ok])) / (4.0 / 3.0))


ISTFT_CASES = [
    (20, 5, 2), (20, 5, 3), (20, 5, 64), (20, 5, 255), (20, 5, 256), (20, 5, 257), (20, 5, 509),
    (20, 5, 510), (20, 5, 1000), (20, 5, 24001),  # 24001 frames: 5 s of Kokoro audio at 24 kHz
    (20, 10, 300), (20, 20, 40), (16, 4, 700), (16, 16, 9), (32, 8, 600), (32, 4, 300),
]


@pytest.mark.parametrize("n_fft,hop,n_frames", ISTFT_CASES)
def test_istft(n_fft, hop, n_frames):
    say("istft", n_fft, hop, n_frames)
    g = configs.rng(n_fft + 7 * n_frames + hop)
    x = (g.standard_normal((2 * (n_fft // 2 + 1), n_frames)) * 0.7).astype(np.float32)
    out = abi.istft_f32(torch.from_numpy(x).cuda(), n_fft=n_fft, hop=hop)
    got = out.cpu().numpy()
    assert got.shape == ((n_frames - 1) * hop,)
    tol = RTOL_F32 * _cola_gain(n_fft, hop)
    assert_close(got, R.istft(x, n_fft, hop), tol, "istft vs oracle")
    assert_close(got, _istft_f64(x, n_fft, hop), tol, "istft vs f64")


def test_istft_short_out_len_and_single_frame():
    x = (configs.rng(3).standard_normal((22, 300)) * 0.7).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    full = R.istft(x, 20, 5)
    guard = torch.full((1000,), 7.0, dtype=torch.float32, device="cuda")
    abi.istft_f32(xd, out_len=777, out=guard)
    got = guard.cpu().numpy()
    assert_close(got[:777], full[:777], RTOL_F32, "istft prefix")
    assert np.all(got[777:] == 7.0), "wrote past out_len"
    # one frame: no samples survive the trim, nothing is written
    one = xd[:, :1].contiguous()
    abi.check(abi.lib().nsr_istft_f32(one.data_ptr(), guard.data_ptr(), 1, 0, 20, 5,
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.all(guard.cpu().numpy()[777:] == 7.0)


@pytest.mark.parametrize("dt", ["f32", "f16"])
@pytest.mark.parametrize("B,C,T", [(1, 1, 1), (1, 3, 5), (2, 4, 1023), (1, 5, 1025), (1, 2, 4800), (2, 3, 11281)])
def test_snake(dt, B, C, T):
    """nsr_snake vs the oracle's snake_activation_tensor restatement and the
    float64 formula (f32 bar for f32, f16 bar for f16 storage)."""
    say("snake", dt, B, C, T)
    g = configs.rng(B * 100 + C * 10 + T)
    x = (g.standard_normal((B, C, T)) * 3).astype(np.float32)
    alpha = g.uniform(0.3, 1.6, C).astype(np.float32)
    if C >= 3:
        alpha[2] = 0.0  # the formula's limit: out = x
    if dt == "f16":
        x = x.astype(np.float16).astype(np.float32)
    xd = torch.from_numpy(x).cuda().to(torch.float32 if dt == "f32" else torch.float16)
    out = abi.snake(xd, torch.from_numpy(alpha).cuda()).float().cpu().numpy()
    orc = R.snake(x, alpha)
    a64 = alpha.astype(np.float64)[None, :, None]
    f64 = x + np.sin(a64 * x) ** 2 / (a64 + 1e-9)
    if dt == "f32":
        assert_close(out, orc, RTOL_F32, "snake vs oracle")
        assert_close(out, f64, RTOL_F32, "snake vs f64")
    else:
        assert_close(out, orc.astype(np.float16).astype(np.float32), RTOL_F16, "snake f16 vs oracle")
        assert_close(out, f64, RTOL_F16, "snake f16 vs f64")
    if C >= 3:
        assert np.array_equal(out[:, 2], x[:, 2]), "alpha = 0 must leave x unchanged"


def test_snake_f16_alpha_and_in_place():
    g = configs.rng(77)
    x = (g.standard_normal((4, 999)) * 2).astype(np.float32)
    alpha = g.uniform(0.5, 1.5, 4).astype(np.float16)
    xd = torch.from_numpy(x).cuda()
    abi.snake(xd, torch.from_numpy(alpha).cuda(), out=xd)
    assert_close(xd.cpu().numpy(), R.snake(x, alpha.astype(np.float32)), RTOL_F32, "snake in place, f16 alpha")
