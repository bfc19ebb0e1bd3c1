"""Fused AdaIN1d + Snake with f16 activations (nsr_adain_snake_f16, the
reference's KokoroGpuBackend::adain_snake over the Triton
adain_snake_fused / adain_snake_looped kernels,
kernels/kokoro_kernels.py:222-331) on the GPU vs the oracle's f32
restatement of adain + snake (src/kokoro/decoder.rs:1416-1428, :1471-1476)
applied to the f16 input, and the float64 closed form. The output is f16, so
the bar is the f16 tolerance |gpu - ref| <= 2e-3 * max(|ref|, 1) (an f16 ulp
is at most 9.8e-4 of the value).

Rows of odd length start at every offset within a 16-byte chunk, which
exercises the partial first and last chunks; lengths cover every kernel
variant up to the 131072-element limit."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi, configs
from oracle import closed_form as CF
from oracle import restated as R

from ._util import RTOL_F16, assert_close, say

pytestmark = pytest.mark.gpu


def _inputs(B, C, T, seed, scale=1.3, shift=0.2):
    g = configs.rng(seed)
    x = (g.standard_normal((B, C, T)) * scale + shift).astype(np.float16)
    gamma = (0.1 * g.standard_normal((B, C))).astype(np.float32)
    beta = (0.1 * g.standard_normal(C)).astype(np.float32)
    alpha = g.uniform(0.5, 1.5, C).astype(np.float32)
    return x, gamma, beta, alpha


def _check(got, x, gamma, beta, alpha, what, oracle=True):
    """Within the f16 bar of float64 and (oracle=True) of the oracle. The oracle sums a row in order in f32 (the
    reference's order), which drifts from the row's exact statistics on long rows with |mean| >> std; there the
    float64 form is the bar."""
    x32 = x.astype(np.float32)
    if oracle:
        orc = R.adain_snake(x32, gamma, beta, alpha).astype(np.float16).astype(np.float64)
        assert_close(got.astype(np.float64), orc, RTOL_F16, what + " vs oracle")
    assert_close(got.astype(np.float64), CF.adain_snake(x32, gamma, beta, alpha), RTOL_F16, what + " vs f64")


def _run(x, gamma, beta, alpha, pdt=torch.float32):
    p = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(pdt).cuda()  # noqa: E731
    out = abi.adain_snake(torch.from_numpy(x).cuda(), p(gamma), p(beta), p(alpha))
    assert out.dtype == torch.float16
    return out.cpu().numpy()


@pytest.mark.parametrize("B,C,T", [(1, 3, 1), (1, 2, 2), (2, 3, 7), (1, 9, 8), (1, 9, 9), (1, 8, 15), (1, 8, 17),
                                   (1, 4, 100), (1, 3, 1023), (1, 3, 2055), (2, 3, 4097), (1, 9, 8191),
                                   (1, 2, 16385), (1, 3, 20481), (1, 2, 49153), (1, 2, 98305), (1, 3, 115200),
                                   (1, 2, 131071), (1, 2, 131072)])
def test_shapes(B, C, T):
    say("adain+snake f16", B, C, T)
    x, gamma, beta, alpha = _inputs(B, C, T, B * 13 + C * 7 + T)
    _check(_run(x, gamma, beta, alpha), x, gamma, beta, alpha, f"{B}x{C}x{T}")


@pytest.mark.parametrize("T", [4800, 4801, 115200])
def test_rows_across_the_statistics_switch(T):
    """The aligned f16 kernels (T = 4800; the persistent long-row kernel at T = 115200) take one-pass
    statistics and the centred two-pass form when 4 mean^2 > var: rows with |mean| / std from 0 to 300 on both
    sides of 1/2, within the f16 bar of the oracle and of float64 (the unaligned kernel, T = 4801, takes the
    same rows)."""
    g = configs.rng(77 + T)
    ratios = np.array([0.0, 0.1, 0.45, 0.49, 0.51, 0.55, 1.0, 3.0, 30.0, 300.0])
    C = len(ratios)
    std = np.array([1.0, 0.05, 20.0, 1.0, 1.0, 2.0, 1.0, 0.5, 1.0, 0.1])
    mean = ratios * std * np.where(np.arange(C) % 2, -1.0, 1.0)
    x = (mean[:, None] + std[:, None] * g.standard_normal((C, T))).astype(np.float16)[None]
    gamma = (0.1 * g.standard_normal((1, C))).astype(np.float32)
    beta = (0.1 * g.standard_normal(C)).astype(np.float32)
    alpha = g.uniform(0.5, 1.5, C).astype(np.float32)
    say("adain+snake f16 rows across the statistics switch", T)
    _check(_run(x, gamma, beta, alpha), x, gamma, beta, alpha, f"T={T}", oracle=T < 100000)


def test_kokoro_known_answer_f16_params():
    """The reference's Kokoro self-test inputs (src/kokoro/gpu_decoder.rs:84-87),
    with x rounded to f16 as the f16 path holds it."""
    for C_, T_ in ((4, 100), (128, 1127)):
        k = configs.kokoro_kat(C_, T_)
        x = k["x"].reshape(1, C_, T_).astype(np.float16)
        say("adain+snake f16 kokoro KAT", C_, T_)
        got = _run(x, k["gamma"], k["beta"], k["alpha"], pdt=torch.float16)
        g32, b32, a32 = (k[n].astype(np.float32) for n in ("gamma", "beta", "alpha"))
        _check(got, x, g32, b32, a32, f"KAT {C_}x{T_}")


def test_ill_conditioned_rows_and_special_alpha():
    x, _, _, _ = _inputs(1, 4, 3001, 31, scale=0.5, shift=200.0)  # |mean| >> std
    x[0, 3] = np.float16(1.25)  # constant row: var = 0
    gamma = np.array([0.1, -0.2, 0.0, 0.3], np.float32)
    beta = np.array([0.0, 0.1, -0.1, 0.2], np.float32)
    alpha = np.array([1.0, 0.0, -0.7, 1e-4], np.float32)
    say("adain+snake f16 ill-conditioned rows")
    _check(_run(x, gamma, beta, alpha), x, gamma, beta, alpha, "ill-conditioned")


@pytest.mark.parametrize("off", [1, 3, 8])
def test_views_at_any_offset_and_no_stray_writes(off):
    """x and out are views starting `off` halves into their buffers (same
    offset within 16 bytes); nothing outside out's elements is written."""
    B, C, T = 2, 3, 517
    x, gamma, beta, alpha = _inputs(B, C, T, 40 + off)
    n = B * C * T
    xb = torch.zeros(n + 16, dtype=torch.float16, device="cuda")
    xb[off:off + n] = torch.from_numpy(x.ravel()).cuda()
    ob = torch.full((n + 16,), 7.0, dtype=torch.float16, device="cuda")
    gd, bd, ad = (torch.from_numpy(np.asarray(a, np.float32)).cuda() for a in (gamma, beta, alpha))
    say("adain+snake f16 views at offset", off)
    abi.check(abi.lib().nsr_adain_snake_f16(xb.data_ptr() + 2 * off, gd.data_ptr(), bd.data_ptr(), ad.data_ptr(),
                                            abi.NSR_F32, C, 0, ob.data_ptr() + 2 * off, B, C, T, 1e-5,
                                            torch.cuda.current_stream().cuda_stream))
    got = ob.cpu().numpy()
    assert np.all(got[:off] == 7.0) and np.all(got[off + n:] == 7.0), "wrote outside out"
    _check(got[off:off + n].reshape(B, C, T), x, gamma, beta, alpha, f"offset {off}")


def test_matches_f32_path_on_f16_values():
    """The f16 and f32 entry points agree on the same (f16-representable)
    input up to the final f16 rounding."""
    x, gamma, beta, alpha = _inputs(2, 4, 3000, 55)
    got16 = _run(x, gamma, beta, alpha).astype(np.float64)
    p = lambda a: torch.from_numpy(np.asarray(a, np.float32)).cuda()  # noqa: E731
    out32 = abi.adain_snake(torch.from_numpy(x.astype(np.float32)).cuda(), p(gamma), p(beta), p(alpha))
    ref = out32.cpu().numpy().astype(np.float16).astype(np.float64)
    assert_close(got16, ref, RTOL_F16, "f16 path vs f32 path")


@pytest.mark.parametrize("B,C,T", [(1, 5, 77832), (2, 160, 81920), (1, 300, 96000), (1, 3, 131064)])
def test_long_aligned_rows_persistent_kernel(B, C, T):
    """Aligned f16 rows of 20-32 slots take the persistent row kernel (10 LDS slots + VGPR slots): the
    smallest row of its first bucket (one element past 19 slots), more rows than CUs (each workgroup refills
    its slots with its next row), and the last bucket."""
    say("adain+snake f16 long aligned rows", B, C, T)
    x, gamma, beta, alpha = _inputs(B, C, T, B * 17 + C * 5 + T)
    _check(_run(x, gamma, beta, alpha), x, gamma, beta, alpha, f"{B}x{C}x{T}")


def test_long_aligned_rows_ill_conditioned_and_special_alpha():
    """The persistent long-row kernel on |mean| >> std rows (the centred path), a constant row and
    alpha = 0, negative and tiny."""
    x, _, _, _ = _inputs(1, 4, 115200, 33, scale=0.5, shift=200.0)
    x[0, 3] = np.float16(1.25)
    gamma = np.array([0.1, -0.2, 0.0, 0.3], np.float32)
    beta = np.array([0.0, 0.1, -0.1, 0.2], np.float32)
    alpha = np.array([1.0, 0.0, -0.7, 1e-4], np.float32)
    say("adain+snake f16 long rows ill-conditioned")
    _check(_run(x, gamma, beta, alpha), x, gamma, beta, alpha, "long ill-conditioned", oracle=False)
