"""Shared checks for the parity tests."""
from __future__ import annotations

import numpy as np

# Tolerances of the parity bar (stated once, used everywhere):
#   f32 norms, rotary, activations:  |gpu - ref| <= 1e-5 * max(|ref|, 1)
#   bf16 outputs:                    |gpu - ref| <= 1e-2 * max(|ref|, 1)
#   f16 outputs:                     |gpu - ref| <= 2e-3 * max(|ref|, 1)  (f16 ulp 9.8e-4)
#   Q8_0 dequant / gather, copies:   bit-exact
RTOL_F32 = 1e-5
RTOL_BF16 = 1e-2
RTOL_F16 = 2e-3


def rel_err(got, ref) -> float:
    """max |got - ref| / max(|ref|, 1), computed in float64."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)))


def pure_rel_err(got, ref, floor=1e-3) -> float:
    """max |got - ref| / |ref| over the elements with |ref| > floor (float64)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    big = np.abs(ref) > floor
    if not big.any():
        return 0.0
    return float(np.max(np.abs(got[big] - ref[big]) / np.abs(ref[big])))


def assert_close(got, ref, rtol, what=""):
    e = rel_err(got, ref)
    assert e <= rtol, (f"{what}: max error {e:.3e} scaled by max(|ref|, 1) > {rtol:.1e} "
                       f"(relative over |ref| > 1e-3: {pure_rel_err(got, ref):.3e})")
    return e


def assert_bitexact(got, ref, what=""):
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, (got.shape, got.dtype, ref.shape, ref.dtype)
    if not np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        gv = got.reshape(-1).view(np.uint32 if got.itemsize == 4 else np.uint16)
        rv = ref.reshape(-1).view(np.uint32 if ref.itemsize == 4 else np.uint16)
        idx = np.flatnonzero(gv != rv)
        raise AssertionError(f"{what}: {idx.size} elements differ, first at {idx[:5]}: "
                             f"{got.reshape(-1)[idx[:5]]} vs {ref.reshape(-1)[idx[:5]]}")


def say(*args):
    """Name the case before a GPU step (flushed, so a crash still shows it)."""
    print("[case]", *args, flush=True)


def dev_tensor(a, device="cuda:0"):
    """numpy -> device tensor; uint16 arrays are taken as bf16 bit patterns,
    uint32 as int32 bit patterns (ids)."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(device)
    return torch.from_numpy(a).to(device)


def host(t):
    """device tensor -> numpy (bf16 as uint16 bit patterns)."""
    import torch

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()
