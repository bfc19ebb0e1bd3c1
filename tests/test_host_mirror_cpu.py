"""C++ host side without a GPU: it builds, links and reports a missing device
as an error (exit status 2, message naming the failed HIP call) rather than
crashing or falling back to the CPU."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "host" / "_build" / "test_host_mirror"
LIB = Path(__file__).resolve().parent.parent / "nspeech_amd" / "lib" / "libnspeech_rocm_host.so"


def _has_gpu():
    import torch

    return torch.cuda.device_count() > 0


def test_host_library_built_and_exports_mirror():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run `python -m nspeech_amd.build`")
    syms = subprocess.run(["nm", "-DC", str(LIB)], capture_output=True, text=True, check=True).stdout
    for name in ("nspeech::rocm::triton_layernorm_std_f32in", "nspeech::rocm::triton_residual_add_layernorm",
                 "nspeech::rocm::enc_layernorm_unit_offset", "nspeech::rocm::enc_gelu",
                 "nspeech::rocm::RocmKokoroBackend::adain_snake_f32", "nspeech::rocm::QEmbedding::forward",
                 "nspeech::rocm::RotaryEmbedding::apply", "nspeech::rocm::RocmKernels::load"):
        assert name in syms, name


def test_no_device_is_an_error():
    if _has_gpu():
        pytest.skip("a GPU is present; the GPU test runs the program")
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built: run `python -m nspeech_amd.build`")
    proc = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2, proc.stdout + proc.stderr
    assert "unexpected error: hipGetDeviceCount" in proc.stdout
