"""C++ host side (nspeech_amd/host/rocm_kernels.h) on the GPU.

Runs tests/host/_build/test_host_mirror, the C++ test program written like
the reference's own Kokoro GPU self-tests (src/kokoro/gpu_decoder.rs:64-456):
known-answer inputs, float64 expectations, one max-error line per test. It
exercises the triton_*/enc_* entry points, KokoroGpuBackend::adain_snake_f32,
QEmbedding::forward (bit-exact, out-of-range ids rejected) and
apply_rotary_pos_emb through the host mirror and the C ABI.
"""
import subprocess
from pathlib import Path

import pytest

from ._util import say

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "host" / "_build" / "test_host_mirror"


def test_host_mirror_program(dev):
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built: run `python -m nspeech_amd.build`")
    say("host mirror C++ tests")
    proc = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    assert "PASSED: 0 failed" in proc.stdout
