"""Build the gfx950 code objects, libnspeech_rocm.so and the CPU oracle.

Run as ``python -m nspeech_amd.build`` (or through ``__graft_entry__.build``).
Every call recompiles. Outputs (git-ignored, shipped to the GPU box with the
tree):

  nspeech_amd/lib/nsr_<unit>_gfx950.hsaco   one code object per kernel unit
  nspeech_amd/lib/libnspeech_rocm.so        C ABI (include/nspeech_rocm.h),
                                            code objects embedded
  nspeech_amd/lib/libnspeech_rocm_host.so   C++ host side (nspeech_amd/host/
                                            rocm_kernels.h) over the C ABI
  nspeech_amd/lib/nsr_enqueue_bench         host time per call of the decode-
                                            step entry points (bench.py)
  tests/host/_build/test_host_mirror        C++ tests of the host side
  oracle/_build/libnsr_oracle.so            CPU oracle (test infrastructure)
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
ARCH = "gfx950"

# Kernel units: kernels/<unit>.hip -> lib/nsr_<unit>_gfx950.hsaco. The same
# list is embedded by runtime/nsr_embed.S and searched by nsr_runtime.cpp.
UNITS = ["q8_0_gather", "layernorm", "rotary", "adain_snake", "elementwise", "gemv_q8", "conv1d", "attention", "istft",
         "calib"]

HIP_FLAGS = [
    "--genco",
    f"--offload-arch={ARCH}",
    "--no-gpu-bundle-output",
    "-O3",
    "-std=c++17",
    "-mcode-object-version=5",
    # keep the compiler from forming packed-FP32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], cwd: Path = ROOT) -> None:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def code_object_path(unit: str) -> Path:
    return LIB / f"nsr_{unit}_{ARCH}.hsaco"


def build_code_objects() -> list[Path]:
    LIB.mkdir(parents=True, exist_ok=True)

    def one(unit: str) -> Path:
        out = code_object_path(unit)
        tmp = out.with_suffix(".hsaco.tmp")
        _run([str(HIPCC), *HIP_FLAGS, "-o", str(tmp), str(CSRC / "kernels" / f"{unit}.hip")])
        os.replace(tmp, out)
        return out

    with ThreadPoolExecutor(max_workers=len(UNITS)) as ex:
        return list(ex.map(one, UNITS))


def build_scratch_object() -> Path:
    """runtime/nsr_scratch.hip (the fixed per-device scratch of the entry
    points that allocate nothing) as a host object with its gfx950 device
    code embedded, linked into libnspeech_rocm.so."""
    out = LIB / "nsr_scratch.o"
    _run([str(HIPCC), "-c", "-fPIC", "-O2", "-std=c++17", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          str(CSRC / "runtime" / "nsr_scratch.hip"), "-o", str(out)])
    return out


def build_library() -> Path:
    out = LIB / "libnspeech_rocm.so"
    tmp = LIB / "libnspeech_rocm.so.tmp"
    scratch = build_scratch_object()
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
        "-Wall", "-Wextra", "-Wno-unused-parameter",
        "-D__HIP_PLATFORM_AMD__",
        f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}",
        f"-DNSR_CO_DIR={LIB}",
        str(CSRC / "runtime" / "nsr_runtime.cpp"),
        str(CSRC / "runtime" / "nsr_embed.S"),
        str(scratch),
        f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
        "-Wl,--no-undefined",
        "-o", str(tmp),
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


HOST_CXX = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__"]


def build_host_library() -> Path:
    """C++ host side (namespace nspeech::rocm) linked against the C ABI."""
    out = LIB / "libnspeech_rocm_host.so"
    tmp = LIB / "libnspeech_rocm_host.so.tmp"
    _run([*HOST_CXX, "-shared", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}",
          str(PKG / "host" / "rocm_kernels.cpp"), str(PKG / "host" / "gguf.cpp"),
          f"-L{LIB}", "-lnspeech_rocm", f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_enqueue_bench() -> Path:
    """nspeech_amd/host/enqueue_bench.cpp -> lib/nsr_enqueue_bench: host time per call of the decode-step entry
    points, run by bench.py."""
    out = LIB / "nsr_enqueue_bench"
    tmp = LIB / "nsr_enqueue_bench.tmp"
    _run([*HOST_CXX, "-O2", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", str(PKG / "host" / "enqueue_bench.cpp"),
          f"-L{LIB}", "-lnspeech_rocm", f"-L{ROCM / 'lib'}", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
          f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_host_tests() -> Path:
    """tests/host/test_host_mirror.cpp -> tests/host/_build/test_host_mirror."""
    src = ROOT / "tests" / "host" / "test_host_mirror.cpp"
    out_dir = ROOT / "tests" / "host" / "_build"
    out_dir.mkdir(parents=True, exist_ok=True)
    out = out_dir / "test_host_mirror"
    tmp = out_dir / "test_host_mirror.tmp"
    _run([*HOST_CXX, f"-I{PKG / 'host'}", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", str(src),
          f"-L{LIB}", "-lnspeech_rocm_host", "-lnspeech_rocm", f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN/../../../nspeech_amd/lib", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(tmp)])
    os.replace(tmp, out)
    # the GGUF reader built with AddressSanitizer (host code only, g++), for
    # the malformed-file tests
    asan = out_dir / "test_gguf_asan"
    _run(["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", f"-I{PKG / 'host'}",
          str(ROOT / "tests" / "host" / "test_gguf_asan.cpp"), str(PKG / "host" / "gguf.cpp"),
          str(PKG / "host" / "rocm_kernels.cpp"), f"-L{LIB}", "-lnspeech_rocm", f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN/../../../nspeech_amd/lib", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(asan) + ".tmp"])
    os.replace(str(asan) + ".tmp", asan)
    return out


def build_oracle() -> Path:
    sys.path.insert(0, str(ROOT))
    from oracle import build as oracle_build  # noqa: E402

    return oracle_build.build()


def build_all() -> None:
    build_code_objects()
    build_library()
    build_host_library()
    build_enqueue_bench()
    build_host_tests()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built:", *(str(p.relative_to(ROOT)) for p in sorted(LIB.glob("*"))), sep="\n  ")
