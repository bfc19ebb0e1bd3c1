"""Static check (CPU only): no kernel in the built gfx950 code objects writes
through the scalar data cache. Every store and atomic in these kernels is a
vector-memory instruction; scalar stores, scalar atomics and the scalar
cache's write-back / invalidate-with-write instructions must not appear.
(This file is host-side tooling only; no GPU run loads it.)"""
import re
import subprocess

import pytest

from .test_code_objects import UNITS, _co, _tool

_SCALAR_WRITE = re.compile(r"^\s*(s_store_|s_buffer_store|s_scratch_store|s_atomic_|s_buffer_atomic_|"
                           r"s_dcache_wb|s_dcache_discard)", re.M)


def test_pattern_matches_planted_lines():
    planted = "\ts_store_dword s1, s[2:3], 0x0\n\ts_load_dword s1, s[2:3], 0x0\n\ts_dcache_wb\n"
    assert len(_SCALAR_WRITE.findall(planted)) == 2


@pytest.mark.parametrize("unit", UNITS)
def test_no_scalar_cache_writes(unit):
    out = subprocess.run([_tool("llvm-objdump"), "-d", "--mcpu=gfx950", str(_co(unit))], capture_output=True,
                         text=True, check=True).stdout
    assert "s_endpgm" in out
    hits = _SCALAR_WRITE.findall(out)
    assert not hits, f"{unit}: scalar-cache writes {sorted(set(hits))}"
