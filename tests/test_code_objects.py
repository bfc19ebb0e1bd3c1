"""Static checks of the built gfx950 code objects (CPU only, no GPU needed).

The code objects are this repository's own build output
(nspeech_amd/lib/nsr_<unit>_gfx950.hsaco); they are inspected with the ROCm
LLVM tools:

* every kernel's AMDGPU metadata reports no VGPR spills and no private
  (scratch) segment, so no kernel moves bytes beyond its algorithmic traffic
  through scratch memory;
* no vector-memory store of more than 64 bits of data is followed directly
  by a VALU instruction that writes one of the store's data registers. On
  gfx950 a buffer store whose offset sits in an SGPR soffset gets no wait
  state there from the compiler, and such stores were observed to write the
  overwritten values; the kernels keep store offsets in the VGPR address, and
  this test keeps it that way;
* the runtime's kernel list (nsr_kernels.def, resolved in full when a
  device's code objects load) names exactly the kernels each code object
  holds, unit by unit;
* no int -> float conversion reads a sign-extended sub-dword operand as
  unsigned (v_cvt_f32_u32 with an SDWA sext source). This compiler folds
  __builtin_amdgcn_sbfe(w, off, 8) followed by an int -> float conversion
  into that form, which turns every negative byte into ~4.29e9.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "nspeech_amd" / "lib"
LLVM = Path("/opt/rocm/llvm/bin")
UNITS = ["q8_0_gather", "layernorm", "rotary", "adain_snake", "elementwise", "gemv_q8", "conv1d", "attention", "istft",
         "calib"]
KERNEL_LIST = ROOT / "nspeech_amd" / "csrc" / "runtime" / "nsr_kernels.def"


def _co(unit):
    p = LIB / f"nsr_{unit}_gfx950.hsaco"
    if not p.exists():
        pytest.fail(f"{p} is not built: run `python -m nspeech_amd.build`")
    return p


def _tool(name):
    t = LLVM / name
    if not t.exists():
        found = shutil.which(name)
        if not found:
            pytest.skip(f"{name} not available")
        return found
    return str(t)


def _metadata(unit):
    out = subprocess.run([_tool("llvm-readobj"), "--notes", str(_co(unit))], capture_output=True, text=True,
                         check=True).stdout
    kernels = {}
    cur = None
    for line in out.splitlines():
        m = re.match(r"\s+\.name:\s+(\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.match(r"\s+\.(private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count|vgpr_count):\s+(\d+)",
                     line)
        if m and cur is not None:
            cur[m.group(1)] = int(m.group(2))
    return kernels


@pytest.mark.parametrize("unit", UNITS)
def test_no_scratch_spills(unit):
    md = _metadata(unit)
    assert md, f"no kernels found in {unit}"
    bad = {k: v for k, v in md.items() if v.get("vgpr_spill_count", 0) or v.get("private_segment_fixed_size", 0)}
    assert not bad, f"kernels spilling to scratch: {bad}"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return int(m.group(1)), int(m.group(2))
    m = re.match(r"v(\d+)$", tok)
    if m:
        return int(m.group(1)), int(m.group(1))
    return None


def store_data_hazards(disasm: str):
    """(store, next instruction) pairs where a >64-bit store's data VGPRs are
    written by the immediately following VALU instruction."""
    insts = []
    for line in disasm.splitlines():
        line = line.split("//")[0].strip()
        if not line or line.endswith(":") or line.startswith("<") or line.startswith("Disassembly"):
            continue
        insts.append(line)
    hits = []
    for i, s in enumerate(insts[:-1]):
        m = re.match(r"(global|buffer|flat|scratch)_store_(dwordx[34]|b96|b128)\s+(.*)", s)
        if not m:
            continue
        ops = [o.strip() for o in m.group(3).split(",")]
        data = ops[0] if m.group(1) == "buffer" else ops[1]
        r = _regs(data)
        if r is None:
            continue
        nxt = insts[i + 1]
        w = re.match(r"v_\w+\s+v\[?(\d+)", nxt)
        if w and not nxt.startswith("v_cmp") and r[0] <= int(w.group(1)) <= r[1]:
            hits.append((s, nxt))
    return hits


def test_hazard_scanner_finds_planted_pattern():
    planted = ("buffer_store_dwordx4 v[4:7], v24, s[12:15], s0 offen nt\n"
               "v_fma_f32 v4, v27, v8, v3\n"
               "global_store_dwordx4 v[0:1], v[8:11], off\n"
               "s_nop 0\n"
               "v_mov_b32 v8, 0\n")
    hits = store_data_hazards(planted)
    assert len(hits) == 1 and hits[0][1].startswith("v_fma_f32 v4")


@pytest.mark.parametrize("unit", UNITS)
def test_no_store_data_hazard(unit):
    out = subprocess.run([_tool("llvm-objdump"), "-d", "--mcpu=gfx950", str(_co(unit))], capture_output=True,
                         text=True, check=True).stdout
    assert "s_endpgm" in out, "disassembly produced no kernel code"
    hits = store_data_hazards(out)
    assert not hits, f"{len(hits)} wide stores with data overwritten by the next VALU op, e.g. {hits[:2]}"


_UNSIGNED_CVT_OF_SEXT = re.compile(r"v_cvt_f32_u32_sdwa\s+v\d+,\s*sext\(")


def test_sext_unsigned_convert_pattern_matches_planted_line():
    planted = ("v_cvt_f32_u32_sdwa v0, sext(v2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n"
               "v_cvt_f32_i32_sdwa v1, sext(v2) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n")
    assert len(_UNSIGNED_CVT_OF_SEXT.findall(planted)) == 1


@pytest.mark.parametrize("unit", UNITS)
def test_no_unsigned_convert_of_sign_extended_bytes(unit):
    out = subprocess.run([_tool("llvm-objdump"), "-d", "--mcpu=gfx950", str(_co(unit))], capture_output=True,
                         text=True, check=True).stdout
    hits = _UNSIGNED_CVT_OF_SEXT.findall(out)
    assert not hits, f"{unit}: {len(hits)} unsigned converts of sign-extended bytes"


def _kernel_names(unit):
    out = subprocess.run([_tool("llvm-readelf"), "--dyn-syms", str(_co(unit))], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1][:-3] for line in out.splitlines() if line.endswith(".kd")}


def test_kernel_list_matches_code_objects():
    listed = {}
    for line in KERNEL_LIST.read_text().splitlines():
        m = re.match(r"NSR_KERNEL\((\w+), (\w+)\)", line)
        if m:
            assert m.group(2) not in listed, f"{m.group(2)} listed twice"
            listed[m.group(2)] = m.group(1)
    for unit in UNITS:
        built = _kernel_names(unit)
        mine = {k for k, u in listed.items() if u == unit}
        assert built == mine, f"{unit}: built but not listed {sorted(built - mine)}, listed but not built " \
                              f"{sorted(mine - built)}"
    assert set(listed.values()) <= set(UNITS)
