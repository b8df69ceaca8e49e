"""Static check of the gfx950 code of every HIP source: no VMEM store wider than 8 bytes may be
followed, as the next instruction of the fall-through path, by a VALU instruction that
overwrites one of the store's data registers.

The hardware reads such a store's data a cycle after issue, so it needs one wait state before
the registers are rewritten; the compiler was seen to omit it where the store ended a basic
block (a pool kernel stored a value that already held the next row's term, on a few lanes).
The kernels avoid the pattern; this test keeps it from coming back.  CPU only: it compiles to
assembly with hipcc (no GPU needed).
"""

import concurrent.futures
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "dwarf_amd" / "csrc"
WIDE_STORE = re.compile(r"^\s+(buffer|global|flat)_store_dwordx[34]\s+(.*)$")


def _vregs(tok: str) -> set:
    tok = tok.strip()
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _hazards(asm: str):
    lines = asm.splitlines()
    found = []
    for i, line in enumerate(lines):
        m = WIDE_STORE.match(line)
        if not m:
            continue
        ops = [t.strip() for t in m.group(2).split(",")]
        data = _vregs(ops[0] if m.group(1) == "buffer" else ops[1])
        j = i + 1
        while j < len(lines):
            t = lines[j].strip()
            if t and not t.startswith((";", ".")) and not t.endswith(":"):
                break
            j += 1
        nxt = lines[j].strip() if j < len(lines) else ""
        if nxt.startswith("v_") and not nxt.startswith(("v_cmp", "v_readfirstlane", "v_readlane")):
            parts = nxt.split(None, 1)
            dst = parts[1].split(",")[0] if len(parts) > 1 else ""
            if _vregs(dst) & data:
                found.append(f"line {i + 1}: {line.strip()} -> {nxt}")
    return found


def _compile(src: Path, out_dir: Path):
    from dwarf_amd.build import HIPCC_FLAGS, hipcc_path
    flags = [f for f in HIPCC_FLAGS if f not in ("-fPIC",) and not f.startswith("-Rpass")]
    out = out_dir / (src.stem + ".s")
    subprocess.run([hipcc_path(), *flags, f"-I{ROOT / 'include'}", "--cuda-device-only", "-S",
                    str(src), "-o", str(out)], check=True, capture_output=True)
    return src.name, out.read_text()


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_no_valu_overwrite_right_after_wide_store(tmp_path):
    sources = sorted(CSRC.glob("*.hip"))
    assert sources
    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as ex:
        results = list(ex.map(lambda s: _compile(s, tmp_path), sources))
    bad = {name: h for name, asm in results for h in [_hazards(asm)] if h}
    assert not bad, "store-data hazards: " + repr(bad)


def test_checker_flags_the_pattern():
    asm = """
    buffer_store_dwordx4 v[0:3], v4, s[0:3], s8 offen
.LBB1_253:
    v_add_f32_e32 v1, v1, v82
    global_store_dwordx4 v[6:7], v[8:11], off
    s_nop 0
    v_mov_b32_e32 v9, 0
    global_store_dwordx2 v[6:7], v[8:9], off
    v_mov_b32_e32 v8, 0
"""
    found = _hazards(asm)
    assert len(found) == 1 and "v_add_f32_e32 v1" in found[0]
