"""Static checks of the gfx950 code of every HIP source, for two sequences the compiler emits
without the wait states the hardware needs.  CPU only: it compiles to assembly with hipcc (no
GPU needed).

1. No VMEM store wider than 8 bytes may be followed, as the next instruction of the
   fall-through path, by a VALU instruction that overwrites one of the store's data registers.
   The hardware reads such a store's data a cycle after issue, so it needs one wait state
   before the registers are rewritten; the compiler was seen to omit it where the store ended a
   basic block (a pool kernel stored a value that already held the next row's term, on a few
   lanes).
2. No MFMA may take as its accumulator input (SrcC) the result of an MFMA of another opcode
   written fewer than 8 wait states earlier.  The compiler treats an exact SrcC overlap as the
   back-to-back accumulation the hardware forwards and inserts no wait states, whatever the two
   opcodes; a v_mfma_f32_16x16x16_bf16 issued right after a v_mfma_f32_16x16x32_bf16 into the
   same accumulator read a stale accumulator (dq's scale_embed term folded into 16x16x32
   products: dq 8x the parity bound; with s_nop 7 between the two it matched).  The kernels
   chain only MFMAs of one opcode through an accumulator.

The kernels avoid both patterns; these tests keep them from coming back.
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


MFMA = re.compile(r"^\s+(v_mfma_\S+)\s+([va]\[\d+:\d+\]),\s*(\S+),\s*(\S+),\s*([va]\[\d+:\d+\]|0)")
MIXED_CHAIN_WAIT_STATES = 8


def _mixed_mfma_chains(asm: str):
    """MFMAs whose SrcC is the exact result registers of an MFMA of another opcode written fewer
    than MIXED_CHAIN_WAIT_STATES wait states earlier in the same basic block (each instruction
    counts one, s_nop N counts N + 1)."""
    last, ws, found = {}, 0, []
    for i, line in enumerate(asm.splitlines()):
        t = line.strip()
        if not t or t.startswith((";", ".")):
            continue
        if t.endswith(":"):
            last.clear()
            continue
        m = MFMA.match(line)
        if m:
            op, dst, _, _, src_c = m.groups()
            prev = last.get(src_c)
            if prev and prev[0] != op and ws - prev[1] < MIXED_CHAIN_WAIT_STATES:
                found.append(f"line {i + 1}: {prev[0]} -> {t}")
            last[dst] = (op, ws)
        ws += int(t.split()[1]) + 1 if t.startswith("s_nop") else 1
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
    mixed = {name: h for name, asm in results for h in [_mixed_mfma_chains(asm)] if h}
    assert not mixed, "mixed-opcode MFMA accumulation chains: " + repr(mixed)


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


def test_checker_flags_mixed_mfma_chains():
    asm = """
    v_mfma_f32_16x16x32_bf16 v[48:51], v[70:73], v[108:111], v[48:51]
    v_mfma_f32_16x16x16_bf16 v[48:51], v[70:71], v[74:75], v[48:51]
    v_mfma_f32_16x16x16_bf16 v[48:51], v[70:71], v[76:77], v[48:51]
    v_mfma_f32_16x16x32_bf16 v[52:55], v[70:73], v[108:111], v[52:55]
    s_nop 7
    v_mfma_f32_16x16x16_bf16 v[52:55], v[70:71], v[74:75], v[52:55]
.LBB0_1:
    v_mfma_f32_16x16x16_bf16 v[56:59], v[70:71], v[74:75], v[52:55]
"""
    found = _mixed_mfma_chains(asm)
    assert len(found) == 1 and "v[48:51]" in found[0]
