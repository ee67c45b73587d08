"""Compiled issue order of the decode tile loads (CPU: hipcc cross-compiles gfx950 assembly).

Each decode partials tile issues its K rows as LDS-DMA loads, then its V rows as register loads,
and waits with ``s_waitcnt vmcnt(16)`` before reading K from LDS: with at most 16 loads still in
flight, that wait covers every K load only if none of them was issued after a V load. The loads
are independent, so the order is the compiler's to choose unless the source pins it; a K load
scheduled among the V loads lets the tile compute on K rows that have not landed (wrong results,
no fault). This test compiles attn_decode.hip with the library's own flags and checks, in every
partials kernel, that no LDS-DMA load follows a register load in a basic block before the next
vmcnt wait.
"""
from __future__ import annotations

import importlib.util
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _build_module():
    spec = importlib.util.spec_from_file_location("qe_build", ROOT / "qengine_amd" / "_build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _order_violations(asm: str) -> dict[str, tuple[int, int]]:
    """kernel -> (LDS-DMA loads, LDS-DMA loads issued after a register load in the same block
    with no vmcnt wait between)."""
    out = {}
    for m in re.finditer(r"^(_Z\S*attn_partials_kernel\S*):", asm, re.M):
        end = asm.index(".Lfunc_end", m.end())
        seen_reg_load = False
        n_lds = bad = 0
        for line in asm[m.end():end].split("\n"):
            t = line.strip()
            if re.match(r"^\.LBB\d+_\d+:|^; %bb", t):
                seen_reg_load = False
            elif t.startswith("s_waitcnt") and "vmcnt" in t:
                seen_reg_load = False
            elif t.startswith("buffer_load") or t.startswith("global_load"):
                if t.endswith(" lds"):
                    n_lds += 1
                    bad += seen_reg_load
                else:
                    seen_reg_load = True
        out[m.group(1)] = (n_lds, bad)
    return out


def test_order_checker_flags_interleaving():
    """The checker itself: a K load after a V load in one block is flagged; a wait or a new block
    clears it."""
    asm = "\n".join([
        "_ZN2qe20attn_partials_kernelILi1EEEvv:",
        "\tbuffer_load_dwordx4 v1, s[0:3], 0 offen nt lds",
        "\tbuffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen nt",
        "\tbuffer_load_dwordx4 v1, s[0:3], 0 offen nt lds",
        "\ts_waitcnt vmcnt(16)",
        "\tbuffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen nt",
        ".LBB0_1:",
        "\tbuffer_load_dwordx4 v1, s[0:3], 0 offen nt lds",
        ".Lfunc_end0:",
    ])
    assert _order_violations(asm) == {"_ZN2qe20attn_partials_kernelILi1EEEvv": (3, 1)}


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not installed")
def test_decode_tile_loads_issue_k_before_v(tmp_path):
    b = _build_module()
    src = b.CSRC / "attn_decode.hip"
    asm_path = tmp_path / "attn_decode.s"
    cmd = [b.HIPCC, *b.HIP_FLAGS, *b.SOURCE_FLAGS.get(src.name, []), "--offload-device-only",
           "-S", str(src), "-o", str(asm_path)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    found = _order_violations(asm_path.read_text())
    assert len(found) >= 8, sorted(found)  # bf16 / fp8 x one-row / multi-row / fused / NT=2
    for name, (n_lds, bad) in found.items():
        assert n_lds > 0, name
        assert bad == 0, (name, n_lds, bad)
