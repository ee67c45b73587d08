"""Compiled issue order of the decode tile loads (CPU: hipcc cross-compiles gfx950 assembly).

A decode partials tile's K rows go to LDS by LDS-DMA loads and its V rows to registers. The
kernels read K from LDS after an explicit ``s_waitcnt vmcnt(16)``, which covers the tile's K loads
only if at most 16 loads (its V) were issued after the last of them. Loads are independent, so
their order is the compiler's to choose unless the source pins it (scheduling barriers); a K load
moved among the later loads lets the tile compute on K rows that have not landed (wrong results,
no fault).

* Look-ahead loop (every partials kernel but the fused prep + decode): a pass issues tile 0's K
  then its V; at the top of tile k (after the wait) tile k+1's K, and after tile k's arithmetic
  tile k+1's V. Runs therefore hold a whole tile's K loads (NK = 16 bf16 or 8 fp8 LDS-DMA loads),
  16 V loads, or tile 0's K followed by its V.
* Single-slot loop (fused prep + decode): K then V per tile.

In both, no LDS-DMA load may follow a register load within a run, and a run holds 0 or NK LDS-DMA
loads. A run is the loads of one basic block between vmcnt waits. This test compiles
attn_decode.hip with the library's own flags and checks every partials kernel.
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


def _runs(body: str) -> list[str]:
    """The load runs of a kernel body: 'L' per LDS-DMA load, 'R' per register load."""
    runs, cur = [], []
    for line in body.split("\n"):
        t = line.strip()
        if re.match(r"^\.LBB\d+_\d+:|^; %bb", t) or (t.startswith("s_waitcnt") and "vmcnt" in t):
            if cur:
                runs.append("".join(cur))
            cur = []
        elif t.startswith("buffer_load") or t.startswith("global_load"):
            cur.append("L" if t.endswith(" lds") else "R")
    if cur:
        runs.append("".join(cur))
    return runs


def _check_kernel(name: str, body: str) -> list[str]:
    """Problems found in one partials kernel (empty when the order is right)."""
    m = re.search(r"attn_partials_kernelILi(\d+)ELb(\d)ELb(\d)ELb(\d)E", name)
    assert m, name
    nk = 8 if m.group(4) == "1" else 16
    runs = _runs(body)
    bad = []
    for r in runs:
        if re.search(r"R.*L", r):
            bad.append(f"LDS-DMA load after a register load: {r}")
        if r.count("L") not in (0, nk):
            bad.append(f"a run with {r.count('L')} K loads: {r}")
    if not any(r.count("L") == nk and r.count("R") == 16 for r in runs):
        bad.append("no tile-0 run (its K then its V)")
    return bad


def _kernels(asm: str) -> dict[str, str]:
    out = {}
    for m in re.finditer(r"^(_Z\S*attn_partials_kernel\S*):", asm, re.M):
        end = asm.index(".Lfunc_end", m.end())
        out[m.group(1)] = asm[m.end():end]
    return out


def test_checker_flags_bad_orders():
    """The checker itself: a K load after a V load in a run, or a tile's K loads split across runs,
    is flagged; the look-ahead loop's runs pass."""
    L16 = "\tbuffer_load_dwordx4 v1, s[0:3], 0 offen nt lds"
    R16 = "\tbuffer_load_dwordx4 v[2:5], v6, s[4:7], 0 offen nt"
    la = "_ZN2qe20attn_partials_kernelILi1ELb0ELb0ELb0ELi4EEEvv"
    good = "\n".join([L16] * 16 + [R16] * 16 + [".LBB0_1:", "\ts_waitcnt vmcnt(16)"] + [L16] * 16
                     + ["\ts_waitcnt vmcnt(31)"] + [R16] * 16)
    assert _check_kernel(la, good) == []
    swapped = "\n".join([L16] * 15 + [R16] + [L16] + [R16] * 15 + [".LBB0_1:"] + [L16] * 16)
    assert any("after a register load" in b for b in _check_kernel(la, swapped))
    split = "\n".join([L16] * 16 + [R16] * 16 + [".LBB0_1:"] + [L16] * 8 + [".LBB0_2:"] + [L16] * 8)
    assert any("a run with 8 K loads" in b for b in _check_kernel(la, split))


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not installed")
def test_decode_tile_loads_issue_order(tmp_path):
    b = _build_module()
    src = b.CSRC / "attn_decode.hip"
    asm_path = tmp_path / "attn_decode.s"
    cmd = [b.HIPCC, *b.HIP_FLAGS, *b.SOURCE_FLAGS.get(src.name, []), "--offload-device-only",
           "-S", str(src), "-o", str(asm_path)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    found = _kernels(asm_path.read_text())
    assert len(found) >= 8, sorted(found)  # bf16 / fp8 x one-row / multi-row / fused / NT=2
    for name, body in found.items():
        assert _check_kernel(name, body) == [], name
