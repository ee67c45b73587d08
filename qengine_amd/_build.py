"""Build recipe for qengine_amd's native code (no setuptools, no hipify).

  libqe_attn.so  : gfx950 HIP kernels + the C ABI of include/qe_attn.h, include/qe_gemv.h,
                   include/qe_step.h and include/qe_gdn.h (hipcc).
  _C<ext>.so     : torch extension with the reference's op signatures (g++ against torch's
                   ROCm build), linked to libqe_attn.so through $ORIGIN.

Run ``python qengine_amd/_build.py`` (as a script: importing the package needs the build). Every call recompiles. Objects go to ``_build/`` at the repo
root and the two libraries are written next to this file.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["attn_prep.hip", "attn_decode.hip", "attn_combine.hip", "attn_prefill.hip",
               "gemv.hip", "gemv_lds.hip", "step.hip", "gdn.hip", "gdn_split.hip"]
# Per-source code-generation flags. The prefill tile loop keeps 128 fp32 accumulators live; the
# compiler's default MFMA register form parks them in AGPRs and copies all of them into VGPRs
# on every iteration. The VGPR form keeps them in place. The max-ILP machine scheduler keeps
# two or more LDS operand reads in flight in the tile loop where the default occupancy-first
# scheduler kept one (same code, same bits; config 5 about 9% faster).
# The decode combine, the Gated DeltaNet split path and the 1-2-row GEMV are scheduled the same
# way; the kernels that measured slower under it (decode partials, the one-workgroup Gated
# DeltaNet step, the 3-8-row GEMV) sit in files of their own with the default.
MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {"attn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", *MAX_ILP],
                "attn_combine.hip": MAX_ILP, "gdn_split.hip": MAX_ILP, "gemv_lds.hip": MAX_ILP}
LIB = PKG / "libqe_attn.so"
EXT = PKG / ("_C" + sysconfig.get_config_var("EXT_SUFFIX"))

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    # no packed fp32 math anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _hip_objects() -> list[Path]:
    OBJ.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in HIP_SOURCES if (CSRC / s).exists()]
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(so[0].name, []), "-c",
                                     str(so[0]), "-o", str(so[1])]),
                    zip(srcs, objs)))
    return objs


def build_lib() -> Path:
    objs = _hip_objects()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_ext() -> Path:
    import torch
    from torch.utils import cpp_extension as ce

    tlib = Path(torch.__file__).resolve().parent / "lib"
    incs = [*ce.include_paths(device_type="cuda"), sysconfig.get_paths()["include"], str(INCLUDE)]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    obj = OBJ / "bindings.o"
    OBJ.mkdir(exist_ok=True)
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-variable",
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
          "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          *[f"-I{i}" for i in incs], "-c", str(CSRC / "bindings.cpp"), "-o", str(obj)])
    tmp = EXT.with_suffix(".tmp")
    _run(["g++", "-shared", "-fPIC", str(obj), "-o", str(tmp),
          f"-L{PKG}", "-lqe_attn", f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
          "-ltorch_hip", "-ltorch_python", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"])
    os.replace(tmp, EXT)
    return EXT


def build() -> None:
    build_lib()
    build_ext()


def built() -> bool:
    return LIB.exists() and EXT.exists()


if __name__ == "__main__":
    build()
    print(f"built {LIB.name} and {EXT.name}")
