"""Builds libcf_hip.so (the HIP kernels and the C ABI) for gfx950.

Usage: python llm-compileforge_amd/csrc/build.py [--jobs N]

Every .hip file in this directory is compiled with hipcc for gfx950 into
_build/, then linked into ../cf_hip/libcf_hip.so.  Floating-point flags:
no fast-math, fp32 division and sqrt correctly rounded, fp32 denormals kept
(IEEE), so quantized FP8 codes match the CPU bit for bit.  Packed-fp32 VALU
instructions are disabled.  MFMA results are kept in VGPRs (not AGPRs).
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sysconfig
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
BUILD = CSRC / "_build"
LIB = PKG / "cf_hip" / "libcf_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the decode loop rescales and stores its
    # accumulators, and AGPR<->VGPR copies each tile cost more than they save.
    "-Xarch_device",
    "-mllvm=-amdgpu-mfma-vgpr-form",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(jobs: int = 8, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no .hip sources in {CSRC}")
    objs = []
    cmds = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        for cmd, _ in zip(cmds, pool.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    build_tablepack()
    return LIB


def build_tablepack() -> Path:
    """The CPython extension that packs paged_attention's request dicts
    (host code, gcc, in-tree next to the ctypes binding)."""
    src = PKG / "cf_hip" / "_tablepack.c"
    out = PKG / "cf_hip" / ("_tablepack" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    _run(["gcc", "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}", str(src), "-o",
          str(tmp)])
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    lib = build(args.jobs, args.verbose)
    print(lib)


if __name__ == "__main__":
    main()
