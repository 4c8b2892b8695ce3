"""Builds se12_amd/_lib/libse12_gfx950.so with hipcc (gfx950 only).

    python -m se12_amd.csrc.build            # or: python se12_amd/csrc/build.py

Every HIP translation unit is compiled in parallel, then linked into one
shared library whose exported symbols are the C ABI of include/se12_gfx950.h.
"""

from __future__ import annotations

import os
import pathlib
import re
import shutil
import subprocess
import sys

CSRC = pathlib.Path(__file__).resolve().parent
PKG = CSRC.parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
LIBDIR = PKG / "_lib"
LIBNAME = "libse12_gfx950.so"
SOURCES = ("se12_abi.hip", "se12_gemv.hip", "se12_gemm.hip", "se12_decode.hip", "se12_encode.hip", "se12_step.hip",
           "se12_probe.hip", "se12_gemm_rx.hip")
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for every HIP unit (hipcc's host pass
# warns that it does not know the feature; that warning is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source flags. The GEMV kernels take matrix 0's hot arguments as their
# first 9 kernel arguments and have the dispatch preload them into SGPRs
# (gfx950 kernarg preload; LLVM also emits the load sequence for firmware
# without it), so their first tile loads need no kernel-argument round trip.
SOURCE_FLAGS = {
    "se12_gemv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
    # the attention kernels' leading arguments likewise (the position pointer,
    # q / k / key cache or the softmax statistics, scores and value cache,
    # and the sizes the first loads' addresses need)
    "se12_step.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
}


def spilling_kernels(remarks: str) -> list[str]:
    """Kernels that hipcc's resource-usage remarks report as spilling VGPRs or
    using scratch memory: a launch bound set too high for the variant. (SGPR
    spills land in VGPR lanes, not memory, and are not counted.)"""
    bad, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+(VGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
        if m and name and int(m.group(2)) > 0 and name not in bad:
            bad.append(name)
    return bad


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the SE12 library needs ROCm's hipcc to build")
    return path


def library_path() -> pathlib.Path:
    return LIBDIR / LIBNAME


def build(verbose: bool = False) -> pathlib.Path:
    """Compiles every source and links the library; returns its path."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    objdir = LIBDIR / "obj"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objects = []
    for src in SOURCES:
        obj = objdir / (src + ".o")
        objects.append(obj)
        cmd = [cc, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), "-Rpass-analysis=kernel-resource-usage", "-c", str(CSRC / src),
               "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed, spills = [], []
    for src, p in procs:
        out, _ = p.communicate()
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and "remark:" not in ln
                 and not ln.lstrip().startswith(("|", "^")) and not re.match(r"\s*\d+ \|", ln)]
        if p.returncode != 0:
            failed.append(src)
            sys.stderr.write("\n".join(lines) + "\n")
        elif verbose and lines:
            print("\n".join(lines))
        spills += spilling_kernels(out)
    if failed:
        raise RuntimeError(f"hipcc failed on {', '.join(failed)}")
    if spills:
        raise RuntimeError(f"kernels spill registers or use scratch (lower their launch bounds): {', '.join(spills)}")
    tmp = LIBDIR / (LIBNAME + ".tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    res = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, library_path())
    return library_path()


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
