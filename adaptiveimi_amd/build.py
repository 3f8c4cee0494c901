"""Build libimi_hip.so (the C-ABI library) for gfx950.

Every .hip source under csrc/ is compiled with hipcc for gfx950 only and the
objects are linked with the host C++ compiler against the HIP runtime that
PyTorch loads (torch/lib/libamdhip64.so), so a process that uses torch and
this library holds exactly one HIP runtime.  The output lands in-tree next to
this file.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libimi_hip.so"
BUILD_DIR = PKG / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",               # every fused multiply-add is spelled out
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]

# Per-source additions.  k-means: matrix-core results go straight to VGPRs
# (its E-step reads every accumulator with VALU code; the AGPR form costs one
# copy per value).
EXTRA_FLAGS = {
    "imi_kmeans.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _torch_lib_dir() -> Path:
    import torch  # noqa: F401  (only to locate the bundled HIP runtime)

    return Path(torch.__file__).resolve().parent / "lib"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int = 4, force: bool = False) -> Path:
    """Compile every source (force) or the ones newer than their object."""
    BUILD_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    headers = list(CSRC.glob("*.hpp")) + [PKG.parent / "include" / "imi_hip.h"]
    newest_header = max(h.stat().st_mtime for h in headers)

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        if not force and obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, newest_header):
            return obj
        cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-I", str(PKG.parent / "include"), "-c",
               str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
        errs = [ln for ln in r.stderr.splitlines() if "warning" in ln and "packed-fp32-ops" not in ln]
        if errs and verbose:
            print("\n".join(errs), file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources()))
    tl = _torch_lib_dir()
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["g++", "-shared", "-o", str(tmp), *map(str, objs), f"-L{tl}", "-lamdhip64", f"-Wl,-rpath,{tl}",
           "-Wl,--no-undefined", "-Wl,-z,defs"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
