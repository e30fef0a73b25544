"""Build the gfx950 shared library libgofann_hip.so in-tree.

Compiles every HIP/C++ source under csrc/ with hipcc for gfx950 only and
links them into go-fann_amd/libgofann_hip.so (the C-ABI library declared in
include/gofann_hip.h).  Run: python go-fann_amd/build.py
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "libgofann_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
    "-Wall", "-Wno-unused-function",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    # Packed FP32 instructions stay disabled on this hardware pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: Path, out_dir: Path = OUT_DIR, defines: tuple = ()) -> Path:
    obj = out_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMMON, *[f"-D{d}" for d in defines]]
    if src.suffix == ".hip":
        cmd += ["-x", "hip", *DEVICE]
    else:
        cmd += ["-D__HIP_PLATFORM_AMD__"]
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"compile failed: {src.name}")
    if res.stderr.strip():
        # hipcc's host pass warns that it does not know the packed-fp32
        # feature; anything else is shown.
        lines = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l
                 and "not a recognized feature" not in l and l.strip()]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(verbose: bool = True, lib: Path = LIB, defines: tuple = ()) -> Path:
    """Compile every source and link `lib`; `defines` are extra -D macros
    (e.g. GOFANN_TRAVERSAL_MIN_WAVES=5) for alternative builds."""
    out_dir = OUT_DIR if not defines else OUT_DIR / "_".join(defines).replace("=", "")
    out_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda src: _compile(src, out_dir, defines), sources))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           "-o", str(tmp), "-lpthread", "-lrocblas"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build()
