"""Build libdmc_hip.so (gfx950) and the CPU oracle, in-tree.

    python -m demonic_amd.build            # library + oracle
    python -m demonic_amd.build --lib      # library only

The library is compiled with hipcc for gfx950 only.  Numerics-relevant flags:
no fast-math, no fp contraction (every fused multiply-add is an explicit
fmaf), f32 denormals kept (-fno-gpu-flush-denormals-to-zero), and packed-fp32
instructions disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import argparse
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libdmc_hip.so"
ORACLE_DIR = ROOT / "oracle"

ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}"]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-ffp-contract=off",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib() -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    for src, device in (("gemv_kernels.hip", True), ("dmc_hip_runtime.cpp", False), ("npz_ingress.cpp", False)):
        obj = OBJ / (src.rsplit(".", 1)[0] + ".o")
        lang = ["-x", "hip"] + DEVICE if device else ["-D__HIP_PLATFORM_AMD__"]
        _run([cc, *COMMON, *lang, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", str(tmp), "-lz", "-pthread"])
    os.replace(tmp, LIB)  # atomic: a concurrent loader never sees a half-written file
    return LIB


def build_oracle() -> None:
    _run(["make", "-C", str(ORACLE_DIR), "-B", "-s"])


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--lib", action="store_true", help="build only libdmc_hip.so")
    ap.add_argument("--oracle", action="store_true", help="build only the CPU oracle")
    a = ap.parse_args(argv)
    if not a.oracle:
        build_lib()
    if not a.lib:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
