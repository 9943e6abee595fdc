"""Build ``libtcfp_hip.so`` (hand-written HIP for gfx950) in-tree.

    python -m tcfp_amd.build

Each ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` to
an object under ``tcfp_amd/_build/`` and the objects are linked into
``tcfp_amd/libtcfp_hip.so``.  The library has no libtorch dependency: the
Python side binds it through ctypes.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtcfp_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{INCLUDE}",
    # packed fp32 VALU ops are kept out of the generated code: some of their
    # forms have given wrong results on MI355X without any error; hipcc's
    # host pass warns it does not know the feature, which is harmless.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-file extra flags.  The quantisation kernels and the GEMM epilogues
# that evaluate GELU must match torch's separately rounded elementwise ops
# bit for bit (and each other: the erf / exp they inline are compiled with
# these flags too): no contraction to FMA.
EXTRA = {
    "quant.hip": ["-ffp-contract=off"],
    "gemm.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")
    return cand


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    procs = []
    objs = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *COMMON_FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print("[tcfp_amd.build]", " ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed.append((src, text))
        elif text.strip() and verbose:
            print(text, flush=True)
    if failed:
        msg = "\n".join(f"--- {s.name} ---\n{t}" for s, t in failed)
        raise RuntimeError(f"HIP build failed:\n{msg}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print("[tcfp_amd.build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
