"""Builds libemel_hip.so for gfx950 from emel.rs_amd/csrc (python emel.rs_amd/emel_build.py).

Every translation unit is compiled by hipcc with
  -ffp-contract=off   a*b+c stays two roundings, as in the reference;
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed-f32 VALU instructions;
and the objects are linked into emel.rs_amd/emel_hip/libemel_hip.so, which
travels with the repository to the GPU box.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = PKG / "emel_hip"
LIB = OUT_DIR / "libemel_hip.so"
OBJ_DIR = PKG / "_build"

ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libemel_hip.so")
    return path


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build(verbose: bool = False) -> Path:
    """Compiles every source (always; no up-to-date check) and links the library."""
    OBJ_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in sources():
        obj = OBJ_DIR / (src.name + ".o")
        objs.append(obj)
        cmd = [cc, *common_flags(), "-c", str(src), "-o", str(obj)]
        if src.suffix == ".hip":
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append((src, out))
        elif verbose and out.strip():
            print(out, flush=True)
    if failed:
        msg = "\n".join(f"--- {s.name}\n{o}" for s, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(link), flush=True)
    r = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
