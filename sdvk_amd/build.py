"""Builds libmi_sdvk.so (the C-ABI library) in-tree with hipcc for gfx950.

Usage: python -m sdvk_amd.build [--save-temps DIR]
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libmi_sdvk.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

SOURCES = ["status.hip", "q8_0.hip", "gemm_q8.hip", "attention.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay off: every kernel is compiled without them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    p = ROCM / "bin" / "hipcc"
    return str(p) if p.exists() else "hipcc"


def build(save_temps: str | None = None, verbose: bool = False) -> Path:
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    if save_temps:
        Path(save_temps).mkdir(parents=True, exist_ok=True)
        cmd.append(f"--save-temps={'obj'}")
    cmd += [str(CSRC / s) for s in SOURCES]
    cmd += ["-o", str(LIB) + ".tmp", f"-Wl,-rpath,{ROCM / 'lib'}"]
    env = dict(os.environ)
    cwd = save_temps if save_temps else None
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, cwd=cwd, env=env, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    st = None
    if "--save-temps" in sys.argv:
        st = sys.argv[sys.argv.index("--save-temps") + 1]
    print(build(save_temps=st, verbose=True))
