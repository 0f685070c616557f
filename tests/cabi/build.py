"""Builds tests/cabi/gpu_harness, the C++ caller of libmi_sdvk.so that drives
the GPU through the C-ABI (host code only: g++ against the HIP runtime).
Called by __graft_entry__.build() after the library is built, so the binary
ships with the library to the GPU box; the GPU test only runs it."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HARNESS = HERE / "gpu_harness"


def build() -> Path:
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
           f"-I{ROOT / 'include'}", str(HERE / "gpu_harness.cpp"), "-o", str(HARNESS) + ".tmp",
           f"-L{ROOT / 'sdvk_amd'}", "-lmi_sdvk", f"-L{ROCM / 'lib'}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../sdvk_amd", f"-Wl,-rpath,{ROCM / 'lib'}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gpu_harness build failed:\n{r.stdout}{r.stderr}")
    os.replace(str(HARNESS) + ".tmp", HARNESS)
    return HARNESS


if __name__ == "__main__":
    print(build())
