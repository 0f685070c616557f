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

SOURCES = ["status.hip", "q8_0.hip", "gemm_q8.hip", "gemm_nn_q8.hip", "attention.hip", "glue.hip", "block.hip",
           "gguf.cpp"]

# Per-source extra flags. The attention kernel rescales its MFMA accumulators
# with VALU ops; keeping MFMA operands in VGPRs (rather than AGPRs) removes the
# per-tile AGPR<->VGPR copies around every rescale.
EXTRA_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

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


def _run(cmd: list[str], cwd: str | None, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)


def build(save_temps: str | None = None, verbose: bool = False) -> Path:
    """Compiles every source to an object (in parallel) and links libmi_sdvk.so."""
    import concurrent.futures
    import tempfile

    with tempfile.TemporaryDirectory(prefix="mi_sdvk_build_") as tmp:
        cwd = save_temps if save_temps else None
        if save_temps:
            Path(save_temps).mkdir(parents=True, exist_ok=True)
        jobs = []
        for src in SOURCES:
            obj = str(Path(tmp) / (src + ".o"))
            cmd = [hipcc(), *HIPCC_FLAGS, "-c", *EXTRA_FLAGS.get(src, []), f"-I{ROOT / 'include'}", f"-I{CSRC}",
                   str(CSRC / src), "-o", obj]
            cmd.remove("-shared")
            if save_temps:
                cmd.append("--save-temps=obj")
            jobs.append((cmd, obj))
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(jobs)) as ex:
            list(ex.map(lambda j: _run(j[0], cwd, verbose), jobs))
        link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[o for _, o in jobs],
                "-o", str(LIB) + ".tmp", f"-Wl,-rpath,{ROCM / 'lib'}"]
        _run(link, cwd, verbose)
    os.replace(str(LIB) + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    st = None
    if "--save-temps" in sys.argv:
        st = sys.argv[sys.argv.index("--save-temps") + 1]
    print(build(save_temps=st, verbose=True))
