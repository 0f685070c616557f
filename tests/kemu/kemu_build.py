"""Builds the emulation library for the CPU kernel checks.

The product's HIP sources (sdvk_amd/csrc) are compiled for the host against
tests/kemu/include/hip/hip_runtime.h and linked with the fiber runtime
(kemu.cpp) into tests/kemu/_build/libkemu_sdvk.so, which exports the same
C-ABI as libmi_sdvk.so but runs every kernel on the CPU, one work-item per
fiber. The only source change is mechanical: each triple-chevron launch
`k<<<grid, block, shmem, stream>>>(args);` becomes
`::kemu::launch("k", k, grid, block, shmem, stream, args);`.

Test infrastructure only: nothing in the product loads this library.
The build is cached on a hash of every input.
"""
from __future__ import annotations

import hashlib
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
# KEMU_CSRC / KEMU_OUT build another copy of the sources into another folder
# (e.g. a deliberately broken kernel, to see that the checks catch it)
CSRC = Path(os.environ.get("KEMU_CSRC", ROOT / "sdvk_amd" / "csrc"))
OUT = Path(os.environ.get("KEMU_OUT", HERE / "_build"))
LIB = OUT / "libkemu_sdvk.so"
CXX = os.environ.get("KEMU_CXX", "/opt/rocm/llvm/bin/clang++")

SOURCES = ["status.hip", "q8_0.hip", "gemm_q8.hip", "gemm_nn_q8.hip", "attention.hip", "glue.hip", "block.hip",
           "gguf.cpp"]
FLAGS = ["-std=c++17", "-O2", "-g0", "-fPIC", "-fno-strict-aliasing", "-Xclang", "-ffloat16-excess-precision=none",
         "-Wno-unused-command-line-argument", "-Wno-psabi"]

LAUNCH = re.compile(r"([A-Za-z_]\w*(?:<[^<>;()]*>)?)\s*<<<(.*?)>>>\s*\((.*?)\)\s*;", re.S)
# empty asm statements that pin a value in a VGPR (register-allocation hints
# with no effect on values) have no host meaning
PIN = re.compile(r'asm\s+volatile\(\s*""\s*:\s*"\+v"\([^;]*?\)\s*\)\s*;')


def transform(text: str) -> str:
    """Rewrites every kernel launch into a call of the emulator's launcher."""
    def repl(m: re.Match) -> str:
        kernel, cfg, args = m.group(1), " ".join(m.group(2).split()), m.group(3)
        name = " ".join(kernel.split())
        sep = ", " if args.strip() else ""
        return f'::kemu::launch("{name}", {kernel}, {cfg}{sep}{args});'

    out = PIN.sub("(void)0;", LAUNCH.sub(repl, text))
    # LDS pointers are plain host pointers here
    out = out.replace("__attribute__((address_space(3)))", "")
    if "<<<" in out or re.search(r"\basm\b", out):
        raise RuntimeError("a kernel launch or an asm statement was not rewritten")
    return out


def _inputs() -> list[Path]:
    return ([CSRC / s for s in SOURCES] + [CSRC / "common.hpp", ROOT / "include" / "mi_sdvk.h", HERE / "kemu.cpp",
             HERE / "kemu.hpp", HERE / "include" / "hip" / "hip_runtime.h", Path(__file__).resolve()])


def _stamp() -> str:
    h = hashlib.sha256()
    for p in _inputs():
        h.update(p.name.encode())
        h.update(p.read_bytes())
    h.update(" ".join([CXX] + FLAGS).encode())
    return h.hexdigest()


def build(force: bool = False) -> Path:
    stamp = _stamp()
    stamp_file = OUT / "stamp"
    if not force and LIB.exists() and stamp_file.exists() and stamp_file.read_text() == stamp:
        return LIB
    (OUT / "src").mkdir(parents=True, exist_ok=True)
    inc = ["-I", str(HERE / "include"), "-I", str(CSRC), "-I", str(ROOT / "include")]
    jobs = []
    for s in SOURCES:
        dst = OUT / "src" / (Path(s).stem + ".cpp")
        dst.write_text(transform((CSRC / s).read_text()))
        jobs.append([CXX, *FLAGS, *inc, "-c", str(dst), "-o", str(OUT / (Path(s).stem + ".o"))])
    jobs.append([CXX, *FLAGS, *inc, "-c", str(HERE / "kemu.cpp"), "-o", str(OUT / "kemu.o")])

    def run(cmd):
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{' '.join(cmd)}\n{r.stderr[-6000:]}")

    with ThreadPoolExecutor(max_workers=min(len(jobs), 6)) as ex:
        list(ex.map(run, jobs))
    objs = [str(OUT / (Path(s).stem + ".o")) for s in SOURCES] + [str(OUT / "kemu.o")]
    run([CXX, "-shared", "-o", str(LIB), *objs])
    stamp_file.write_text(stamp)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
