"""Static checks of the gfx950 code the compiler makes of the product kernels.

Parity tests cannot see a software pipeline that the compiler has undone: a
load hoisted next to its consumer, a wait count made conservative by a load
under a branch, a register spill inside the K loop (a scratch reload waits for
every global load in flight). Those show up only as time on the GPU. This
module compiles a source to gfx950 assembly (the same flags as the product
build) and measures, for every loop that issues MFMAs, how many MFMAs the wave
issues between each global load and the `s_waitcnt vmcnt` that retires it
(vector-memory counters retire in issue order), and whether the loop touches
scratch.
"""
from __future__ import annotations

import re
import subprocess
import sys
from dataclasses import dataclass
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "sdvk_amd" / "csrc"
sys.path.insert(0, str(ROOT))


@dataclass
class Loop:
    kernel: str          # mangled name
    label: str
    instructions: int
    mfma: int
    loads: int
    scratch: int
    distances: list      # MFMAs issued between a load and the wait that retires it (steady state)

    @property
    def min_distance(self) -> int | None:
        return min(self.distances) if self.distances else None


def compile_asm(source: str, out: Path) -> Path:
    """gfx950 assembly of one product source, built with the product's flags."""
    from sdvk_amd import build as b

    flags = [f for f in b.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [b.hipcc(), *flags, *b.EXTRA_FLAGS.get(source, []), "--cuda-device-only", "-S", f"-I{ROOT / 'include'}",
           f"-I{CSRC}", str(CSRC / source), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S {source} failed:\n{r.stderr[-3000:]}")
    return out


def _is_load(ins: str) -> bool:
    return ins.startswith(("buffer_load", "global_load", "scratch_load", "flat_load"))


@dataclass
class _Block:
    label: str
    header: bool
    ins: list
    succ: list


def _blocks(body: list) -> list:
    """Basic blocks of one function's assembly: a block starts at a label or
    after a branch; its successors are the branch target and, unless it ends
    in an unconditional branch or s_endpgm, the next block."""
    out = [_Block("", False, [], [])]
    for line in body:
        x = line.strip()
        lab = re.match(r"^(\.LBB\w+):", x)
        if lab:
            out.append(_Block(lab.group(1), "Loop Header" in line, [], []))
            continue
        if not x or x.startswith((";", ".")):
            continue
        out[-1].ins.append(x)
        if re.match(r"s_c?branch", x) or x.startswith("s_endpgm"):
            out.append(_Block("", False, [], []))
    index = {b.label: i for i, b in enumerate(out) if b.label}
    for i, b in enumerate(out):
        last = b.ins[-1] if b.ins else ""
        br = re.match(r"s_(c?)branch\w*\s+(\.LBB\w+)", last)
        if br and br.group(2) in index:
            b.succ.append(index[br.group(2)])
        if not (last.startswith("s_endpgm") or (br and not br.group(1))) and i + 1 < len(out):
            b.succ.append(i + 1)
    return out


def _natural_loop(blocks: list, h: int) -> set:
    reach, todo = set(), [h]
    while todo:  # blocks reachable from the header
        b = todo.pop()
        for t in blocks[b].succ:
            if t not in reach:
                reach.add(t)
                todo.append(t)
    loop = {h}
    todo = [b for b in reach if h in blocks[b].succ]
    while todo:  # back from the latches to the header
        b = todo.pop()
        if b in loop:
            continue
        loop.add(b)
        todo += [p for p in range(len(blocks)) if b in blocks[p].succ and p in reach and p not in loop]
    return loop


def loops(asm_path: Path) -> list[Loop]:
    """Every loop (LLVM's 'Loop Header' blocks and the blocks of their natural
    loop) that issues MFMAs."""
    text = asm_path.read_text()
    found = []
    for part in re.split(r"\n(?=_Z\S+:\s*; @)", text):
        m = re.match(r"(_Z\S+):", part)
        if not m:
            continue
        blocks = _blocks(part.split(".Lfunc_end")[0].split("\n"))
        for h, blk in enumerate(blocks):
            if not blk.header:
                continue
            label = blk.label
            # the natural loop: the header and every block that reaches one of
            # its back edges without passing the header (the compiler may place
            # the latch blocks above the header), in layout order
            ins = [x for b in sorted(_natural_loop(blocks, h)) for x in blocks[b].ins]
            nm = sum("v_mfma" in x for x in ins)
            if nm == 0:
                continue
            # two passes over the body: the second one is the steady state
            outstanding, mf, dist = [], 0, []
            for k, x in enumerate(ins + ins):
                if _is_load(x):
                    outstanding.append(mf)
                elif "v_mfma" in x:
                    mf += 1
                else:
                    w = re.search(r"vmcnt\((\d+)\)", x)
                    if w:
                        while len(outstanding) > int(w.group(1)):
                            issued = outstanding.pop(0)
                            if k >= len(ins):
                                dist.append(mf - issued)
            found.append(Loop(m.group(1), label, len(ins), nm, sum(_is_load(x) for x in ins),
                              sum("scratch_" in x for x in ins), dist))
    return found


@dataclass
class Resources:
    kernel: str          # mangled name
    vgpr: int            # arch VGPRs
    agpr: int            # accumulation VGPRs
    sgpr: int
    lds: int             # static LDS bytes per workgroup
    scratch: int         # private segment bytes per work-item
    vgpr_spills: int
    sgpr_spills: int
    max_threads: int     # launch bound (work-items per workgroup)

    @property
    def waves_per_simd(self) -> int:
        """Waves of this kernel one SIMD can hold by registers: 512 unified
        registers per lane, allocated in granules of 8 (the metadata's
        vgpr_count already includes the AGPRs)."""
        used = max(8, -(-self.vgpr // 8) * 8)
        return min(8, 512 // used)


def resources(asm_path: Path) -> list[Resources]:
    """Register, LDS and scratch use of every kernel, from the code object's
    metadata (the amdhsa.kernels list of .amdgpu_metadata)."""
    import yaml

    text = asm_path.read_text()
    meta = text.split("\n\t.amdgpu_metadata", 1)[1].split("\n\t.end_amdgpu_metadata", 1)[0]
    doc = yaml.safe_load(meta.split("---", 1)[1].split("\n...", 1)[0])
    out = []
    for k in doc["amdhsa.kernels"]:
        out.append(Resources(kernel=k[".name"], vgpr=k[".vgpr_count"], agpr=k.get(".agpr_count", 0),
                             sgpr=k[".sgpr_count"], lds=k[".group_segment_fixed_size"],
                             scratch=k[".private_segment_fixed_size"], vgpr_spills=k.get(".vgpr_spill_count", 0),
                             sgpr_spills=k.get(".sgpr_spill_count", 0),
                             max_threads=k.get(".max_flat_workgroup_size", 1024)))
    return out
