"""The compiled K loops keep their software pipelines (CPU: gfx950 assembly of
the product sources, analysed by tests/isa_sched.py).

For every loop that issues MFMAs in the GEMM and attention kernels:
  * no scratch access (a spilled register reloaded inside the loop waits for
    every global load in flight);
  * every global load has at least a quarter of the loop's MFMAs (half a K
    step: the loops run two steps per trip) issued between it and the wait
    that retires it. A load under a branch, or a consumer hoisted next to its
    load, drops this to 0-2 and the wave then sits out the memory latency.
And for every kernel of those sources (test_register_budgets): the 8-wave
builds fit two waves per SIMD, LDS fits the CU, and scratch is used only by
the listed build, within its budget.
Excluded: the attention kernel's scalar-load build (head dims that are not a
multiple of 8, or unaligned tensors; no SDXL shape takes it) and the NN GEMM's
untiled kernel (the general path for unaligned shapes; not pipelined).
"""
from __future__ import annotations

import shutil

import pytest

import isa_sched

CASES = {
    "gemm_q8.hip": ("gemm_q8_kernel",),
    "attention.hip": ("attn_f16_kernel", "attn_kernel"),
    "gemm_nn_q8.hip": ("gemm_nn_q8_tiled_kernel",),
}


def _excluded(kernel: str) -> bool:
    # attn_kernel<TI, TO, VEC = false>: element-wise loads for unaligned inputs
    return "attn_kernel" in kernel and kernel.endswith("Lb0EEEvNS0_8AttnArgsE")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    from sdvk_amd import build as b

    if shutil.which(b.hipcc()) is None:
        pytest.skip("no hipcc for the gfx950 assembly")
    d = tmp_path_factory.mktemp("isa")
    paths = {src: isa_sched.compile_asm(src, d / (src + ".s")) for src in CASES}
    return {src: isa_sched.loops(path) for src, path in paths.items()} | {
        ("resources", src): isa_sched.resources(path) for src, path in paths.items()}


@pytest.mark.parametrize("src", list(CASES))
def test_k_loops_keep_loads_ahead_of_their_waits(asm, src):
    loops = [l for l in asm[src] if any(k in l.kernel for k in CASES[src]) and not _excluded(l.kernel)]
    assert loops, f"no MFMA loops found in {src}"
    bad = []
    for l in loops:
        need = max(1, l.mfma // 4)
        if l.scratch:
            bad.append(f"{l.kernel} {l.label}: {l.scratch} scratch accesses in the loop")
        if l.loads and (l.min_distance is None or l.min_distance < need):
            bad.append(f"{l.kernel} {l.label}: a load is waited for {l.min_distance} MFMAs after issue "
                       f"(loop of {l.mfma} MFMAs; want >= {need})")
    print(f"{src}: {len(loops)} loops checked")
    assert not bad, "\n".join(bad)


# Kernels that may keep values in scratch around (never inside) their K loop,
# and how many bytes per lane: the 8-wave 256x256 LDS build at its 256-register
# limit (epilogue indices across the loop); the burst attention build at its
# 168-register limit (three waves per SIMD; prologue values across the loop).
SCRATCH_ALLOWED = {"gemm_q8_kernelILi256ELi256ELi4ELi2E": 16, "attn_f16_kernelIDF16_Li4ELi0ELi1E": 24,
                   "attn_f16_kernelIfLi4ELi0ELi1E": 24}
# Builds that must hold three waves per SIMD (their purpose).
THREE_WAVES = ("attn_f16_kernelIDF16_Li4ELi0ELi1E", "attn_f16_kernelIfLi4ELi0ELi1E")


@pytest.mark.parametrize("src", list(CASES))
def test_register_budgets(asm, src):
    """Every 8-wave (512-thread) build fits two waves per SIMD, the burst
    attention build three, every kernel's LDS fits the CU, and scratch appears
    only where listed, within its budget."""
    res = asm[("resources", src)]
    assert res, f"no kernels in {src}"
    bad = []
    for r in res:
        allowed = max([v for k, v in SCRATCH_ALLOWED.items() if k in r.kernel], default=0)
        if r.scratch > allowed:
            bad.append(f"{r.kernel}: {r.scratch} B of scratch per lane (allowed {allowed})")
        if r.lds > 160 * 1024:
            bad.append(f"{r.kernel}: {r.lds} B of LDS")
        if r.max_threads == 512 and r.waves_per_simd < 2:
            bad.append(f"{r.kernel}: {r.vgpr} registers, under two waves per SIMD")
        if any(k in r.kernel for k in THREE_WAVES) and r.waves_per_simd < 3:
            bad.append(f"{r.kernel}: {r.vgpr} registers, under three waves per SIMD")
    print(f"{src}: {len(res)} kernels checked")
    assert not bad, "\n".join(bad)
