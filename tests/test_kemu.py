"""CPU checks of the HIP kernels on the kernel emulator (tests/kemu).

The product's .hip sources are compiled for the host against an emulation of
the gfx950 builtins they use (wave-wide MFMA / DPP / transposing LDS reads as
64-lane rendezvous, range-checked buffer resources, LDS filled with NaN
before every workgroup, deferred asynchronous copies) and called through the
same C-ABI. Every case compares with the CPU oracle to the GPU tests' bar,
checks that nothing outside the logical output changed, runs on buffers that
end at a PROT_NONE page (an out-of-bounds access faults and names the
kernel, workgroup and work-item), and runs under two schedules: one
wave operation per wave per pass, and wave-major with lanes and waves
reversed, so a missing barrier changes the result under one of them.

This is where paths are checked before they reach a GPU (the NN GEMM, the
cached-K/V block, the GGUF uploads, the fused GEGLU / residual epilogues). The "fullsize" family runs every
kernel build the benchmark launches at the benchmark's own shapes, with a
few workgroups emulated per launch (the first and the bottom-right tile,
every K split of them): grids, split choices and offsets are those of the
GPU run, and the written tiles are compared with the oracle's rows (the
config-4 block at full size is a bounds check only);
it does not measure anything and nothing in the product loads the emulation
build. test_emulator_catches_planted_faults pins the checker itself: copies
of the sources with one planted mistake each (compiled for the host only)
must fail.
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
KEMU = HERE / "kemu"
ROOT = HERE.parent
CSRC = ROOT / "sdvk_amd" / "csrc"
BOTH = [0, 7]  # interleaved; wave-major with lanes and waves reversed

FAMILIES = {
    # LDS-tiled kernel through the shape rules (choose), every tile config,
    # K splits, the general-K path, both weight layouts, batch / strides
    "gemm_lds": [
        dict(M=1, N=1, K=32), dict(M=77, N=96, K=64), dict(M=100, N=100, K=96),
        dict(M=130, N=257, K=320), dict(M=130, N=257, K=320, mode=1), dict(M=154, N=96, K=2048),
        dict(M=60, N=40, K=100, layout="split"), dict(M=77, N=96, K=64, layout="split", mode=1),
        dict(M=300, N=300, K=256, cfg="0"), dict(M=300, N=200, K=256, cfg="1", layout="split"),
        # K splits (partials in the workspace, fixed-order reduce): 16-byte reduce with an unaligned
        # bias, the scalar reduce (N % 4 != 0), mode 1; the same shape without a workspace (no split)
        dict(M=154, N=96, K=2048, bias_off=1), dict(M=154, N=98, K=2048, mode=0),
        dict(M=154, N=96, K=2048, mode=1), dict(M=154, N=96, K=2048, ws=False),
        # the any-K kernel (split layout): K % 4 != 0, an A only 4-byte aligned, modes 1 / 2
        dict(M=70, N=50, K=37, layout="split"), dict(M=100, N=100, K=96, layout="split", a_off=1),
        dict(M=65, N=33, K=70, layout="split", mode=1, lda=75), dict(M=65, N=33, K=5, layout="split", mode=2),
        dict(M=130, N=100, K=128, cfg="2"), dict(M=70, N=70, K=128, cfg="3", front=True),
        dict(M=300, N=300, K=256, cfg="4"), dict(M=200, N=300, K=512, cfg="0:3"),
        dict(M=70, N=36, K=64, batch=3, lda=72, ldc=40, sA=5200, sC=3000),
        dict(M=70, N=36, K=128, batch=2, lda=132, ldc=40, sA=9300, sC=3000, cfg="4:2", mode=1),
        # 192x256 (8 waves of 96x64)
        dict(M=400, N=300, K=256, cfg="5"), dict(M=200, N=260, K=320, cfg="5:2", layout="split", mode=1),
        # more K splits: many splits of one tile, batch items with strides, mode 2 (the residual op)
        dict(M=64, N=64, K=2048, cfg="3:16"), dict(M=70, N=36, K=512, batch=3, lda=520, ldc=40, sA=37000,
                                                   sC=3000, cfg="3:4", mode=1),
        dict(M=130, N=200, K=512, cfg="1:3", mode=2), dict(M=200, N=300, K=640, cfg="5:3", front=True),
        # 128x128 as 8 waves of 32x64: partial tiles, a K split, the split layout
        dict(M=300, N=300, K=640, cfg="6"), dict(M=130, N=200, K=512, cfg="6:2", mode=1),
        dict(M=200, N=260, K=320, cfg="6", layout="split", mode=2, front=True),
    ],
    # fused epilogues: residual mode 2 (C += A W^T + bias) and the GEGLU GEMM
    "gemm_fused": [
        dict(case="gemm_nt", M=77, N=96, K=64, mode=2), dict(case="gemm_nt", M=130, N=257, K=320, mode=2),
        dict(case="gemm_nt", M=300, N=200, K=256, cfg="0:2", mode=2, layout="split"),
        dict(case="gemm_nt", M=60, N=40, K=100, layout="split", mode=2),
        dict(case="gemm_nt", M=154, N=96, K=2048, mode=2, bias_off=1),  # K splits: 16-byte bias add, unaligned bias
        dict(case="gemm_geglu", M=77, F=48, K=64), dict(case="gemm_geglu", M=300, F=200, K=256, cfg="4"),
        dict(case="gemm_geglu", M=130, F=100, K=96), dict(case="gemm_geglu", M=300, F=130, K=256, cfg="0", ldg=136),
        dict(case="gemm_geglu", M=260, F=96, K=128, cfg="2", front=True),
        dict(case="gemm_geglu", M=70, F=40, K=128, cfg="1", bias=False),
        dict(case="gemm_nt", M=200, N=300, K=256, cfg="1:2", mode=2), dict(case="gemm_geglu", M=200, F=260, K=128, cfg="3"),
        dict(case="gemm_geglu", M=200, F=130, K=128, cfg="5"), dict(case="gemm_nt", M=200, N=300, K=256, cfg="5:2", mode=2),
        # fp16 activations: the fp16-A GEMM equals the fp32 GEMM on the same values (tiles, K splits, modes)
        dict(case="gemm_f16a", M=77, N=96, K=64), dict(case="gemm_f16a", M=154, N=96, K=2048, mode=2),
        dict(case="gemm_f16a", M=300, N=200, K=256, cfg="0", mode=1), dict(case="gemm_f16a", M=400, N=300, K=256, cfg="5"),
        dict(case="gemm_f16a", M=130, N=100, K=96, front=True),
        # fp16 output (the block's fp16 Q / K / V): the rounding of the fp32 GEMM's result, padded rows
        dict(case="gemm_f16o", M=77, N=96, K=64), dict(case="gemm_f16o", M=300, N=260, K=256, cfg="5", ldc=264),
        dict(case="gemm_f16o", M=130, N=98, K=320, front=True),
        dict(case="gemm_geglu", M=200, F=130, K=128, cfg="6"), dict(case="gemm_f16a", M=300, N=200, K=256, cfg="6"),
        dict(case="gemm_f16o", M=300, N=260, K=256, cfg="6", ldc=264), dict(case="gemm_nt", M=260, N=300, K=256, cfg="6", mode=2),
    ],
    "gemm_nn": [
        dict(M=64, N=64, K=32), dict(M=100, N=72, K=96), dict(M=130, N=260, K=100, mode=1),
        dict(M=60, N=36, K=44, batch=3, lda=48, ldb=40, ldc=44, sA=3000, sB=1800, sC=2800),
        dict(M=5, N=4, K=4), dict(M=64, N=64, K=0), dict(M=64, N=64, K=0, mode=1),
        dict(M=33, N=68, K=36, front=True),
        # tiled kernel (K % 64 == 0, lda / sA multiples of 16): edges, K splits (mode 0 / 1), batch / strides
        dict(M=130, N=260, K=128), dict(M=300, N=520, K=640, mode=1), dict(M=64, N=64, K=1024),
        dict(M=70, N=36, K=256, batch=3, lda=272, ldb=40, ldc=44, sA=19056, sB=10248, sC=3100),
        dict(M=129, N=300, K=256, front=True), dict(M=130, N=260, K=128, kernel="general"),
        dict(M=129, N=300, K=256, ldc=302),  # K splits, ldc % 4 != 0: the scalar reduce pass
        dict(M=300, N=520, K=640, mode=1, ws=False),  # no workspace: no split
    ],
    "attention": [
        dict(Tq=100, Tk=300, C=128, heads=2), dict(Tq=100, Tk=300, C=128, heads=2, causal=True),
        dict(Tq=1, Tk=1, C=64, heads=1), dict(Tq=50, Tk=100, C=40, heads=1),
        dict(batch=2, Tq=70, Tk=77, C=640, heads=10, f16_in=True, f16_out=True, kv_len=[77, 40]),
        dict(batch=2, Tq=130, Tk=200, C=128, heads=2, f16_in=True, f16_out=True, causal=True),
        dict(batch=2, Tq=33, Tk=70, C=320, heads=5, f16_in=True, f16_out=False, kv_len=[1, 70]),
        # the 4-wave fp16 kernel (chosen for large grids) on small shapes
        dict(batch=2, Tq=200, Tk=300, C=128, heads=2, f16_in=True, f16_out=True, causal=True, nw=4),
        dict(batch=2, Tq=130, Tk=77, C=640, heads=10, f16_in=True, f16_out=False, kv_len=[77, 13], nw=4),
        # one far-outlying key per tile, in either lane half of a query (the running max spans both)
        dict(Tq=64, Tk=192, C=128, heads=2, f16_in=True, outliers=[5, 66, 134]),
        dict(Tq=64, Tk=192, C=128, heads=2, outliers=[5, 66, 134]),
        # output stores straight from the MFMA layout (the path for rows not 16-byte aligned), both kernels
        dict(batch=2, Tq=70, Tk=77, C=640, heads=10, f16_in=True, f16_out=True, kv_len=[77, 40], direct_store=True),
        dict(Tq=100, Tk=300, C=128, heads=2, causal=True, direct_store=True),
        # key-split plans (mi_fused_attention_ws, forced): pieces of uneven tile counts, a partial query
        # block, hd = 40, fp16 / fp32 output, an outlying key inside one piece
        dict(batch=1, Tq=256, Tk=512, C=128, heads=2, f16_in=True, f16_out=True, split="2:4", nw=4),
        dict(batch=2, Tq=300, Tk=1000, C=128, heads=2, f16_in=True, f16_out=False, split="3:3", nw=4),
        dict(Tq=200, Tk=130, C=80, heads=2, f16_in=True, f16_out=False, split="1:2", nw=4),
        dict(Tq=128, Tk=256, C=64, heads=1, f16_in=True, split="1:4", nw=4, outliers=[5, 70, 200]),
        # MI_ATTN_PREC_SPLIT (P's fp16 residual on every tile), held to a tenth of the bar: both kernels,
        # key padding, causal, a forced key split; MI_ATTN_PREC_AUTO picks it for fp32 outputs
        dict(Tq=130, Tk=300, C=128, heads=2, f16_in=True, precision=0, tol=2e-4),
        dict(Tq=100, Tk=150, C=128, heads=2, causal=True, precision=0, tol=2e-4),
        dict(batch=2, Tq=130, Tk=150, C=128, heads=2, f16_in=True, kv_len=[150, 37], nw=4, precise=True, tol=2e-4),
        dict(Tq=100, Tk=300, C=128, heads=2, f16_in=True, causal=True, nw=2, precise=True, tol=2e-4),
        dict(Tq=70, Tk=130, C=128, heads=2, causal=True, precise=True, tol=2e-4),
        dict(Tq=200, Tk=130, C=80, heads=2, f16_in=True, split="1:2", nw=4, precise=True, tol=2e-4),
        # the burst build (three waves per SIMD, picked for grids of more than two workgroups per CU):
        # key padding, partial query and key tiles, hd = 40, a key split, outlying keys, fp32 output
        dict(batch=2, Tq=130, Tk=77, C=640, heads=10, f16_in=True, f16_out=True, kv_len=[77, 13], simd_waves="3"),
        dict(batch=2, Tq=300, Tk=1000, C=128, heads=2, f16_in=True, f16_out=False, split="3:3", simd_waves="3"),
        dict(Tq=200, Tk=130, C=80, heads=2, f16_in=True, f16_out=True, simd_waves="3"),
        dict(Tq=64, Tk=192, C=128, heads=2, f16_in=True, nw=4, outliers=[5, 66, 134], simd_waves="3"),
        dict(Tq=128, Tk=64, C=64, heads=1, f16_in=True, f16_out=True, simd_waves="3"),
    ],
    "block": [
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=160),
        dict(B=2, T=64, C=128, H=2, Tc=77, Cc=256, F=256, masked=True),
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=160, fused=True),
        dict(B=2, T=64, C=128, H=2, Tc=77, Cc=256, F=256, masked=True, fused=True),
        dict(B=2, T=64, C=128, H=2, Tc=77, Cc=256, F=256, masked=True, qkv_joint=True),
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=160, qkv_joint=True, fused=True),
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=64, qkv_joint=True),
        dict(B=2, T=64, C=128, H=2, Tc=77, Cc=256, F=256, masked=True, half=True),
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=160, qkv_joint=True, fused=True, half=True),
        # fp16 attention inputs: against the oracle, and the other flags bit for bit against the flag alone
        dict(B=2, T=64, C=128, H=2, Tc=77, Cc=256, F=256, masked=True, hattn=True),
        dict(B=1, T=33, C=64, H=1, Tc=5, Cc=96, F=160, qkv_joint=True, fused=True, half=True, hattn=True),
    ],
    "gguf_upload": [dict()],
    "q8": [dict(n=32), dict(n=4096), dict(n=224, front=True)],
    "glue": [dict(rows=9, d=1280), dict(rows=3, d=37, affine=False), dict(rows=1, d=4, affine=False),
             dict(rows=5, d=4096, front=True)],
}
CASE_OF = {"gemm_lds": "gemm_nt"}


def _fullsize() -> list[dict]:
    """The benchmark's shapes at full size with sampled workgroups (cases.py
    gemm_full / gemm_nn_full / attention_full): every GEMM shape through the
    tile rules, every build of the benchmark's GEMM candidate sweep (shapes in
    rotation; the 192-row build also on the widest-output and the deepest-K
    shape), the NN GEMM at the SDXL conv shapes, and every attention
    shape with the default and both pinned workgroup sizes."""
    sys.path.insert(0, str(ROOT))
    import bench
    g = [(M, N, K) for _, M, N, K in bench.GEMM_SHAPES + [bench.CONFIG0]]
    specs = [dict(case="gemm_full", M=M, N=N, K=K) for M, N, K in g]
    specs.append(dict(case="gemm_full", M=9216, N=1280, K=1280, layout="split"))
    for i, cfg in enumerate(bench.GEMM_CANDIDATES):
        M, N, K = g[i % len(g)]
        specs.append(dict(case="gemm_full", M=M, N=N, K=K, cfg=cfg))
    for cfg in ("5",):
        for M, N, K in ((8192, 5120, 640), (2048, 1280, 5120)):
            specs.append(dict(case="gemm_full", M=M, N=N, K=K, cfg=cfg))
    specs += [dict(case="gemm_nn_full", M=M, N=N, K=K) for _, M, N, K in bench.NN_SHAPES]
    for _, b, h, tq, tk, masked in bench.ATTN_SHAPES:
        for nw in (None, 2, 4):
            specs.append(dict(case="attention_full", batch=b, Tq=tq, Tk=tk, C=64 * h, heads=h, masked=masked, nw=nw))
    # the config-4 block: bounds only (first / last workgroups of every launch)
    specs += [dict(case="block_full"), dict(case="block_full", cached=True),
              dict(case="block_full", fused=True, qkv_joint=True),
              dict(case="block_full", fused=True, qkv_joint=True, half=True, hattn=True, cached=True)]
    unique = {json.dumps(s, sort_keys=True): s for s in specs}
    return list(unique.values())


FAMILIES["fullsize"] = _fullsize()
SCHEDULES = {"fullsize": [0]}  # the barrier-sensitive schedules run at the small shapes above


def _workers() -> int:
    return max(1, min(8, os.cpu_count() or 1))


def _run(spec: dict, env: dict | None = None, timeout: int = 600) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(KEMU / "cases.py"), json.dumps(spec)], capture_output=True, text=True,
                          timeout=timeout, env=env, cwd=str(ROOT))


@pytest.fixture(scope="module")
def emulator():
    if not Path(os.environ.get("KEMU_CXX", "/opt/rocm/llvm/bin/clang++")).exists():
        pytest.skip("no host clang++ for the emulation build")
    sys.path.insert(0, str(KEMU))
    import kemu_build
    from oracle import binding as ob
    ob.build()
    return kemu_build.build()


@pytest.mark.parametrize("family", list(FAMILIES))
def test_kernels_on_emulator(emulator, family):
    sched = SCHEDULES.get(family, BOTH)
    specs = [dict({"case": CASE_OF.get(family, family)}, schedules=sched, **s) for s in FAMILIES[family]]
    with ThreadPoolExecutor(_workers()) as ex:
        results = list(ex.map(_run, specs))
    failed = []
    for spec, r in zip(specs, results):
        ok = r.returncode == 0 and r.stdout.count("OK ") == len(sched)
        print(f"{json.dumps(spec)}: {r.stdout.strip() if ok else 'FAILED'}")
        if not ok:
            failed.append(f"{json.dumps(spec)}\n{(r.stdout + r.stderr).strip()[-1500:]}")
    assert not failed, "\n\n".join(failed)


# The tile rules at the SDXL shapes of the benchmark: (op, dims, grid, work-items
# per workgroup). GEMM (choose in gemm_q8.hip): 192x256 (8 waves) when that gives
# >= 120 tiles and K >= 1280 (256x128, 8 waves, when both give under one round
# and 256x128 more tiles); 128x128 (4 waves) when that gives >= 160 tiles,
# as 8 waves of 32x64 when those are fewer than 256 and K is not split; else
# 64x64 (4 waves). Grid = (tiles, splits, batch). With a workspace
# ("gemm_ws"): 128x128 grids under 256 tiles with K >= 4096 run 256x128 tiles (8
# waves) with K split into the most parts (>= 1024 k each) with tiles x parts <= 256, 64x64
# grids under 512 tiles split K (powers of two) to about 256 workgroups with
# >= 128 k per split. NN GEMM: 128x256 tiles (8 waves), grid (N tiles, M tiles,
# splits); with a workspace ("nn_ws") the most K splits with tiles x splits <= 256
# and each split keeps >= 4 steps of 64. fp16 attention: 4-wave workgroups of
# 128 queries, 2-wave ones of 64 when Tq <= 64.
ROUTING = [
    ["gemm", [8192, 640, 640], [160, 1, 1], 512], ["gemm", [8192, 5120, 640], [1280, 1, 1], 512],
    ["gemm", [8192, 640, 2560], [160, 1, 1], 512], ["gemm", [2048, 1280, 1280], [160, 1, 1], 512],
    ["gemm", [2048, 10240, 1280], [440, 1, 1], 512], ["gemm", [2048, 1280, 5120], [160, 1, 1], 512],
    ["gemm_ws", [2048, 1280, 5120], [80, 3, 1], 512],
    ["gemm", [154, 640, 2048], [30, 1, 1], 256], ["gemm_ws", [154, 640, 2048], [30, 8, 1], 256],
    ["gemm", [154, 1280, 2048], [60, 1, 1], 256], ["gemm_ws", [154, 1280, 2048], [60, 4, 1], 256],
    ["gemm", [9216, 1280, 1280], [240, 1, 1], 512], ["gemm_ws", [9216, 1280, 1280], [240, 1, 1], 512],
    ["gemm", [2048, 3840, 1280], [240, 1, 1], 512],  # the block's joint Q/K/V: 256x128 tiles
    ["nn_ws", [320, 4096, 2880], [16, 3, 5], 512], ["nn_ws", [640, 4096, 5760], [16, 5, 3], 512],
    ["nn_ws", [1280, 1024, 11520], [4, 10, 6], 512], ["nn_ws", [1280, 1024, 640], [4, 10, 2], 512],
    ["nn", [1280, 1024, 11520], [4, 10, 1], 512],
    ["attn", [2, 10, 4096, 4096], [640, 1, 1], 256], ["attn", [2, 20, 1024, 1024], [320, 1, 1], 256],
    ["attn", [2, 10, 4096, 77], [640, 1, 1], 256], ["attn", [2, 20, 1024, 77], [320, 1, 1], 256],
]


def test_routing_at_sdxl_shapes(emulator):
    r = _run({"case": "routing", "table": ROUTING})
    assert r.returncode == 0 and "OK routing" in r.stdout, (r.stdout + r.stderr)[-3000:]


# One planted mistake per copy of the sources: (file, text, replacement, case).
PLANTED = {
    # the LDS kernel's barrier between a step's MFMAs / store phase and the next step removed
    "missing_barrier": ("gemm_q8.hip",
                        "            __syncthreads();\n            load_step(phys(min(j + 3, last)), S1{});",
                        "            load_step(phys(min(j + 3, last)), S1{});",
                        dict(case="gemm_nt", M=300, N=200, K=256, cfg="6")),
    # ping-pong loop (builds 0 and 5): a wave group reads the stage it has just written before the
    # barrier that orders every wave's writes (the barrier count kept)
    "missing_barrier_pingpong": ("gemm_q8.hip",
                                 "                mem(min(j + 2, last), S0{}, S1{});\n                __syncthreads();\n"
                                 "                comp(S1{});\n                __syncthreads();\n",
                                 "                mem(min(j + 2, last), S0{}, S1{});\n"
                                 "                comp(S1{});\n                __syncthreads();\n                __syncthreads();\n",
                                 dict(case="gemm_nt", M=300, N=300, K=640, cfg="5")),
    # staged epilogue without the wave barrier between its LDS writes and reads
    "missing_wave_barrier": ("gemm_q8.hip", "__builtin_amdgcn_wave_barrier();", "",
                             dict(case="gemm_nt", M=77, N=96, K=64)),
    # NN GEMM weight rows past M read through a plain pointer (out of bounds)
    "oob_read": ("gemm_nn_q8.hip", "if (wm_row < a.M && k < a.K) {", "if (k < a.K) {",
                 dict(case="gemm_nn", M=60, N=64, K=32)),
    # tiled NN GEMM: B's 4 x 4 register transpose taken the wrong way round
    "nn_transpose": ("gemm_nn_q8.hip", "static_cast<_Float16>(braw[rs][p][1][e])",
                     "static_cast<_Float16>(braw[rs][p][e][1])", dict(case="gemm_nn", M=130, N=260, K=128)),
    # tiled NN GEMM: the barrier between storing stage 1 and reading it removed
    "nn_missing_barrier": ("gemm_nn_q8.hip",
                           "        __syncthreads();\n        load(min(s_begin + j + 3, last), S1{});",
                           "        load(min(s_begin + j + 3, last), S1{});",
                           dict(case="gemm_nn", M=130, N=260, K=256)),
    # fp16 attention: the vmcnt wait for the iteration's K / V DMA removed before the barrier
    "attn_dma_wait": ("attention.hip", "            dma_wait();\n            __syncthreads();\n        };",
                      "            __syncthreads();\n        };",
                      dict(case="attention", batch=2, Tq=130, Tk=200, C=128, heads=2, f16_in=True, f16_out=True)),
    # the burst attention loop without its wait for the iteration's K / V DMA before the barrier
    "attn_burst_dma_wait": ("attention.hip",
                            "            for (int t = 0; t < 2; ++t) s0[t] = s1[t];\n            dma_wait();\n",
                            "            for (int t = 0; t < 2; ++t) s0[t] = s1[t];\n",
                            dict(case="attention", batch=2, Tq=130, Tk=200, C=128, heads=2, f16_in=True,
                                 f16_out=True, simd_waves="3")),
    # attention: output rows read back from LDS without the wave barrier after the wave's writes
    "attn_store_wave_barrier": ("attention.hip", "    __builtin_amdgcn_wave_barrier();\n    constexpr int RPI",
                                "    constexpr int RPI",
                                dict(case="attention", batch=2, Tq=130, Tk=77, C=640, heads=10, f16_in=True,
                                     f16_out=False, kv_len=[77, 13], nw=4)),
    # the lane index the 8-wave GEMM epilogue takes from v_mbcnt, off by one
    "lane_id": ("common.hpp", "__builtin_amdgcn_mbcnt_lo(~0u, 0u)", "__builtin_amdgcn_mbcnt_lo(~0u, 1u)",
                dict(case="gemm_nt", M=300, N=300, K=256, cfg="0")),
    # GGUF upload refills a staging buffer without waiting for its last copy
    "staging_reuse": ("gguf.cpp",
                      "    if (g->stage_used[i] && hipEventSynchronize(g->done[i]) != hipSuccess)\n"
                      "        return fail(MI_ERR_HIP, \"%s: staging wait failed\", fn);\n", "",
                      dict(case="gguf_upload", big_rows=2048, big_cols=1280)),
}


def test_emulator_catches_planted_faults(emulator, tmp_path):
    """Each planted mistake makes its case fail (wrong result, a fault or a
    deadlock report); the unmodified sources pass the same cases."""
    def build_and_run(name):
        fname, old, new, spec = PLANTED[name]
        src = tmp_path / name / "src"
        shutil.copytree(CSRC, src)
        text = (src / fname).read_text()
        assert old in text, f"{name}: planting site not found in {fname}"
        text = text.replace(old, new, 1)
        if name == "oob_read":  # a plain-pointer read, so the stray row really leaves the buffer
            text = text.replace("__builtin_amdgcn_raw_buffer_load_b32(rA, fl, 0, 0)",
                                "*reinterpret_cast<const uint32_t*>(a.Aq + fl)", 1)
        (src / fname).write_text(text)
        env = dict(os.environ, KEMU_CSRC=str(src), KEMU_OUT=str(tmp_path / name / "build"))
        r = subprocess.run([sys.executable, str(KEMU / "kemu_build.py")], capture_output=True, text=True, env=env,
                           timeout=900)
        assert r.returncode == 0, r.stderr[-2000:]
        return _run(dict(spec, schedules=BOTH + [4]), env=env)

    with ThreadPoolExecutor(2) as ex:
        results = dict(zip(PLANTED, ex.map(build_and_run, PLANTED)))
    for name, r in results.items():
        print(f"{name}: rc={r.returncode} {(r.stdout + r.stderr).strip().splitlines()[-1][:160]}")
        assert r.returncode != 0, f"planted mistake {name} went unnoticed"
    clean = [dict(PLANTED[n][3], schedules=BOTH + [4]) for n in PLANTED]
    with ThreadPoolExecutor(_workers()) as ex:
        for spec, r in zip(clean, ex.map(_run, clean)):
            assert r.returncode == 0, f"unmodified sources fail {spec}: {r.stderr[-1500:]}"
