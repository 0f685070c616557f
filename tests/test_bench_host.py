"""bench.py's host logic on the CPU, over a stand-in device layer.

No GPU here, so the bench's own Python (case set-up, the timed loop's event
bookkeeping, the roofline / breakdown / block-stack / extras assembly and the
JSON line) would otherwise first run at the end of a round. The stand-in
`hip` hands out fake device addresses and fixed event times; every `ops` call
is bound against the real `sdvk_amd.ops` signature, so a wrong argument name
or count fails here. Nothing is computed.
"""
from __future__ import annotations

import inspect
import json
import os
import sys
import types
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


class _Buf:
    _next = 1 << 32

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.value = _Buf._next
        _Buf._next += (self.nbytes + 255) // 256 * 256 + 256

    @classmethod
    def from_array(cls, a):
        return cls(np.asarray(a).nbytes)

    def fill_zero(self, stream=None):
        pass

    def copy_from(self, src, nbytes, stream=None):
        assert nbytes <= self.nbytes

    def upload(self, a, offset=0):
        pass

    def download(self, dtype, count):
        return np.zeros(count, dtype=dtype)


class _Stream:
    def synchronize(self):
        pass


class _Event:
    t = 0.0

    def __init__(self, flags=0):
        self.at = None

    def record(self, stream=None):
        _Event.t += 0.25
        self.at = _Event.t

    def synchronize(self):
        pass

    def elapsed_ms(self, end):
        assert self.at is not None and end.at is not None
        return end.at - self.at


class _Graph:
    def __init__(self, stream):
        self.stream = stream

    def begin(self):
        pass

    def end(self):
        pass

    def launch(self):
        pass


def _fake_hip():
    m = types.SimpleNamespace(DeviceBuffer=_Buf, Stream=_Stream, Event=_Event, Graph=_Graph, device_count=lambda: 1,
                              device_name=lambda d=0: "stand-in", synchronize=lambda: None)
    return m


def _fake_ops(calls):
    from sdvk_amd import ops as real

    def wrap(name):
        sig = inspect.signature(getattr(real, name))

        def f(*a, **k):
            sig.bind(*a, **k)
            calls.append(name)
            if name in ("block_workspace_bytes", "block_ctx_kv_bytes"):
                return 1 << 20
            if name in ("gemm_workspace_bytes", "gemm_nn_workspace_bytes", "fused_attention_ws_bytes"):
                return 1 << 16
            return None
        return f

    names = [n for n, v in vars(real).items() if inspect.isfunction(v) and v.__module__ == real.__name__]
    ns = {n: wrap(n) for n in names}
    ns.update(BlockDims=real.BlockDims, BlockWeights=real.BlockWeights)
    ns.update({k: v for k, v in vars(real).items() if k.startswith("MI_")})

    class _Tuning:  # the context-manager form of tuning_set
        def __init__(self, **over):
            self.over = over

        def __enter__(self):
            for k, v in self.over.items():
                ns["tuning_set"](k, v)
            return self

        def __exit__(self, *exc):
            for k in self.over:
                ns["tuning_set"](k, None)
            return False

    ns["tuning"] = _Tuning
    return types.SimpleNamespace(**ns)


@pytest.fixture
def fake_device(monkeypatch):
    import sdvk_amd
    from sdvk_amd import _lib

    calls = []
    monkeypatch.setattr(sdvk_amd, "hip", _fake_hip(), raising=False)
    monkeypatch.setattr(sdvk_amd, "ops", _fake_ops(calls), raising=False)
    monkeypatch.setattr(_lib, "load", lambda: None)
    return calls


@pytest.mark.parametrize("launch", [None, "graph"])
def test_bench_line_on_stand_in_device(fake_device, monkeypatch, capsys, launch):
    import bench

    # the extras child runs in-process here (same code path, no subprocess)
    def child(reps, timeout_s=420):
        from sdvk_amd import hip, ops
        return bench.extras(np.random.default_rng(2), hip, ops, hip.Stream(), reps)

    monkeypatch.setattr(bench, "run_extras_child", child)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "2", "--warmup", "1", "--reps", "2",
                                      "--no-cpu-baseline"] + (["--launch", launch] if launch else []))
    assert bench.main() == 0
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("{")]
    assert len(lines) == 1
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["value"] > 0
    if launch == "graph":  # graph replays, checked against an eager pass
        assert out["config"]["launch"].startswith("one HIP graph per kernel family")
        assert out["config"]["launch_check"] == "graph replay outputs bitwise equal to an eager pass"
    else:  # the default
        assert out["config"]["launch"].startswith("eager") and out["config"]["launch_check"] is None
    r = out["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and 0 < r["frac"] == pytest.approx(r["achieved"] / r["peak"],
                                                                                            rel=1e-3)
    assert len(out["breakdown"]) == len(bench.GEMM_SHAPES) + len(bench.ATTN_SHAPES)
    assert out["block_stack"]["blocks"] == 10
    assert out["block_stack"]["variant"] == {"cached_kv": True, "fused_epilogues": True, "joint_qkv": True,
                                             "fp16_activations": True, "fp16_attention": True}
    ks = out["block_stack"]["kernel_share"]
    assert "error" not in ks, ks
    assert set(ks["us_per_block"]) == {"gemm_q8", "attention", "glue"}
    assert ks["hot_kernels_share"] == pytest.approx(ks["share"]["gemm_q8"] + ks["share"]["attention"], abs=2e-4)
    ex = out["extras"]
    for part in ("config0_gemm", "nn_gemm", "block_stack_plain", "block_stack_cached_kv",
                 "block_stack_fused_epilogues", "block_stack_joint_qkv", "block_stack_fp16_activations",
                 "block_stack_all_but_fp16_activations", "block_stack_fp16_attention",
                 "block_stack_all_but_fp16_attention", "gemm_candidates", "attention_candidates", "step_graph"):
        assert part in ex and "error" not in ex[part], (part, ex.get(part))
    assert set(ex["gemm_candidates"]["us"]) == set(bench.GEMM_CANDIDATES) | {"default"}
    assert len(ex["gemm_candidates"]["default_us"]) == len(bench.GEMM_SHAPES) + 1
    assert set(ex["attention_candidates"]["us"]) == {"default", "nw2", "nw4", "simd2", "simd3", "nosplit"}
    assert len(ex["gemm_candidates"]["best"]) == len(bench.GEMM_SHAPES) + 1
    assert ex["block_stack_plain"]["variant"] == {"cached_kv": False, "fused_epilogues": False, "joint_qkv": False,
                                                  "fp16_activations": False, "fp16_attention": False}
    for name in ("gemm_nt_q8_0", "fused_attention_ws", "gemm_nn_q8", "sdxl_block_forward", "block_ctx_kv",
                 "sdxl_block_forward_kv", "q8_0_quantize", "gemm_nt_q8_0_f16o"):
        assert name in fake_device, name


def test_extras_emit_partial_results(fake_device):
    """Every emitted line is a growing prefix of the final extras (so a child
    stopped early leaves what it measured), one line per GEMM candidate build."""
    import bench
    from sdvk_amd import hip, ops

    seen = []
    final = bench.extras(np.random.default_rng(2), hip, ops, hip.Stream(), 2, emit=lambda o: seen.append(json.dumps(o)))
    emitted = [json.loads(x) for x in seen]
    assert len(emitted) >= len(bench.GEMM_CANDIDATES) + 9
    for a, b in zip(emitted, emitted[1:]):
        assert set(a) <= set(b)
    assert emitted[-1] == json.loads(json.dumps(final))
    cand = [e["gemm_candidates"] for e in emitted if "gemm_candidates" in e]
    assert [len(c["us"]) for c in cand[:3]] == [1, 2, 3]


@pytest.mark.parametrize("how", ["timeout", "crash", "ok"])
def test_extras_child_keeps_the_last_complete_line(monkeypatch, how):
    import subprocess

    import bench

    partial = '{"config0_gemm": {"us": 1.0}}\n{"config0_gemm": {"us": 1.0}, "nn_gemm": []}\n{"trunc'

    def fake_run(cmd, **kw):
        assert "--extras-child" in cmd
        if how == "timeout":
            raise subprocess.TimeoutExpired(cmd, kw["timeout"], output=partial.encode())
        return subprocess.CompletedProcess(cmd, 0 if how == "ok" else -11, stdout=partial)

    monkeypatch.setattr(subprocess, "run", fake_run)
    r = bench.run_extras_child(2, timeout_s=5)
    assert r["nn_gemm"] == [] and r["config0_gemm"] == {"us": 1.0}
    assert ("error" in r) == (how != "ok")


def test_traffic_only_from_a_profile_of_these_sources(tmp_path, monkeypatch):
    """roofline.traffic comes from the committed counter profile only when that
    profile was measured on the current kernel sources."""
    import bench
    from sdvk_amd.profiling import sources_digest

    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    assert bench.profiled_traffic("gemm_q8") == (None, None)
    f = tmp_path / "profiles" / "traffic_gemm_q8_sdxl1024.json"
    f.write_text(json.dumps({"bytes_per_launch": 123, "sources_sha256": "0" * 64}))
    t, note = bench.profiled_traffic("gemm_q8")
    assert t is None and note["bytes_per_launch"] == 123 and "earlier" in note["build"]
    for d in ("sdvk_amd/csrc", "include"):
        (tmp_path / d).mkdir(parents=True)
    (tmp_path / "sdvk_amd/csrc/k.hip").write_text("kernel")
    f.write_text(json.dumps({"bytes_per_launch": 123, "sources_sha256": sources_digest(tmp_path)}))
    assert bench.profiled_traffic("gemm_q8")[0] == 123
    (tmp_path / "sdvk_amd/csrc/k.hip").write_text("kernel, changed")
    assert bench.profiled_traffic("gemm_q8")[0] is None


def test_joint_qkv_weights_are_back_to_back(fake_device):
    import bench
    from sdvk_amd import hip, ops

    st = bench.BlockStack(np.random.default_rng(0), hip, ops, nblocks=2, joint_qkv=True)
    C = bench.BlockStack.DIMS[2]
    nb = C * C // 32 * 34
    for w in st.weights:
        assert w.attn1_k == w.attn1_q + nb and w.attn1_v == w.attn1_k + nb


def test_gpus_above_one_exits_with_a_message(monkeypatch, capsys):
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "2"])
    assert bench.main() == 2
    assert "one GPU" in capsys.readouterr().out


def test_cpu_baseline_one_pass():
    """The CPU baseline leg (the oracle's OpenMP restatement over one full step
    of the same shapes) reports a positive rate with its sample description."""
    import bench

    r = bench.cpu_baseline(threads=max(1, (os.cpu_count() or 1)), min_seconds=0.0, max_passes=1)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s" and r["passes"] == 1
    assert r["value"] > 0 and r["seconds"] > 0 and r["cores"] >= 1
    assert "8 config-1 GEMM shapes" in r["sample"]
