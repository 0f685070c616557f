"""The rocprofv3 summarisers (sdvk_amd.profiling) on synthetic CSVs with the
columns rocprofv3 writes: kernel families and per-call aggregates for every
kernel this library launches, and the copy-probe byte calibration."""
from __future__ import annotations

import csv

import pytest

from sdvk_amd import profiling as p

ATTN_F16 = "_ZN2mi12_GLOBAL__N_115attn_f16_kernelIDF16_Li4EEEvNS0_8AttnArgsEj"
GEMM = "_ZN2mi12_GLOBAL__N_114gemm_q8_kernelILi256ELi128ELi4ELi2ELi2ELi0ELb0ELb0ELi2ELi0EEEvNS0_8GemmArgsE"
INIT = "_ZN2mi12_GLOBAL__N_116gemm_fill_kernelEPfPKfjjjmj"
REDUCE = "_ZN2mi12_GLOBAL__N_120splitk_reduce_kernelILi0ELb1EEEvPKfmjPfS3_jjjmj"
ANY = "_ZN2mi12_GLOBAL__N_118gemm_q8_any_kernelENS0_8GemmArgsE"
NN = "_ZN2mi12_GLOBAL__N_123gemm_nn_q8_tiled_kernelILb1EEEvNS0_6NnArgsE"
MERGE = "_ZN2mi12_GLOBAL__N_117attn_merge_kernelIDF16_EEvNS0_8AttnArgsEj"
COPY = "__amd_rocclr_copyBuffer"


@pytest.mark.parametrize("name,family,main", [
    (ATTN_F16, "attention", True), (MERGE, "attention", False), (GEMM, "gemm_q8", True), (INIT, "gemm_q8", False),
    (REDUCE, "gemm_q8", False), (ANY, "gemm_q8", True), (NN, "gemm_nn_q8", True),
    (COPY, None, None),
    ("void mi::(anonymous namespace)::gemm_q8_kernel<64, 64, 2, 2, 2, 0, true, false, 2, 0>(mi::GemmArgs)",
     "gemm_q8", True),
])
def test_families(name, family, main):
    assert p.family_of(name) == family
    if family:
        assert p.is_main(name, family) == main


def test_short_names():
    assert p.short_name(ATTN_F16) == "attn_f16_kernel<_Float16, 4>"
    assert p.short_name(GEMM).startswith("gemm_q8_kernel<256, 128")


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_stats_report_aggregates_per_call(tmp_path):
    f = tmp_path / "k.csv"
    hdr = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"]
    _write(f, hdr, [[GEMM, 4, 400000, 100000, 40, 90000, 110000],
                    [INIT, 2, 20000, 10000, 2, 9000, 11000],
                    [ANY, 2, 100000, 50000, 10, 50000, 50000],
                    [ATTN_F16, 3, 300000, 100000, 30, 100000, 100000],
                    [NN, 1, 50000, 50000, 5, 50000, 50000],
                    [COPY, 1, 1000, 1000, 0.1, 1000, 1000]])
    md = p.stats_report(str(f), "cmd")
    agg = {l.split("|")[1].strip(): float(l.split("|")[3]) for l in md.splitlines()
           if l.startswith("| ") and l.count("|") == 4 and not l.startswith("| family")}
    assert agg["gemm_q8"] == pytest.approx((400000 + 20000 + 100000) / 6 / 1e3, abs=0.01)  # 6 calls, helpers timed
    assert agg["attention"] == pytest.approx(100.0, abs=0.01)
    assert agg["gemm_nn_q8"] == pytest.approx(50.0, abs=0.01)
    assert "attn_f16_kernel<_Float16, 4>" in md


def test_traffic_report_scales_by_the_copy_probe(tmp_path):
    hdr = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    # copy probe of 1 MiB: FETCH_SIZE reads half its bytes (factor 2), WRITE_SIZE all of them
    _write(fetch, hdr, [[COPY, 1024, "FETCH_SIZE", 512], [GEMM, 4096, "FETCH_SIZE", 1000],
                        [GEMM, 4096, "FETCH_SIZE", 3000], [ATTN_F16, 512, "FETCH_SIZE", 7]])
    _write(write, hdr, [[COPY, 1024, "WRITE_SIZE", 1024], [GEMM, 4096, "WRITE_SIZE", 100],
                        [GEMM, 4096, "WRITE_SIZE", 100], [ATTN_F16, 512, "WRITE_SIZE", 7]])
    r = p.traffic_report(str(fetch), str(write), 1, "gemm_q8", "cmd")
    assert r["fetch_size_factor"] == pytest.approx(2.0) and r["write_size_factor"] == pytest.approx(1.0)
    (k,) = r["per_kernel_grid"]
    assert k["dispatches"] == 2
    assert k["fetch_bytes"] == round(2000 * 1024 * 2.0) and k["write_bytes"] == round(100 * 1024)
    assert r["bytes_per_launch"] == round(2000 * 1024 * 2.0 + 100 * 1024)
    assert r["sources_sha256"] == p.sources_digest()  # the build the counters were read on


def test_traffic_report_splits_duration_classes_and_rates(tmp_path):
    """One grid serving shapes of very different cost (self- and cross-attention)
    is reported per duration class, each with its GB/s over the profiled duration."""
    hdr = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    _write(fetch, hdr, [[COPY, 1024, "FETCH_SIZE", 512, 0, 10], [ATTN_F16, 512, "FETCH_SIZE", 1000, 0, 100000],
                        [ATTN_F16, 512, "FETCH_SIZE", 10, 0, 5000], [ATTN_F16, 512, "FETCH_SIZE", 1000, 0, 100000]])
    _write(write, hdr, [[COPY, 1024, "WRITE_SIZE", 1024, 0, 10], [ATTN_F16, 512, "WRITE_SIZE", 500, 0, 100000],
                        [ATTN_F16, 512, "WRITE_SIZE", 10, 0, 5000], [ATTN_F16, 512, "WRITE_SIZE", 500, 0, 100000]])
    r = p.traffic_report(str(fetch), str(write), 1, "attention", "cmd")
    short, long_ = r["per_kernel_grid"]
    assert short["dispatches"] == 1 and long_["dispatches"] == 2
    assert short["profiled_us"] == 5.0 and long_["profiled_us"] == 100.0
    assert long_["fetch_bytes"] == round(1000 * 1024 * 2.0) and long_["write_bytes"] == 500 * 1024
    assert long_["gbs"] == pytest.approx((1000 * 1024 * 2.0 + 500 * 1024) / 100e3, rel=1e-3)
