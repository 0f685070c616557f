"""Summaries of rocprofv3 output for this library's kernels.

Two reports, both plain text so they can be kept next to the source:

* ``stats``: a ``*_kernel_stats.csv`` (``rocprofv3 --kernel-trace --stats``)
  turned into a markdown table per kernel plus per-family aggregates
  (``gemm_q8`` = the NT GEMM kernels with their split-K init / bias fills, one
  entry per API call; ``attention`` = the fused attention kernels;
  ``gemm_nn_q8`` = the NN GEMM kernels with their split-K clear).
* ``traffic``: two ``*_counter_collection.csv`` files (``--pmc FETCH_SIZE``,
  then ``--pmc WRITE_SIZE``) turned into HBM bytes per launch of a family.
  Each counter (KiB per dispatch) is scaled by what it reads for the runtime's
  device-to-device copy of a known size in the same run (``bench.py
  --copy-probe-mib``): the copy reads and writes exactly that many bytes, so
  ``factor = bytes / (counter x 1024)``.

* ``counters``: ``*_counter_collection.csv`` files of other ``--pmc`` passes
  (MFMA / VALU busy cycles, LDS bank conflicts, wait cycles) averaged per
  kernel and grid, with the derived busy fractions.

Usage:
  python -m sdvk_amd.profiling stats  <kernel_stats.csv> <out.md> --command "<cmd>"
  python -m sdvk_amd.profiling traffic <fetch.csv> <write.csv> <copy_mib> <family> <out.json> --command "<cmd>"
  python -m sdvk_amd.profiling counters <out.md> <counter_collection.csv>... --command "<cmd>"
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import re
import shutil
import subprocess
import sys
from pathlib import Path

# family -> (main kernels: one launch per API call, helper kernels of the same calls)
# (the K-split reduce pass is shared by both GEMMs; it is counted with gemm_q8)
FAMILIES = {
    "gemm_q8": (("gemm_q8_kernel", "gemm_q8_any_kernel"),
                ("gemm_fill_kernel", "splitk_reduce_kernel")),
    "attention": (("attn_kernel", "attn_f16_kernel"), ("attn_merge_kernel",)),
    "gemm_nn_q8": (("gemm_nn_q8_kernel", "gemm_nn_q8_tiled_kernel"), ()),
}
COPY_KERNEL = re.compile(r"copyBuffer", re.I)


def short_name(name: str) -> str:
    """`void mi::(anonymous namespace)::gemm_q8_kernel<256, 128, ...>(mi::...)` -> `gemm_q8_kernel<256, 128, ...>`."""
    if name.startswith("_Z"):
        tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
        if tool:
            name = subprocess.run([tool, name], capture_output=True, text=True).stdout.strip() or name
        m = re.search(r"\d([a-z][a-z_0-9]*?_kernel)I((?:DF16_|f|Lb[01]E|Li\d+E)+)E", name) if name.startswith("_Z") \
            else None
        if m:  # template arguments this library uses that binutils' demangler may not know (_Float16)
            toks = re.findall(r"DF16_|f|Lb[01]E|Li\d+E", m.group(2))
            conv = {"DF16_": "_Float16", "f": "float", "Lb0E": "false", "Lb1E": "true"}
            name = f"{m.group(1)}<{', '.join(conv.get(t, t[2:-1]) for t in toks)}>"
    n = re.sub(r"^void\s+", "", name)
    n = n.replace("mi::(anonymous namespace)::", "")
    n = re.sub(r"\(.*\)$", "", n)
    return n


def _has(name: str, key: str) -> bool:
    """key as a whole identifier of a kernel name: mangled (length-prefixed,
    `...15attn_f16_kernelI...`) or demangled (`...::attn_f16_kernel<...`)."""
    if name.startswith("_Z"):
        return f"{len(key)}{key}" in name
    return re.search(r"(?<![A-Za-z0-9_])" + re.escape(key) + r"(?![A-Za-z0-9_])", name) is not None


def is_main(name: str, family: str) -> bool:
    return any(_has(name, k) for k in FAMILIES[family][0])


def family_of(name: str) -> str | None:
    for fam, (main, helpers) in FAMILIES.items():
        if any(_has(name, k) for k in main + helpers):
            return fam
    return None


def stats_report(csv_path: str, command: str, flops: dict | None = None) -> str:
    """flops: {family: algorithmic FLOP per API call}; adds the achieved rate of
    each such family (FLOP per call / its average time per call) and its
    fraction of the 2500 TFLOP/s fp16 MFMA peak."""
    rows = list(csv.DictReader(open(csv_path)))
    lines = [f"# rocprofv3 kernel statistics", "", f"Command: `{command}`", "",
             "| kernel | calls | avg us | min us | max us | total % |", "|---|---:|---:|---:|---:|---:|"]
    fam = collections.defaultdict(lambda: [0, 0.0])  # calls of the main kernel, total ns (incl. helpers)
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"]
        calls, tot = int(r["Calls"]), float(r["TotalDurationNs"])
        lines.append(f"| `{short_name(name)}` | {calls} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
        f = family_of(name)
        if f:
            if is_main(name, f):
                fam[f][0] += calls
            fam[f][1] += tot
    lines += ["", "Family aggregates (total time of the family's kernels / calls of its main kernel, i.e. per API "
                  "call; the GEMM family includes its K-split reduce passes, attention its key-split merge passes):", "",
              "| family | calls | avg us per call |", "|---|---:|---:|"]
    for f, (calls, tot) in fam.items():
        if calls:
            lines.append(f"| {f} | {calls} | {tot / calls / 1e3:.2f} |")
    for f, fl in (flops or {}).items():
        calls, tot = fam.get(f, (0, 0.0))
        if calls:
            tf = fl / (tot / calls * 1e-9) / 1e12
            lines += ["", f"{f}: {fl:.6g} algorithmic FLOP per call / {tot / calls / 1e3:.2f} us per call = "
                          f"{tf:.1f} TFLOP/s = {tf / 2500.0:.4f} of the 2500 TFLOP/s fp16 MFMA peak"]
    return "\n".join(lines) + "\n"


def _per_dispatch(csv_path: str, counter: str):
    """[(kernel, grid, counter value, duration ns or None)] in dispatch order."""
    out = []
    for r in csv.DictReader(open(csv_path)):
        if r["Counter_Name"] == counter:
            dur = None
            if r.get("Start_Timestamp") and r.get("End_Timestamp"):
                dur = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
            out.append((r["Kernel_Name"], int(r["Grid_Size"]), float(r["Counter_Value"]), dur))
    return out


def sources_digest(root: Path | None = None) -> str:
    """sha256 over the kernel sources and the C-ABI header (names and contents):
    identifies the build a counter profile was measured on."""
    import hashlib

    root = Path(root) if root else Path(__file__).resolve().parents[1]
    h = hashlib.sha256()
    files = sorted((root / "sdvk_amd" / "csrc").glob("*")) + sorted((root / "include").glob("*.h"))
    for f in files:
        if f.suffix in (".hip", ".hpp", ".cpp", ".h"):
            h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()


def traffic_report(fetch_csv: str, write_csv: str, copy_mib: int, family: str, command: str) -> dict:
    nbytes = copy_mib << 20
    result = {"family": family, "copy_probe_bytes": nbytes, "command": command, "sources_sha256": sources_digest()}
    per_shape = collections.OrderedDict()  # (kernel, grid) -> {"fetch": [(bytes, ns)], "write": [...]}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _per_dispatch(path, counter)
        copies = [v for n, _, v, _ in rows if COPY_KERNEL.search(n)]
        if not copies:
            raise SystemExit(f"{path}: no copy-probe dispatch found")
        factor = nbytes / (max(copies) * 1024.0)
        result[f"{counter.lower()}_factor"] = round(factor, 5)
        result[f"{counter.lower()}_copy_kib"] = max(copies)
        for n, grid, v, dur in rows:
            if is_main(n, family):
                d = per_shape.setdefault((short_name(n), grid), {"fetch": [], "write": []})
                d["fetch" if counter == "FETCH_SIZE" else "write"].append((v * 1024.0 * factor, dur))
    shapes = []
    tot, cnt = 0.0, 0
    for (name, grid), d in per_shape.items():
        # the two runs launch the same sequence: pair the i-th dispatch of each, then split
        # the pairs into duration classes (one grid can serve shapes of very different cost)
        pairs = [(fd[1] if fd[1] is not None else 0.0, (fd[0], wd[0], fd[1], wd[1]))
                 for fd, wd in zip(d["fetch"], d["write"])]
        for cls in _duration_classes(pairs):
            k = len(cls)
            f = sum(x[0] for _, x in cls) / k
            w = sum(x[1] for _, x in cls) / k
            durs = [x[2] for _, x in cls if x[2] is not None] + [x[3] for _, x in cls if x[3] is not None]
            entry = {"kernel": name, "grid": grid, "fetch_bytes": round(f), "write_bytes": round(w), "dispatches": k}
            if durs:
                us = sum(durs) / len(durs) / 1e3
                entry["profiled_us"] = round(us, 2)
                entry["gbs"] = round((f + w) / (us * 1e3), 1)  # bytes / ns = GB/s
            shapes.append(entry)
            tot += (f + w) * k
            cnt += k
    result["per_kernel_grid"] = shapes
    result["bytes_per_launch"] = round(tot / cnt) if cnt else None
    result["note"] = ("fetch_bytes / write_bytes: HBM-side bytes per dispatch (FETCH_SIZE / WRITE_SIZE scaled by the "
                      "copy probe); profiled_us: the profiled (serialised) dispatch's duration; gbs: their sum over it")
    return result


# Derived figures of the counter report (per dispatch; rocprofv3's CSV sums each
# counter over all its instances). GRBM_GUI_ACTIVE is counted once per XCD, so
# the dispatch's active cycles are its sum / 8. SQ_VALU_MFMA_BUSY_CYCLES sums
# the busy cycles of every SIMD, so MFMA busy = that / (active cycles x 1024
# SIMDs); for v_mfma_f32_32x32x16_f16 it equals 32 cycles x the MFMA count, i.e.
# FLOP / 1024 (checked against the 9216x1280x1280 GEMM: 29.49 M = 30.2 GFLOP /
# 1024). SQ_ACTIVE_INST_VALU and SQ_WAVE_CYCLES are per-wave sums in quad-cycles.
XCDS = 8
SIMDS = 256 * 4


def _duration_classes(items):
    """Splits dispatches [(duration_ns, counters)] into classes at gaps of more
    than 2x in duration: one (kernel, grid) can serve shapes of very different
    cost (the attention kernel's self- and cross-attention shapes share a grid)."""
    items = sorted(items, key=lambda x: x[0])
    out, cur = [], []
    for it in items:
        if cur and it[0] > 2.0 * cur[-1][0]:
            out.append(cur)
            cur = []
        cur.append(it)
    if cur:
        out.append(cur)
    return out


def counters_report(csv_paths: list[str], command: str) -> str:
    """Per (kernel, grid, duration class): the average of every counter over the
    dispatches, with MFMA busy / VALU busy / LDS bank conflicts per LDS
    instruction / wait fraction where the counters are present."""
    disp = collections.OrderedDict()  # (path, dispatch id) -> (name, grid, duration, {counter: value})
    for path in csv_paths:
        for r in csv.DictReader(open(path)):
            k = (path, r["Dispatch_Id"])
            if k not in disp:
                dur = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
                disp[k] = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]), dur, {})
            disp[k][3][r["Counter_Name"]] = float(r["Counter_Value"])
    groups = collections.OrderedDict()
    for name, grid, dur, cnt in disp.values():
        groups.setdefault((name, grid), []).append((dur, cnt))
    names = sorted({c for _, _, _, cnt in disp.values() for c in cnt})
    lines = ["# rocprofv3 counters per kernel and grid", "", f"Command: `{command}`", "",
             "Averages per dispatch (each counter summed over its instances by rocprofv3); dispatches of one "
             "kernel and grid are split where their durations differ by more than 2x (shapes of different cost "
             "on one grid). active = GRBM_GUI_ACTIVE / 8 (one count per XCD); mfma_busy = "
             "SQ_VALU_MFMA_BUSY_CYCLES / (active x 1024 SIMDs); valu_busy = 4 x SQ_ACTIVE_INST_VALU "
             "(quad-cycles, summed over waves) / (active x 1024); lds_conflict_per_lds = SQ_LDS_BANK_CONFLICT "
             "cycles / SQ_INSTS_LDS; wait_frac = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (both quad-cycles summed "
             "over waves). Durations are those of the profiled (serialised) dispatches.", ""]
    hdr = ["kernel", "grid", "dispatches", "avg us"] + names + ["mfma_busy", "valu_busy", "lds_conflict_per_lds",
                                                               "wait_frac"]
    lines += ["| " + " | ".join(hdr) + " |", "|" + "---|" * len(hdr)]
    for (name, grid), items in groups.items():
        for cls in _duration_classes(items):
            avg = {}
            for c in names:
                vals = [cnt[c] for _, cnt in cls if c in cnt]
                if vals:
                    avg[c] = sum(vals) / len(vals)
            us = sum(d for d, _ in cls) / len(cls) / 1e3
            gui = avg.get("GRBM_GUI_ACTIVE")
            active = gui / XCDS if gui else None

            def frac(num, scale=1.0):
                return f"{scale * avg[num] / (active * SIMDS):.3f}" if active and num in avg else ""
            conf = (f"{avg['SQ_LDS_BANK_CONFLICT'] / avg['SQ_INSTS_LDS']:.3f}"
                    if avg.get("SQ_INSTS_LDS") and "SQ_LDS_BANK_CONFLICT" in avg else "")
            wait = (f"{avg['SQ_WAIT_INST_ANY'] / avg['SQ_WAVE_CYCLES']:.3f}"
                    if avg.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_ANY" in avg else "")
            row = [f"`{name}`", str(grid), str(len(cls)), f"{us:.2f}"]
            row += [f"{avg[c]:.4g}" if c in avg else "" for c in names]
            row += [frac("SQ_VALU_MFMA_BUSY_CYCLES"), frac("SQ_ACTIVE_INST_VALU", 4.0), conf, wait]
            lines.append("| " + " | ".join(row) + " |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("out")
    s.add_argument("--command", required=True)
    s.add_argument("--flops", action="append", default=[], metavar="FAMILY=FLOP",
                   help="algorithmic FLOP per API call of a family (adds its achieved rate)")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_csv")
    t.add_argument("write_csv")
    t.add_argument("copy_mib", type=int)
    t.add_argument("family", choices=sorted(FAMILIES))
    t.add_argument("out")
    t.add_argument("--command", required=True)
    c = sub.add_parser("counters")
    c.add_argument("out")
    c.add_argument("csvs", nargs="+")
    c.add_argument("--command", required=True)
    a = ap.parse_args(argv)
    if a.cmd == "counters":
        Path(a.out).write_text(counters_report(a.csvs, a.command))
    elif a.cmd == "stats":
        fl = {k: float(v) for k, v in (x.split("=", 1) for x in a.flops)}
        Path(a.out).write_text(stats_report(a.csv, a.command, fl))
    else:
        Path(a.out).write_text(json.dumps(traffic_report(a.fetch_csv, a.write_csv, a.copy_mib, a.family,
                                                         a.command), indent=1) + "\n")
    print(Path(a.out).read_text())
    return 0


if __name__ == "__main__":
    sys.exit(main())
