"""Map rocprofv3 per-dispatch records of the engine to its launch sites.

The engine names the launch site of every kernel dispatch of a profiled step
(``Engine.launch_order()``, ``mace_get_launch_order``); ``bench.py --launch-order FILE``
writes that list.  A steady-state step is the same dispatch sequence every time
(the same launches, replayed from a captured HIP graph or issued eagerly), so in a
rocprofv3 kernel trace or counter collection every run of exactly that many
dispatches starting at the edge front end (``k_edge_fwd``) is one step, and its
k-th dispatch belongs to the k-th site of the list.  Steps that also rebuild the
neighbour list (sort / scan kernels) or upload the species embedding have a
different length and are left out.

Used by ``bench.py --summarize DIR`` to write the per-site tables under
``profiles/`` and the traffic figures ``bench.py`` reports.
"""

from __future__ import annotations

import collections
import csv
import glob
import json
import os
import re
from typing import Dict, List, Tuple

FIRST_KERNEL = "k_edge_fwd"
# one rocprofv3 --pmc pass (6 SQ counters and 1 GRBM counter fit the block limits together)
N_XCD = 8  # MI355X: GRBM_GUI_ACTIVE of a dispatch is summed over its eight XCDs
MFMA_COUNTERS = ("SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_F32",
                 "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE")


def short_name(n: str) -> str:
    """Readable kernel name from a rocprofv3 record (demangled or not)."""
    if n.startswith("_Z"):  # names the profiler left mangled (_Float16 parameters)
        m = re.search(r"\d+(k_[a-z0-9_]+)(I(?:L[ib]\d+E)+E)?", n)
        if not m:
            return n[:40]
        if m.group(2):
            return m.group(1) + "<" + ",".join(re.findall(r"L[ib](\d+)E", m.group(2))) + ">"
        return m.group(1)
    n = n.replace("mace::(anonymous namespace)::", "").replace("void ", "")
    n = re.sub(r"\(.*", "", n)
    n = re.sub(r"rocprim::\S*?detail::trampoline_kernel<rocprim::\S*?detail::wrapped_(\w+?)_config.*",
               r"rocprim \1", n)
    for plain in ("k_gemm_group", "k_mlp_hidden", "k_edge_fwd"):
        if n.startswith(plain + "<"):
            return plain
    return n.replace(" ", "")[:48]


def _csv(pattern: str) -> List[dict]:
    files = sorted(glob.glob(pattern, recursive=True))
    if not files:
        raise FileNotFoundError(pattern)
    rows = []
    for f in files:
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def steady_steps(names: List[str], n_sites: int) -> List[int]:
    """Start indices of every run of n_sites dispatches that begins at the edge front end
    and is followed by the next step's front end (or the end of the record)."""
    starts = [i for i, nm in enumerate(names) if nm == FIRST_KERNEL]
    out = []
    for a, b in zip(starts, starts[1:] + [len(names)]):
        if b - a == n_sites:
            out.append(a)
    return out


def site_durations(trace_rows: List[dict], order: List[str]) -> Tuple[Dict[str, list], Dict[str, str], int]:
    """{site: [duration ns per launch]}, {site: kernel name}, number of steps used."""
    rows = sorted(trace_rows, key=lambda r: int(r["Start_Timestamp"]))
    names = [short_name(r["Kernel_Name"]) for r in rows]
    steps = steady_steps(names, len(order))
    acc, kname = collections.defaultdict(list), {}
    for a in steps:
        for k, site in enumerate(order):
            r = rows[a + k]
            acc[site].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            kname[site] = names[a + k]
    return acc, kname, len(steps)


def step_spans(trace_rows: List[dict], order: List[str]) -> List[Tuple[float, float]]:
    """(span us, busy us) of every steady-state step."""
    rows = sorted(trace_rows, key=lambda r: int(r["Start_Timestamp"]))
    names = [short_name(r["Kernel_Name"]) for r in rows]
    out = []
    for a in steady_steps(names, len(order)):
        seg = rows[a:a + len(order)]
        span = (int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3
        busy = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in seg) / 1e3
        out.append((span, busy))
    return out


def site_counters(counter_rows: List[dict], order: List[str], counter: str) -> Tuple[Dict[str, float], int]:
    """{site: mean counter value per launch} over the steady-state steps of a
    counter-collection record (one row per dispatch and counter)."""
    rows = [r for r in counter_rows if r.get("Counter_Name", counter) == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    names = [short_name(r["Kernel_Name"]) for r in rows]
    steps = steady_steps(names, len(order))
    acc = collections.defaultdict(list)
    for a in steps:
        for k, site in enumerate(order):
            acc[site].append(float(rows[a + k]["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}, len(steps)


def calibration(counter_rows: List[dict], mib: float) -> float:
    """Counter value of the calibration kernel (torch.mul over `mib` MiB in and out)
    -> scale factor to KiB actually moved."""
    for r in sorted(counter_rows, key=lambda r: int(r["Dispatch_Id"])):
        if "MulFunctor" in r["Kernel_Name"]:
            return mib * 1024.0 / float(r["Counter_Value"])
    raise ValueError("calibration kernel (torch.mul) not found in the counter record")


def summarize(d: str, out_dir: str, calib_mib: float = 256.0, commands: Dict[str, str] = None) -> dict:
    """Write <out_dir>/kernel_trace_<workload>.md, hbm_traffic_<workload>.md and traffic_<workload>.json
    from a measurement directory holding launch_order.txt, bench.json (the bench line of the
    traced run), trace/ (rocprofv3 --kernel-trace --stats csv) and, optionally, pmc_fetch/ and
    pmc_write/ (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE csv)."""
    order = [l for l in open(os.path.join(d, "launch_order.txt")).read().split("\n") if l]
    bench = json.loads(open(os.path.join(d, "bench.json")).read())
    wl = bench["config"]["workload"]
    tag = wl.lower().replace("-", "_")
    commands = commands or {}
    trace = _csv(os.path.join(d, "trace", "**", "*kernel_trace.csv"))
    acc, kname, nsteps = site_durations(trace, order)
    spans = step_spans(trace, order)
    tot = sum(sum(v) for v in acc.values())
    dom = bench["roofline"]["kernel"]
    L = []
    w = L.append
    w(f"# Kernel trace: {wl}, {bench['config']['properties']} step (bench.py workload)\n")
    w("Command (on the GPU box, from the repository root):\n")
    w("    " + commands.get("trace", "rocprofv3 --kernel-trace --stats --output-format csv ... -- python3 bench.py ..."))
    w("\nSummarised by `python bench.py --summarize <dir>` (`mace_mlx_amd/rocprof_sites.py`): every run of "
      f"{len(order)} dispatches that starts at `{FIRST_KERNEL}` is one steady-state step (graph-replayed or eager), "
      "its k-th dispatch belongs to the k-th launch site the engine reports (`mace_get_launch_order`); steps that "
      "rebuild the neighbour list or upload the species embedding have other lengths and are left out.\n")
    if spans:
        sp = sum(s for s, _ in spans) / len(spans)
        bu = sum(b for _, b in spans) / len(spans)
        w(f"Steady-state steps: {nsteps}; span {sp:.1f} us per step, kernels busy {bu:.1f} us "
          f"(gaps {sp - bu:.1f} us).\n")
    w(f"bench.py line of the traced run: `ms_per_step` {bench['ms_per_step']} (under the profiler), dominant site "
      f"`{dom}` with `avg_launch_ms` {bench['roofline']['avg_launch_ms']} (HIP events on the engine stream); the "
      f"trace average for the same site: {sum(acc[dom]) / len(acc[dom]) / 1e6:.5f} ms.\n" if dom in acc else "")
    w("## Per launch site\n")
    w("| site | kernel | launches | avg us | share |\n|---|---|---:|---:|---:|")
    for k, v in sorted(acc.items(), key=lambda kv: -sum(kv[1])):
        w(f"| {k} | {kname[k]} | {len(v)} | {sum(v) / len(v) / 1e3:.1f} | {sum(v) / tot * 100:.1f}% |")
    stats = glob.glob(os.path.join(d, "trace", "**", "*kernel_stats.csv"), recursive=True)
    if stats:
        st = _csv(stats[0])
        st.sort(key=lambda r: -float(r["TotalDurationNs"]))
        w("\n## rocprofv3 --stats (whole run, all launch sites merged, top 16 by total time)\n")
        w("| kernel | calls | total ms | avg us | % |\n|---|---:|---:|---:|---:|")
        for r in st[:16]:
            w(f"| {short_name(r['Name'])} | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
              f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    spath = os.path.join(d, "pmc_sq")
    if os.path.isdir(spath):  # instruction counts (rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_SALU)
        srows = _csv(os.path.join(spath, "**", "*counter_collection.csv"))
        names = [c for c in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_SALU")
                 if any(r.get("Counter_Name") == c for r in srows)]
        per = {c: site_counters(srows, order, c)[0] for c in names}
        w("\n## Instructions per launch (millions of wave-instructions)\n")
        w("    " + commands.get("sq", "rocprofv3 --pmc " + " ".join(names) + " ... -- python3 bench.py ..."))
        w("\nVALU issue time = VALU wave-instructions x 4 cycles / (1024 SIMDs x 2.4 GHz).\n")
        w("| site | " + " | ".join(names) + " | VALU issue us | avg us |\n|---|" + "---:|" * (len(names) + 2))
        top = sorted(per[names[0]].items(), key=lambda kv: -kv[1])[:10] if names else []
        for k, _ in top:
            vals = " | ".join(f"{per[c].get(k, 0.0) / 1e6:.2f}" for c in names)
            issue = per["SQ_INSTS_VALU"].get(k, 0.0) * 4 / (1024 * 2.4e3) if "SQ_INSTS_VALU" in per else 0.0
            avg = sum(acc[k]) / len(acc[k]) / 1e3 if k in acc else float("nan")
            w(f"| {k} | {vals} | {issue:.1f} | {avg:.1f} |")
    mpath = os.path.join(d, "pmc_mfma")
    if os.path.isdir(mpath):  # matrix-core counters (rocprofv3 --pmc SQ_INSTS_MFMA ... GRBM_GUI_ACTIVE)
        mrows = _csv(os.path.join(mpath, "**", "*counter_collection.csv"))
        have = {r.get("Counter_Name") for r in mrows}
        mc = {c: site_counters(mrows, order, c)[0] for c in MFMA_COUNTERS if c in have}
        w("\n## Matrix cores per launch\n")
        w("    " + commands.get("mfma", "rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " ... -- python3 bench.py ..."))
        w("\nMFMA instructions (`SQ_INSTS_MFMA`); matrix flops executed = (`SQ_INSTS_VALU_MFMA_MOPS_F16` + "
          "`_F32`) x 512, i.e. the hardware's count, which includes the three fp16 products of each split-operand "
          "product; achieved = those flops / the launch's trace duration; MFMA busy = "
          "`SQ_VALU_MFMA_BUSY_CYCLES` / (`GRBM_GUI_ACTIVE` / 8 x 1024 SIMDs), the share of SIMD cycles the matrix "
          "unit was busy while the kernel ran (rocprofv3's MfmaUtil; `GRBM_GUI_ACTIVE` per dispatch is the sum over "
          "the eight XCDs: 8 x 2.35 GHz x the duration).  A 16x16x32 fp16 MFMA keeps the unit busy 16 cycles, the "
          "dense-peak rate (2.5 PF/s over 1024 SIMDs), so MFMA busy is also the achieved share of the fp16 matrix "
          "peak.\n")
        w("| site | MFMA instr (M) | fp16 matrix GFLOP | fp32 matrix GFLOP | achieved TF/s | MFMA busy | avg us |\n"
          "|---|---:|---:|---:|---:|---:|---:|")
        key = "SQ_INSTS_MFMA"
        top = sorted(mc.get(key, {}).items(), key=lambda kv: -kv[1])
        for k, v in top:
            if v <= 0:
                continue
            f16 = mc.get("SQ_INSTS_VALU_MFMA_MOPS_F16", {}).get(k, 0.0) * 512
            f32 = mc.get("SQ_INSTS_VALU_MFMA_MOPS_F32", {}).get(k, 0.0) * 512
            busy = mc.get("SQ_VALU_MFMA_BUSY_CYCLES", {}).get(k, 0.0)
            gui = mc.get("GRBM_GUI_ACTIVE", {}).get(k, 0.0)
            avg = sum(acc[k]) / len(acc[k]) / 1e3 if k in acc else float("nan")
            tfs = (f16 + f32) / (avg * 1e-6) / 1e12 if avg == avg and avg > 0 else float("nan")
            util = busy / (gui / N_XCD * 1024) if gui > 0 else float("nan")
            w(f"| {k} | {v / 1e6:.3f} | {f16 / 1e9:.2f} | {f32 / 1e9:.2f} | {tfs:.1f} | {util * 100:.1f}% | {avg:.1f} |")
        result_mfma = {k: {c: mc[c].get(k, 0.0) for c in mc} for k in mc.get(key, {})}
    else:
        result_mfma = None
    os.makedirs(out_dir, exist_ok=True)
    with open(os.path.join(out_dir, f"kernel_trace_{tag}.md"), "w") as f:
        f.write("\n".join(L) + "\n")
    result = {"sites": {k: sum(v) / len(v) / 1e3 for k, v in acc.items()}, "steps": nsteps}
    if result_mfma is not None:
        result["mfma"] = result_mfma
    fpath, wpath = os.path.join(d, "pmc_fetch"), os.path.join(d, "pmc_write")
    if not (os.path.isdir(fpath) and os.path.isdir(wpath)):
        return result
    frows = _csv(os.path.join(fpath, "**", "*counter_collection.csv"))
    wrows = _csv(os.path.join(wpath, "**", "*counter_collection.csv"))
    fs_, ws_ = calibration(frows, calib_mib), calibration(wrows, calib_mib)
    fk, nf = site_counters(frows, order, "FETCH_SIZE")
    wk, _ = site_counters(wrows, order, "WRITE_SIZE")
    tj = {"_calibration": {"workload": wl, "kernel": f"torch.mul(a, 2.0, out=b), {calib_mib:g} MiB in / out",
                           "fetch_scale": fs_, "write_scale": ws_, "steps_averaged": nf}}
    for k in sorted(fk):
        tj[k] = {"fetch_kib": round(fk[k], 1), "write_kib": round(wk.get(k, 0.0), 1),
                 "bytes_per_launch": round((fk[k] * fs_ + wk.get(k, 0.0) * ws_) * 1024.0)}
    with open(os.path.join(out_dir, f"traffic_{tag}.json"), "w") as f:
        json.dump(tj, f, indent=1, sort_keys=True)
    T = []
    t = T.append
    t(f"# HBM traffic per launch: {wl}, {bench['config']['properties']} step\n")
    t("Commands (on the GPU box, from the repository root; one counter per run):\n")
    for key in ("fetch", "write"):
        t("    " + commands.get(key, f"rocprofv3 --pmc {key.upper()}_SIZE ... -- python3 bench.py ... "
                                      f"--copy-calib-mb {calib_mib:g}"))
    t(f"\nCalibration: `--copy-calib-mb {calib_mib:g}` first runs one elementwise kernel `b = 2 a` over "
      f"{calib_mib:g} MiB (reads and writes {calib_mib * 1024:.0f} KiB).  FETCH_SIZE is scaled by {fs_:.4f} and "
      f"WRITE_SIZE by {ws_:.4f} so that the calibration kernel reads its true bytes; HBM bytes per launch = "
      f"(FETCH_SIZE x {fs_:.3f} + WRITE_SIZE x {ws_:.3f}) KiB x 1024, averaged over {nf} steady-state steps "
      f"(dispatches mapped to sites as in the kernel-trace summary).  `traffic_{tag}.json` holds the same numbers for "
      "bench.py.  FETCH_SIZE counts L2 misses, which may still hit the last-level (Infinity) cache.\n")
    t("| site | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB per launch (scaled) |\n|---|---:|---:|---:|")
    for k in sorted(fk, key=lambda k: -tj[k]["bytes_per_launch"]):
        t(f"| {k} | {tj[k]['fetch_kib']:.1f} | {tj[k]['write_kib']:.1f} | {tj[k]['bytes_per_launch'] / 1e6:.1f} |")
    with open(os.path.join(out_dir, f"hbm_traffic_{tag}.md"), "w") as f:
        f.write("\n".join(T) + "\n")
    result["traffic"] = tj
    return result
