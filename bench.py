"""Benchmark: ms per energy+forces step and atom-steps/s on one MI355X.

Workload: diamond Si 5x5x5 (1000 atoms, rattled
sigma 0.03 from seed 1), MACE 'medium' architecture (128x0e+128x1o, lmax 3,
correlation 3, 2 layers, 8 Bessel, r_cut 6, ZBL on), random-init fp32 weights
from seed 0, energy + forces per step; neighbour list cached (skin 0.5, the
reference's benchmark protocol, docs/prototypes/xbench.py:89-101).

Timed region: W warm-up steps, then K steps of ``mace_step_device`` (positions
and results resident in HBM; no host copies), bracketed by device
synchronisation.  A second pass of K steps with per-launch HIP events gives each
kernel's average duration; the dominant kernel's algorithmic bytes (or flops)
per launch divided by that duration is the roofline ``achieved`` figure.  The CPU
baseline is the float32 CPU oracle (a restatement of the reference algorithm;
MLX cannot run here) on the host cores, on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mace-mlx_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP32_MFMA_PEAK_TFS = 157.3     # MI355X dense fp32 matrix


def peak_of(site: str, bound: str, ctx: dict) -> float:
    """Roofline peak for a site: HBM bandwidth, or the matrix-core rate of its data type."""
    return HBM_PEAK_GBS if bound == "hbm" else FP32_MFMA_PEAK_TFS


def algorithmic_work(site: str, ctx: dict):
    """(bound, amount per launch, unit) for a kernel site of the step.

    Bytes count compulsory unique traffic (node arrays once, fp32, int32
    indices); flops count multiply-adds as 2."""
    N, E, C, nb, H = ctx["N"], ctx["E"], 128, ctx["nb"], 64
    name, _, lyr = site.partition(".L")
    lay = ctx["layers"][int(lyr)] if lyr else None
    fused = ctx.get("fused")
    tabw = 72 if lay and lay["lin"] >= 2 else 0  # M1 table entries per edge (l1 = 1 slots)
    if name == "tp_fwd":
        if fused:  # radial-MLP output layer inside: reads h3 (split planes + scale), writes w for the VJP
            b = 4 * (N * lay["din"] + E * (16 + tabw) + E * lay["wn"] + N * lay["dmid"]) + E * (4 * H + 4)
            return "hbm", b + 4 * (E + N + 1), "GB/s"
        b = 4 * (N * lay["din"] + E * 16 + E * lay["wn"] + N * lay["dmid"]) + 4 * (E + N + 1)
        return "hbm", b, "GB/s"
    if name == "tp_bwd":
        if fused:  # reads w, writes dL/dx rows (after the first layer), dL/dY and dL/dh3 partials
            parts = 2 if lay["lin"] == 1 else 4
            gx = E * lay["din"] if int(lyr) > 0 else 0
            b = 4 * (N * lay["dmid"] + N * lay["din"] + E * (16 + tabw) + E * lay["wn"] + gx
                     + E * 16 * parts + E * H * parts)
            return "hbm", b + 8 * (E + N + 1), "GB/s"
        b = 4 * (N * lay["dmid"] + N * lay["din"] + 2 * E * 16 + 2 * E * lay["wn"]) + 8 * (E + N + 1)
        return "hbm", b, "GB/s"
    if name == "tp_gather":  # segmented sum of the per-edge input-gradient rows
        return "hbm", 4 * (E * lay["din"] + N * lay["din"]) + 4 * (N + 1), "GB/s"
    if name == "mlp_hidden":  # three small layers
        return "mfma", 2 * E * (nb * H + 2 * H * H), "TFLOP/s"
    if name in ("mlp_out", "mlp_gh3"):
        # w = h3 @ W3 and dL/dh3 = gw @ W3^T.  On fp16 matrix cores (split fp32 operands, or the
        # float16 policy) the product needs at most a quarter of the time of the E x W stream it
        # writes / reads, so the bound is HBM: that stream plus the E x 64 side
        if ctx.get("half"):
            return "hbm", 2 * E * lay["wn"] + 2 * E * H + (8 * E if name == "mlp_gh3" else 0), "GB/s"
        if ctx.get("split"):
            return "hbm", 4 * E * lay["wn"] + 4 * E * H + 4 * E, "GB/s"
        return "mfma", 2 * E * H * lay["wn"], "TFLOP/s"
    if name == "mlp_hidden_bwd":
        # the three transposed products; with split products the forward layers are recomputed
        # (no saved derivatives), doubling the work
        return "mfma", 2 * E * (nb * H + 2 * H * H) * (2 if ctx.get("split") else 1), "TFLOP/s"
    if name.startswith("linear") or name.startswith("skip"):
        return "mfma", ctx["linear_flops"].get(site, 0), "TFLOP/s"
    if name in ("sc_fwd", "sc_bwd"):
        return "hbm", 4 * N * (16 * C + lay["dhid"]) * (2 if name == "sc_bwd" else 1), "GB/s"
    if name == "edge_fwd":
        return "hbm", E * (8 + 12 + 16 + 16 * 4 + nb * 4 + 4) + N * 24, "GB/s"
    if name == "edge_bwd":
        return "hbm", E * (16 + 16 * 4 + nb * 4 + 12 + 8), "GB/s"
    if name == "forces":
        return "hbm", E * (12 * 2 + 8) + N * 24 + 8 * (N + 1), "GB/s"
    return "hbm", 0, "GB/s"


def linear_flops(cfg_layers, N):
    """2 * rows * K * Cout summed per linear site (all blocks of a layer)."""
    out = {}
    C = 128
    for l, lay in enumerate(cfg_layers):
        lin, lhid, nslot_by_l = lay["lin"], lay["lhid"], lay["nslot_by_l"]
        up = sum(2 * N * (2 * b + 1) * C * C for b in range(lin))
        msg = sum(2 * N * (2 * lo + 1) * nslot_by_l[lo] * C * C for lo in range(4))
        prod = sum(2 * N * (2 * b + 1) * C * C for b in range(lhid))
        skip = sum(2 * N * (2 * b + 1) * C * C for b in range(min(lin, lhid)))
        out.update({f"linear_up.L{l}": up, f"linear_msg.L{l}": msg, f"linear_prod.L{l}": prod,
                    f"skip.L{l}": skip, f"linear_up_bwd.L{l}": up, f"linear_msg_bwd.L{l}": msg,
                    f"linear_prod_bwd.L{l}": prod, f"skip_bwd.L{l}": skip})
    return out


def load_traffic(site: str, workload: str):
    """HBM bytes per launch of `site` measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (profiles/traffic.json, written from the committed pmc summaries) for this workload,
    or None."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
        if d.get("_calibration", {}).get("workload") != workload:
            return None
        rec = d.get(site)
        return None if rec is None else float(rec["bytes_per_launch"])
    except (ValueError, KeyError, TypeError):
        return None


def cpu_baseline(bc, weights, edges, species, budget_s=25.0):
    """float32 oracle on the host cores (bounded sample: 1 warm-up + up to 3 steps)."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.model import OracleMACE
    threads = len(os.sched_getaffinity(0))  # all host cores this process may use
    torch.set_num_threads(threads)
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    m = OracleMACE(cfg=bc.model, weights=weights, dtype=torch.float32)
    s = bc.system
    ei = np.stack([edges[0], edges[1]]).astype(np.int64)
    t0 = time.perf_counter()
    m.energy_forces(s.positions, species, ei, edges[2], s.cell)
    warm = time.perf_counter() - t0
    times = []
    while len(times) < 3 and sum(times) + warm < budget_s:
        t = time.perf_counter()
        m.energy_forces(s.positions, species, ei, edges[2], s.cell)
        times.append(time.perf_counter() - t)
    med = float(np.median(times)) if times else warm
    return {"value": len(s) / med, "unit": "atom-steps/s", "cores": threads, "kind": "port",
            "sample": f"{bc.name} E+F, float32 CPU oracle (torch, {threads} threads on {model}), median of "
                      f"{max(len(times), 1)} step(s) after 1 warm-up; {med * 1e3:.0f} ms/step"}


def layer_shapes(dm):
    """Per-layer widths (din, dhid, dmid, wn, slots per output degree) of a device model."""
    sys.path.insert(0, str(ROOT / "mace-mlx_amd" / "csrc"))
    import gen_tables
    layers = []
    for l in range(dm.dims["num_layers"]):
        lin, lhid = dm.dims["layer_in_blocks"][l], dm.dims["layer_hid_blocks"][l]
        slots = gen_tables.tp_layout(lin)
        layers.append(dict(lin=lin, lhid=lhid, din=128 * lin * lin, dhid=128 * lhid * lhid,
                           dmid=128 * sum(2 * x[2] + 1 for x in slots), wn=128 * len(slots),
                           nslot_by_l=[sum(1 for x in slots if x[2] == lo) for lo in range(4)]))
    return layers


def tp_scatter_frac(per_step, ctx):
    """Edge TP + scatter kernels (forward, VJP, gather) against the compulsory bytes of both
    passes of every layer: achieved GB/s / HBM peak."""
    sites = [k for k in per_step if k.split(".")[0] in ("tp_fwd", "tp_bwd", "tp_gather")]
    t = sum(per_step[k][0] for k in sites)
    b = sum(algorithmic_work(k, ctx)[1] for k in sites if not k.startswith("tp_gather"))
    return (b / (t * 1e-3) / 1e9) / HBM_PEAK_GBS if t > 0 else 0.0


def measure_config(idx, steps, warmup, separate=False, graphs=None):
    """Steady-state and rebuild step times plus per-site roofline for configuration idx."""
    import torch
    from mace_mlx_amd._ffi import Engine
    from mace_mlx_amd.device_model import build_device_model
    from mace_mlx_amd.model_io import random_init
    from mace_mlx_amd.systems import make_config
    bc = make_config(idx)
    weights = random_init(bc.model, 0)
    dm = build_device_model(bc.model, weights, dtype=bc.dtype)
    eng = Engine(0)
    eng.load_model(dm)
    if separate:
        eng.set_fused_tp(False)
    if graphs is not None:
        eng.set_graphs(graphs)
    s = bc.system
    zmap = {int(z): k for k, z in enumerate(dm.z_table)}
    species = np.array([zmap[int(z)] for z in s.numbers], np.int32)
    eng.set_system(species, s.cell, s.pbc, 0.5)
    stress = "stress" in bc.properties
    eng.step(s.positions, stress=stress)
    N, E = len(s), len(eng.get_edges()[0])
    pos_d = torch.from_numpy(np.ascontiguousarray(s.positions, dtype=np.float64)).cuda()
    out_d = torch.zeros(10 + 3 * N, dtype=torch.float64, device="cuda")
    for _ in range(warmup):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    eng.sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    t0 = time.perf_counter()
    for _ in range(3):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress, force_nl=True)
    eng.sync()
    ms_nl = (time.perf_counter() - t0) / 3 * 1e3
    eng.set_profiling(True)
    for _ in range(steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    eng.sync()
    kt = eng.kernel_times()
    eng.set_profiling(False)
    layers = layer_shapes(dm)
    ctx = dict(N=N, E=E, nb=dm.dims["num_bessel"], layers=layers, linear_flops=linear_flops(layers, N),
               half=bc.dtype == "float16", split=bc.dtype != "float16",
               fused=not separate and bc.dtype != "float16" and max(x["lin"] for x in layers) <= 2)
    per_step = {k: (v[0] / steps, v[1] // steps) for k, v in kt.items()}
    dom = max(per_step, key=lambda k: per_step[k][0])
    b, a, u = algorithmic_work(dom, ctx)
    t, n = per_step[dom]
    ach = (a / max(n, 1)) / (t / max(n, 1) * 1e-3) / (1e9 if b == "hbm" else 1e12)
    frac = ach / peak_of(dom, b, ctx)
    res = {"workload": bc.name, "n_atoms": N, "n_edges": E, "properties": "+".join(bc.properties),
           "feature_dtype": bc.dtype, "ms_per_step": round(ms, 4), "ms_per_step_nl_rebuild": round(ms_nl, 4),
           "atom_steps_per_s": round(N / ms * 1e3, 1), "dominant": dom, "dominant_frac": round(frac, 4),
           "tp_scatter_hbm_frac": round(tp_scatter_frac(per_step, ctx), 4)}
    del eng, pos_d, out_d
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=1, help="benchmark configuration index 0..4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--separate-mlp-out", action="store_true",
                    help="float32 policy: radial-MLP output layer as its own pass (not fused into the TP)")
    ap.add_argument("--kernel-table", action="store_true", help="print per-kernel times to stderr")
    ap.add_argument("--graphs", choices=("on", "off"), default=None,
                    help="replay the step through captured HIP graphs (on) or launch it eagerly (off); "
                         "default: the engine's default")
    ap.add_argument("--sweep", action="store_true",
                    help="also measure every benchmark configuration (table on stderr, 'sweep' in the JSON)")
    ap.add_argument("--copy-calib-mb", type=float, default=0.0,
                    help="run a plain device copy of this size first (rocprof counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    import torch
    from mace_mlx_amd._ffi import Engine
    from mace_mlx_amd.device_model import build_device_model
    from mace_mlx_amd.model_io import random_init
    from mace_mlx_amd.systems import make_config
    if args.copy_calib_mb > 0:
        # counter calibration: one elementwise kernel that reads and writes exactly
        # copy_calib_mb MiB each (b = 2 a); its FETCH_SIZE / WRITE_SIZE give the scale
        n = int(args.copy_calib_mb * (1 << 20) // 4)
        a = torch.ones(n, device="cuda", dtype=torch.float32)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        torch.mul(a, 2.0, out=b)
        torch.cuda.synchronize()
        del a, b

    bc = make_config(args.config)
    weights = random_init(bc.model, 0)
    dm = build_device_model(bc.model, weights, dtype=bc.dtype)
    eng = Engine(0)
    eng.load_model(dm)
    if args.separate_mlp_out:
        eng.set_fused_tp(False)
    graphs = None if args.graphs is None else args.graphs == "on"
    if graphs is not None:
        eng.set_graphs(graphs)
    s = bc.system
    zmap = {int(z): k for k, z in enumerate(dm.z_table)}
    species = np.array([zmap[int(z)] for z in s.numbers], np.int32)
    eng.set_system(species, s.cell, s.pbc, 0.5)
    stress = "stress" in bc.properties
    E_host, _, F_host, _ = eng.step(s.positions, stress=stress)          # builds the neighbour list
    edges = eng.get_edges()
    N, E = len(s), len(edges[0])

    pos_d = torch.from_numpy(np.ascontiguousarray(s.positions, dtype=np.float64)).cuda()
    out_d = torch.zeros(10 + 3 * N, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    eng.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    eng.sync()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) / args.steps * 1e3
    out = out_d.cpu().numpy()
    assert abs(out[0] - E_host) <= 1e-9 * abs(E_host) and np.abs(out[10:].reshape(N, 3) - F_host).max() < 1e-9

    # host-array path (PCIe-inclusive, as the ASE calculator uses it)
    th = time.perf_counter()
    for _ in range(args.steps):
        eng.step(s.positions, stress=stress)
    ms_host = (time.perf_counter() - th) / args.steps * 1e3

    # per-kernel pass
    eng.set_profiling(True)
    for _ in range(args.steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    kt = eng.kernel_times()
    eng.set_profiling(False)
    layers = layer_shapes(dm)
    ctx = dict(N=N, E=E, nb=dm.dims["num_bessel"], layers=layers, linear_flops=linear_flops(layers, N),
               half=bc.dtype == "float16", split=bc.dtype != "float16",
               fused=not args.separate_mlp_out and bc.dtype != "float16"
               and max(x["lin"] for x in layers) <= 2)
    per_step = {k: (v[0] / args.steps, v[1] // args.steps) for k, v in kt.items()}
    dom = max(per_step, key=lambda k: per_step[k][0])
    bound, amount, unit = algorithmic_work(dom, ctx)
    launches = max(per_step[dom][1], 1)
    avg_ms = per_step[dom][0] / launches
    if bound == "hbm":
        achieved = amount / launches / (avg_ms * 1e-3) / 1e9 if launches > 1 else amount / (avg_ms * 1e-3) / 1e9
    else:
        achieved = amount / launches / (avg_ms * 1e-3) / 1e12
    peak = peak_of(dom, bound, ctx)
    roofline = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": load_traffic(dom, bc.name), "kernel": dom,
                "avg_launch_ms": round(avg_ms, 5), "tp_scatter_hbm_frac": round(tp_scatter_frac(per_step, ctx), 4)}
    if args.kernel_table:
        tot = sum(v[0] for v in per_step.values())
        print(f"{'site':24s} {'ms/step':>9s} {'share':>6s} {'launch':>6s}  roofline", file=sys.stderr)
        for k, (t, n) in sorted(per_step.items(), key=lambda kv: -kv[1][0]):
            b, a, u = algorithmic_work(k, ctx)
            per = t / max(n, 1) * 1e-3
            ach = (a / max(n, 1)) / per / (1e9 if b == "hbm" else 1e12) if a else 0.0
            pk = peak_of(k, b, ctx)
            print(f"{k:24s} {t:9.4f} {t / tot * 100:5.1f}% {n:6d}  {ach:9.2f} {u} ({ach / pk * 100:.1f}% of {b})",
                  file=sys.stderr)

    # neighbour-list rebuild included (the reference's benchmark.py:168-style number)
    eng.sync()
    tr = time.perf_counter()
    nrb = max(3, args.steps // 4)
    for _ in range(nrb):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress, force_nl=True)
    eng.sync()
    ms_rebuild = (time.perf_counter() - tr) / nrb * 1e3
    del pos_d, out_d

    sweep = None
    if args.sweep:
        del eng
        sweep = [measure_config(i, max(5, args.steps // 2), args.warmup, args.separate_mlp_out, graphs)
                 for i in range(5)]
        print(f"{'config':16s} {'N':>6s} {'E':>9s} {'ms/step':>9s} {'+NL ms':>8s} {'atom-steps/s':>13s}  "
              f"dominant site (frac of its roofline)   TP+scatter HBM frac", file=sys.stderr)
        for r in sweep:
            print(f"{r['workload']:16s} {r['n_atoms']:6d} {r['n_edges']:9d} {r['ms_per_step']:9.3f} "
                  f"{r['ms_per_step_nl_rebuild']:8.3f} {r['atom_steps_per_s']:13.0f}  "
                  f"{r['dominant']:18s} ({r['dominant_frac']:.3f})   {r['tp_scatter_hbm_frac']:.3f}", file=sys.stderr)

    cpu = None if args.no_cpu_baseline else cpu_baseline(bc, weights, edges, species)
    line = {
        "metric": "ms per energy+forces step (Si1000, medium arch, fp32); atom-steps/sec",
        "value": round(N * args.steps / (t1 - t0), 1),
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_host_arrays": round(ms_host, 4),
        "ms_per_step_nl_rebuild": round(ms_rebuild, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32" if bc.dtype == "float32" else "fp16 features / fp32 accumulation",
        "data": "synthetic (seeded lattice + rattle, random-init weights)",
        "config": {"workload": bc.name, "n_atoms": N, "n_edges": E,
                   "properties": "energy+forces+stress" if stress else "energy+forces",
                   "neighbour_list": "cached (skin 0.5)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if sweep is not None:
        line["sweep"] = sweep
    print(json.dumps(line))


if __name__ == "__main__":
    main()
