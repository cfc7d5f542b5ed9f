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
FP16_MFMA_PEAK_TFS = 2500.0    # MI355X dense fp16 / bf16 matrix
RADIAL_H = 64                  # radial-MLP hidden width (last hidden layer -> TP weights)


def tp_bytes(name, lay, N, E, s, fused):
    """Algorithmic HBM bytes of one edge-TP + scatter layer-pass (the benchmark's definition):

        B_fwd = s (N D_in + E 16 + E W + N D_mid) + 4 (E + N + 1)
        B_bwd = s (N D_mid + 2 N D_in + 2 E 16 + 2 E W) + 8 (E + N + 1)

    with s = 4 bytes (2 for fp16 features) and W the TP weights per edge.  With the radial
    MLP's output layer fused into the TP kernel (`fused`), the per-edge weights never reach
    HBM: E W is replaced by E 64 (the last hidden activation) and the layer's flops are
    counted separately (tp_flops)."""
    W = RADIAL_H if fused else lay["wn"]
    if name == "tp_fwd":
        return s * (N * lay["din"] + E * 16 + E * W + N * lay["dmid"]) + 4 * (E + N + 1)
    return s * (N * lay["dmid"] + 2 * N * lay["din"] + 2 * E * 16 + 2 * E * W) + 8 * (E + N + 1)


def tp_flops(lay, E, fused):
    """Flops of the radial MLP's output layer inside a fused TP pass: w = h3 W3 (forward) or
    dL/dh3 = dL/dw W3^T (VJP), 2 E 64 W each; 0 when the layer runs as its own pass."""
    return 2 * E * RADIAL_H * lay["wn"] if fused else 0


def site_work(site: str, ctx: dict):
    """(algorithmic bytes, algorithmic flops, flop peak TF/s) per launch of a launch site.

    Bytes count compulsory unique traffic (node arrays once, int32 indices); flops count
    multiply-adds as 2 and are priced on the matrix-core peak of the arithmetic type the
    product computes in (fp32 for the float32 policy: the split-fp16 products emulate it)."""
    N, E, C, nb, H = ctx["N"], ctx["E"], ctx.get("C", 128), ctx["nb"], RADIAL_H
    half = ctx.get("half")
    s = 2 if half else 4
    fpk = FP16_MFMA_PEAK_TFS if half else FP32_MFMA_PEAK_TFS
    name, _, lyr = site.partition(".L")
    lay = ctx["layers"][int(lyr)] if lyr else None
    fused = ctx.get("fused")
    if name in ("tp_fwd", "tp_bwd"):
        return tp_bytes(name, lay, N, E, s, fused), tp_flops(lay, E, fused), fpk
    if name == "tp_gather":  # segmented sum of the per-edge input-gradient rows (implementation traffic;
        # the fused VJP writes them as fp16 values under the float16 policy)
        return ctx.get("gx_bytes", 4) * E * lay["din"] + 4 * N * lay["din"] + 4 * (N + 1), 0, fpk
    if name == "mlp_hidden":  # three small layers: ef in, last hidden activation out
        return E * (4 * nb + s * H), 2 * E * (nb * H + 2 * H * H), fpk
    if name == "mlp_hidden_bwd":  # the three transposed products: dL/dh3 in, dL/def out (+ ef)
        return E * (8 * nb + 4 * H), 2 * E * (nb * H + 2 * H * H), fpk
    if name == "mlp_ln":  # mh-1 LayerNorm radial MLP (three layers) and density MLP: ef in, h3 + density out
        return E * (4 * nb + s * H + 4), 2 * E * (2 * nb * H + 2 * H * H + H), fpk
    if name == "mlp_ln_bwd":  # both MLPs recomputed, then their transposed products: dL/dh3 in, dL/def out
        return E * (8 * nb + 4 * H + 8), 4 * E * (2 * nb * H + 2 * H * H + H), fpk
    if name in ("mlp_out", "mlp_gh3"):  # w = h3 W3, dL/dh3 = dL/dw W3^T over the E x W stream
        return s * E * (lay["wn"] + H), 2 * E * H * lay["wn"], fpk
    if name.startswith("linear") or name.startswith("message_skip"):
        f, b = ctx["linear_work"].get(site, (0, 0))
        return b, f, fpk
    if name in ("sc_fwd", "sc_bwd"):
        return 4 * N * (16 * C + lay["dhid"]) * (2 if name == "sc_bwd" else 1), 0, fpk
    if name == "edge_fwd":
        return E * (8 + 12 + 16 + 16 * 4 + nb * 4 + 4) + N * 24, 0, fpk
    if name == "edge_bwd":
        return E * (16 + 16 * 4 + nb * 4 + 12 + 8), 0, fpk
    if name == "forces":
        return E * (12 * 2 + 8) + N * 24 + 8 * (N + 1), 0, fpk
    return 0, 0, fpk


def roofline_of(site: str, ctx: dict, avg_ms: float):
    """Roofline record of one launch: the binding bound is the larger of bytes / HBM peak
    and flops / matrix peak; frac = that time / the measured launch time."""
    b, f, fpk = site_work(site, ctx)
    t = avg_ms * 1e-3
    tb, tf = b / (HBM_PEAK_GBS * 1e9), f / (fpk * 1e12)
    if tb >= tf:
        rec = {"bound": "hbm", "achieved": b / t / 1e9 if t > 0 else 0.0, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    else:
        rec = {"bound": "mfma", "achieved": f / t / 1e12 if t > 0 else 0.0, "peak": fpk, "unit": "TFLOP/s"}
    rec.update(frac=max(tb, tf) / t if t > 0 else 0.0, algorithmic_bytes=int(b), algorithmic_flops=int(f),
               hbm_frac=tb / t if t > 0 else 0.0, mfma_frac=tf / t if t > 0 else 0.0)
    return rec


def linear_work(cfg_layers, N):
    """(flops, bytes) per grouped-product site: 2 rows K Cout summed over the problems of a
    layer; bytes = the input and output node rows (fp32) plus the weights.  The skip
    connection's product is the second operand of linear_prod (forward) and linear_up_bwd
    (VJP); the message skip of a non-residual block is a site of its own."""
    out = {}
    for l, lay in enumerate(cfg_layers):
        C = lay["C"]
        lin, lhid, nslot_by_l, nskip = lay["lin"], lay["lhid"], lay["nslot_by_l"], lay["nskip"]
        blk = lambda nb: sum(2 * N * (2 * b + 1) * C * C for b in range(nb))
        dint = 16 * C
        skip_in = 4 * N * C * sum((2 * b + 1) for b in range(nskip))
        msg = sum(2 * N * (2 * lo + 1) * nslot_by_l[lo] * C * C for lo in range(4))
        by_msg = 4 * N * (lay["dmid"] + dint) + 4 * sum(nslot_by_l) * C * C
        out[f"linear_up.L{l}"] = (blk(lin), 4 * N * 2 * lay["din"] + 4 * lin * C * C)
        out[f"linear_up_bwd.L{l}"] = (blk(lin) + blk(nskip),
                                      4 * N * 2 * lay["din"] + skip_in + 4 * (lin + nskip) * C * C)
        out[f"linear_msg.L{l}"] = out[f"linear_msg_bwd.L{l}"] = (msg, by_msg)
        out[f"linear_prod.L{l}"] = (blk(lhid) + blk(nskip),
                                    4 * N * (dint + lay["dhid"]) + skip_in + 4 * (lhid + nskip) * C * C)
        out[f"linear_prod_bwd.L{l}"] = (blk(lhid), 4 * N * (dint + lay["dhid"]) + 4 * lhid * C * C)
        if not lay["resid"]:
            out[f"message_skip.L{l}"] = out[f"message_skip_bwd.L{l}"] = (blk(4), 4 * N * 2 * dint + 4 * 4 * C * C)
    return out


def tp_scatter_summary(per_step, ctx):
    """The edge TP + scatter kernels of a step (forward, VJP and the gather of the VJP's
    per-edge rows, both layers) against (a) the benchmark's unfused compulsory bytes at HBM
    peak (`hbm_frac_unfused_bytes`: the TP weights counted as an E x W stream, the
    definition of the <= 60 % target) and (b) their own roofline with the radial MLP's
    output layer fused in (`roofline_frac`: sum over sites of max(bytes / HBM peak,
    flops / matrix peak) over the measured time)."""
    sites = [k for k in per_step if k.split(".")[0] in ("tp_fwd", "tp_bwd", "tp_gather")]
    t = sum(per_step[k][0] for k in sites) * 1e-3
    if t <= 0:
        return {"ms": 0.0, "hbm_frac_unfused_bytes": 0.0, "roofline_frac": 0.0}
    s = 2 if ctx.get("half") else 4
    unf = tmin = 0.0
    for k in sites:
        name, _, lyr = k.partition(".L")
        if name == "tp_gather":
            continue
        lay = ctx["layers"][int(lyr)]
        unf += tp_bytes(name, lay, ctx["N"], ctx["E"], s, False)
        b, f, fpk = site_work(k, ctx)
        tmin += max(b / (HBM_PEAK_GBS * 1e9), f / (fpk * 1e12))
    return {"ms": round(t * 1e3, 4), "unfused_bytes": int(unf),
            "hbm_frac_unfused_bytes": round(unf / t / (HBM_PEAK_GBS * 1e9), 4),
            "roofline_frac": round(tmin / t, 4)}


def load_traffic(site: str, workload: str):
    """HBM bytes per launch of `site` measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (profiles/traffic_<workload>.json, written from the committed pmc summaries), or None."""
    p = ROOT / "profiles" / f"traffic_{workload.lower().replace('-', '_')}.json"
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


def cpu_baseline(bc, weights, edges, species, budget_s=40.0):
    """float32 CPU restatement on the host cores with the reference's CPU-path forms (the conv TP
    as x2-first batched products, `tensor_product.py:545-575`; the row-compressed symmetric
    contraction, `symmetric_contraction.py:530-540`; activations kept, no recomputation), timed as
    the reference's benchmark protocol: 3 warm-ups, then the median of 10 E+F steps
    (`docs/prototypes/xbench.py:89-101`), fewer if the budget runs out (the count is reported)."""
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
    m = OracleMACE(cfg=bc.model, weights=weights, dtype=torch.float32, gemm_tp=True, recompute=False,
                   edge_chunk=4096)
    s = bc.system
    ei = np.stack([edges[0], edges[1]]).astype(np.int64)
    t0 = time.perf_counter()
    nwarm = 0
    while nwarm < 3 and (nwarm == 0 or time.perf_counter() - t0 < budget_s / 4):
        m.energy_forces(s.positions, species, ei, edges[2], s.cell)
        nwarm += 1
    warm = time.perf_counter() - t0
    times = []
    while len(times) < 10 and (not times or sum(times) + warm < budget_s):
        t = time.perf_counter()
        m.energy_forces(s.positions, species, ei, edges[2], s.cell)
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    return {"value": len(s) / med, "unit": "atom-steps/s", "cores": threads, "kind": "port",
            "sample": f"{bc.name} E+F, float32 CPU restatement in the reference's CPU-path forms (torch, "
                      f"{threads} threads on {model}), median of {len(times)} step(s) after {nwarm} warm-up(s); "
                      f"{med * 1e3:.0f} ms/step"}


def layer_shapes(dm):
    """Per-layer widths (din, dhid, dmid, wn, slots per output degree) of a device model, at the
    engine's channel count (a narrower model runs zero-padded to it: this is the work executed)."""
    sys.path.insert(0, str(ROOT / "mace-mlx_amd" / "csrc"))
    import gen_tables
    layers = []
    for l in range(dm.dims["num_layers"]):
        lhid = dm.dims["layer_hid_blocks"][l]
        # input blocks of the conv TP: linear_up's output in a non-linear (mh-1) layer
        lin = dm.dims["layer_edge_blocks"][l] if dm.dims.get("nonlinear") else dm.dims["layer_in_blocks"][l]
        slots = gen_tables.tp_layout(lin)
        C = dm.dims["num_channels"]
        resid = not (l == 0 and dm.dims.get("first_nonresidual")) or bool(dm.dims.get("nonlinear"))
        layers.append(dict(lin=lin, lhid=lhid, C=C, resid=resid, nskip=min(lin, lhid) if resid else 0, din=C * lin * lin, dhid=C * lhid * lhid,
                           dmid=C * sum(2 * x[2] + 1 for x in slots), wn=C * len(slots),
                           nslot_by_l=[sum(1 for x in slots if x[2] == lo) for lo in range(4)]))
    return layers


def _setup(idx, separate=False, graphs=None, store_w=False):
    from mace_mlx_amd._ffi import Engine
    from mace_mlx_amd.device_model import build_device_model
    from mace_mlx_amd.model_io import random_init
    from mace_mlx_amd.systems import make_config
    bc = make_config(idx)
    weights = random_init(bc.model, 0)
    dm = build_device_model(bc.model, weights, dtype=bc.dtype)
    eng = Engine(0, channels=dm.dims["num_channels"])
    eng.load_model(dm)
    if separate:
        eng.set_fused_tp(False)
    if store_w:
        eng.set_rebuild_w(False)
    if graphs is not None:
        eng.set_graphs(graphs)
    zmap = {int(z): k for k, z in enumerate(dm.z_table)}
    species = np.array([zmap[int(z)] for z in bc.system.numbers], np.int32)
    eng.set_system(species, bc.system.cell, bc.system.pbc, 0.5)
    return bc, weights, dm, eng, species


def _timed(eng, pos_d, out_d, stress, steps, force_nl=False):
    """Wall time per step of `steps` device-resident steps, bracketed by device synchronisation."""
    import torch
    eng.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress, force_nl=force_nl)
    eng.sync()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def calculator_ms(bc, weights, warmup=3, reps=10):
    """The reference's end-to-end timing protocol (`docs/prototypes/xbench.py:89-101`): through
    the ASE calculator, `warmup` calls of get_potential_energy() + get_forces() with the results
    cleared before each, then the median over `reps` such calls (ms).  Also (min, max)."""
    import tempfile
    from mace_mlx_amd.calculators import MACECalculator
    from mace_mlx_amd.model_io import save_model
    with tempfile.TemporaryDirectory() as d:
        save_model(d, bc.model, weights)
        calc = MACECalculator(model_path=d, default_dtype=bc.dtype)
    atoms = bc.system.copy()
    ts = []
    for k in range(warmup + reps):
        calc.results = {}
        t0 = time.perf_counter()
        calc.get_potential_energy(atoms)
        calc.get_forces(atoms)
        if k >= warmup:
            ts.append(time.perf_counter() - t0)
    del calc
    return float(np.median(ts)) * 1e3, float(np.min(ts)) * 1e3, float(np.max(ts)) * 1e3


def run_workload(idx, steps, warmup, separate=False, graphs=None, extras=False, launch_order=None, store_w=False):
    """Measure one benchmark configuration: steady-state device-resident steps (neighbour
    list cached), steps that rebuild the neighbour list, and a per-launch-site pass with HIP
    events; with `extras` also the host-array path, the true-fp32 matrix-core variant and
    the CPU-baseline inputs."""
    import torch
    bc, weights, dm, eng, species = _setup(idx, separate, graphs, store_w)
    s = bc.system
    stress = "stress" in bc.properties
    E_host, _, F_host, _ = eng.step(s.positions, stress=stress)          # builds the neighbour list
    edges = eng.get_edges()
    N, E = len(s), len(edges[0])
    pos_d = torch.from_numpy(np.ascontiguousarray(s.positions, dtype=np.float64)).cuda()
    out_d = torch.zeros(10 + 3 * N, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    _timed(eng, pos_d, out_d, stress, warmup)
    wall = _timed(eng, pos_d, out_d, stress, steps)
    ms = wall / steps * 1e3
    out = out_d.cpu().numpy()
    assert abs(out[0] - E_host) <= 1e-9 * abs(E_host) and np.abs(out[10:].reshape(N, 3) - F_host).max() < 1e-9
    res = {"workload": bc.name, "n_atoms": N, "n_edges": E,
           "properties": "energy+forces+stress" if stress else "energy+forces", "feature_dtype": bc.dtype,
           "channels": bc.model.num_features, "engine_channels": dm.dims["num_channels"],
           "ms_per_step": round(ms, 4), "atom_steps_per_s": round(N / ms * 1e3, 1), "_wall": wall}
    if extras:
        # device-resident steps of a periodic system leave the positions of the last list build
        # on the device only, so the first host-array step rebuilds the list: warm up first
        for _ in range(max(warmup, 2)):
            eng.step(s.positions, stress=stress)
        # per-step wall times of back-to-back host-array steps: the median (the reference's
        # protocol) and the mean
        ts = []
        for _ in range(steps):
            th = time.perf_counter()
            eng.step(s.positions, stress=stress)
            ts.append(time.perf_counter() - th)
        res["ms_per_step_host_arrays"] = round(float(np.median(ts)) * 1e3, 4)
        res["ms_per_step_host_arrays_mean"] = round(float(np.mean(ts)) * 1e3, 4)
        med, lo, hi = calculator_ms(bc, weights)
        res["ms_per_step_calculator"] = round(med, 4)
        res["ms_per_step_calculator_range"] = [round(lo, 4), round(hi, 4)]
        if bc.dtype == "float32" and dm.dims["num_channels"] == 128:
            # the same step with every product on fp32 matrix cores (the 256-channel engine runs
            # the split-product path only)
            eng.set_split_products(False)
            _timed(eng, pos_d, out_d, stress, 2)
            res["ms_per_step_fp32_mfma"] = round(_timed(eng, pos_d, out_d, stress, steps) / steps * 1e3, 4)
            eng.set_split_products(True)
    eng.set_profiling(True)
    for _ in range(steps):
        eng.step_device(pos_d.data_ptr(), out_d.data_ptr(), stress=stress)
    kt = eng.kernel_times()
    order = eng.launch_order()
    eng.set_profiling(False)
    if launch_order:
        Path(launch_order).parent.mkdir(parents=True, exist_ok=True)
        Path(launch_order).write_text("\n".join(order) + "\n")
    layers = layer_shapes(dm)
    ctx = dict(N=N, E=E, C=dm.dims["num_channels"], nb=dm.dims["num_bessel"], layers=layers,
               linear_work=linear_work(layers, N),
               half=bc.dtype in ("float16", "bfloat16"),
               gx_bytes=2 if (bc.dtype == "float16" and not separate) else 4,
               fused=not separate)
    per_step = {k: (v[0] / steps, v[1] // steps) for k, v in kt.items()}
    dom = max(per_step, key=lambda k: per_step[k][0])
    launches = max(per_step[dom][1], 1)
    avg_ms = per_step[dom][0] / launches
    rl = roofline_of(dom, ctx, avg_ms)
    traffic = load_traffic(dom, bc.name)
    roof = {"bound": rl["bound"], "achieved": round(rl["achieved"], 3), "peak": rl["peak"], "unit": rl["unit"],
            "frac": round(rl["frac"], 4), "traffic": traffic, "kernel": dom, "avg_launch_ms": round(avg_ms, 5),
            "algorithmic_bytes": rl["algorithmic_bytes"], "algorithmic_flops": rl["algorithmic_flops"],
            "hbm_frac": round(rl["hbm_frac"], 4), "mfma_frac": round(rl["mfma_frac"], 4),
            "traffic_over_algorithmic_bytes": round(traffic / rl["algorithmic_bytes"], 2) if traffic else None,
            "boundary": ("radial-MLP output layer fused into the TP kernels: E*W -> E*64 in the TP bytes, "
                         "2*E*64*W flops added" if ctx["fused"] else "separate radial-MLP output pass")}
    res.update(dominant=dom, dominant_frac=roof["frac"], roofline=roof,
               tp_scatter=tp_scatter_summary(per_step, ctx), per_step=per_step, ctx=ctx)
    # steps that rebuild the neighbour list (the reference's benchmark.py:168-style number), after
    # two untimed ones (as the steady steps have their warm-up)
    nrb = max(8, steps // 2)
    _timed(eng, pos_d, out_d, stress, 2, force_nl=True)
    res["ms_per_step_nl_rebuild"] = round(_timed(eng, pos_d, out_d, stress, nrb, force_nl=True) / nrb * 1e3, 4)
    res["_edges"], res["_species"], res["_bc"], res["_weights"] = edges, species, bc, weights
    del eng, pos_d, out_d
    torch.cuda.empty_cache()
    return res


def kernel_table(per_step, ctx):
    tot = sum(v[0] for v in per_step.values())
    print(f"{'site':24s} {'ms/step':>9s} {'share':>6s} {'launch':>6s}  roofline (binding bound)", file=sys.stderr)
    for k, (t, n) in sorted(per_step.items(), key=lambda kv: -kv[1][0]):
        rl = roofline_of(k, ctx, t / max(n, 1))
        print(f"{k:24s} {t:9.4f} {t / tot * 100:5.1f}% {n:6d}  {rl['achieved']:9.2f} {rl['unit']} "
              f"({rl['frac'] * 100:.1f}% of {rl['bound']})", file=sys.stderr)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=1, help="benchmark configuration index 0..4 (5: an mh-1 model on the "
                    "Si1000 system; 6, 7: MACE-OFF-shaped models of 96 and 192 channels on an organic liquid)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--separate-mlp-out", action="store_true",
                    help="float32 policy: radial-MLP output layer as its own pass (not fused into the TP)")
    ap.add_argument("--store-w", action="store_true",
                    help="half-precision policies: the forward stores the per-edge weights and the VJP reads "
                         "them back (default: the VJP rebuilds them)")
    ap.add_argument("--kernel-table", action="store_true", help="print per-kernel times to stderr")
    ap.add_argument("--graphs", choices=("on", "off"), default=None,
                    help="replay the step through captured HIP graphs (on) or launch it eagerly (off); "
                         "default: the engine's default")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the bounded measurement of every benchmark configuration ('sweep' in the JSON)")
    ap.add_argument("--copy-calib-mb", type=float, default=0.0,
                    help="run a plain device copy of this size first (rocprof counter calibration)")
    ap.add_argument("--launch-order", default=None,
                    help="write the launch site of every dispatch of one profiled step to this file")
    ap.add_argument("--json-out", default=None, help="also write the JSON line to this file")
    ap.add_argument("--summarize", default=None, metavar="DIR",
                    help="no GPU: summarise a measurement directory (launch_order.txt, bench.json, rocprofv3 "
                         "trace/ and pmc_fetch/ pmc_write/ csv) into profiles/")
    args = ap.parse_args()
    if args.summarize:
        from mace_mlx_amd.rocprof_sites import summarize
        cmd = {}
        cf = Path(args.summarize) / "commands.json"
        if cf.exists():
            cmd = json.loads(cf.read_text())
        r = summarize(args.summarize, str(ROOT / "profiles"), args.copy_calib_mb or 256.0, cmd)
        print(json.dumps({"sites": len(r["sites"]), "steps": r["steps"], "traffic": "traffic" in r}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    import torch
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

    graphs = None if args.graphs is None else args.graphs == "on"
    head = run_workload(args.config, args.steps, args.warmup, args.separate_mlp_out, graphs, extras=True,
                        launch_order=args.launch_order, store_w=args.store_w)
    if args.kernel_table:
        kernel_table(head["per_step"], head["ctx"])
    sweep = None
    if not args.no_sweep:
        sweep = []
        for i in range(8):  # the five benchmark configurations, an mh-1 model on Si1000, MACE-OFF widths
            r = head if i == args.config else run_workload(i, max(5, args.steps // 2), args.warmup,
                                                           args.separate_mlp_out, graphs, store_w=args.store_w)
            sweep.append({k: r[k] for k in ("workload", "n_atoms", "n_edges", "properties", "feature_dtype",
                                             "channels", "engine_channels", "ms_per_step",
                                             "ms_per_step_nl_rebuild", "atom_steps_per_s", "dominant",
                                             "dominant_frac")}
                         | {"tp_scatter_hbm_frac_unfused_bytes": r["tp_scatter"]["hbm_frac_unfused_bytes"],
                            "tp_scatter_roofline_frac": r["tp_scatter"]["roofline_frac"]})
        print(f"{'config':24s} {'N':>6s} {'E':>9s} {'ms/step':>9s} {'+NL ms':>8s} {'atom-steps/s':>13s}  "
              f"dominant site (frac of its roofline)   TP+scatter HBM frac (unfused bytes)", file=sys.stderr)
        for r in sweep:
            print(f"{r['workload']:24s} {r['n_atoms']:6d} {r['n_edges']:9d} {r['ms_per_step']:9.3f} "
                  f"{r['ms_per_step_nl_rebuild']:8.3f} {r['atom_steps_per_s']:13.0f}  "
                  f"{r['dominant']:18s} ({r['dominant_frac']:.3f})   "
                  f"{r['tp_scatter_hbm_frac_unfused_bytes']:.3f}", file=sys.stderr)

    bc = head["_bc"]
    cpu = None if args.no_cpu_baseline else cpu_baseline(bc, head["_weights"], head["_edges"], head["_species"])
    N, E = head["n_atoms"], head["n_edges"]
    line = {
        "metric": "ms per energy+forces step (Si1000, medium arch, fp32); atom-steps/sec",
        "value": round(N * args.steps / head["_wall"], 1),
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "ms_per_step_host_arrays": head["ms_per_step_host_arrays"],
        "ms_per_step_host_arrays_mean": head["ms_per_step_host_arrays_mean"],
        "ms_per_step_calculator": head["ms_per_step_calculator"],
        "ms_per_step_calculator_range": head["ms_per_step_calculator_range"],
        "ms_per_step_nl_rebuild": head["ms_per_step_nl_rebuild"],
        "ms_per_step_fp32_mfma": head.get("ms_per_step_fp32_mfma"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float32": "fp32", "float16": "fp16 features / fp32 accumulation",
                  "bfloat16": "bf16 features / fp32 accumulation"}[bc.dtype],
        "data": "synthetic (seeded lattice + rattle, random-init weights)",
        "config": {"workload": bc.name, "n_atoms": N, "n_edges": E, "properties": head["properties"],
                   "neighbour_list": "cached (skin 0.5)"},
        "roofline": head["roofline"],
        "tp_scatter": head["tp_scatter"],
        "cpu_baseline": cpu,
    }
    if sweep is not None:
        line["sweep"] = sweep
    text = json.dumps(line)
    if args.json_out:
        Path(args.json_out).parent.mkdir(parents=True, exist_ok=True)
        Path(args.json_out).write_text(text + "\n")
    print(text)


if __name__ == "__main__":
    main()
