"""The benchmark's work model and the rocprofv3 site mapping (no GPU).

The algorithmic bytes of the edge TP + scatter follow the benchmark definition for
configuration 2 (Si1000 medium, N = 1000, E = 46,000): B_fwd = 106.0 / 261.2 MB and
B_bwd = 203.9 / 501.9 MB for layers 0 / 1, 1.073 GB per step; with the radial MLP's
output layer fused, E W -> E 64 plus 2 E 64 W flops per pass.
"""

import csv

import pytest

import bench
from mace_mlx_amd import rocprof_sites

LAYERS = [dict(lin=1, lhid=2, C=128, resid=True, nskip=1, din=128, dhid=512, dmid=2048, wn=512,
               nslot_by_l=[1, 1, 1, 1]),
          dict(lin=2, lhid=1, C=128, resid=True, nskip=1, din=512, dhid=128, dmid=5120, wn=1280,
               nslot_by_l=[2, 3, 3, 2])]


def _ctx(E=46000, fused=True):
    return dict(N=1000, E=E, nb=8, layers=LAYERS, linear_work=bench.linear_work(LAYERS, 1000),
                half=False, fused=fused)


@pytest.mark.parametrize("site,mb", [("tp_fwd.L0", 106.0), ("tp_fwd.L1", 261.2),
                                     ("tp_bwd.L0", 203.9), ("tp_bwd.L1", 501.9)])
def test_unfused_tp_bytes_match_definition(site, mb):
    b, f, _ = bench.site_work(site, _ctx(fused=False))
    assert abs(b / 1e6 - mb) < 0.1 and f == 0


def test_unfused_total_per_step():
    ps = {k: (0.1, 1) for k in ("tp_fwd.L0", "tp_fwd.L1", "tp_bwd.L0", "tp_bwd.L1", "tp_gather.L1")}
    r = bench.tp_scatter_summary(ps, _ctx(fused=True))
    assert abs(r["unfused_bytes"] / 1e9 - 1.073) < 0.001


def test_fused_boundary():
    b, f, pk = bench.site_work("tp_bwd.L1", _ctx(E=46002))
    assert abs(b / 1e6 - 54.4) < 0.05 and abs(f / 1e9 - 7.537) < 0.01 and pk == bench.FP32_MFMA_PEAK_TFS
    r = bench.roofline_of("tp_bwd.L1", _ctx(E=46002), 0.1662)
    assert r["bound"] == "mfma" and abs(r["frac"] - 0.288) < 0.002 and abs(r["hbm_frac"] - 0.041) < 0.001


def test_linear_work_counts_the_fused_skip():
    """The skip connection's product is counted where it runs: operand 2 of linear_prod and
    of linear_up_bwd; a non-residual first block has a message-skip site (four blocks) and no
    skip operand."""
    N, CC = 1000, 128 * 128
    w = bench.linear_work(LAYERS, N)
    assert w["linear_prod.L0"][0] == 2 * N * (1 + 3 + 1) * CC          # PLin blocks 0, 1 + skip block 0
    assert w["linear_prod_bwd.L0"][0] == 2 * N * (1 + 3) * CC
    assert w["linear_up_bwd.L1"][0] == 2 * N * (1 + 3 + 1) * CC        # Up blocks 0, 1 + skip block 0
    assert "message_skip.L0" not in w
    nonres = [dict(LAYERS[0], resid=False, nskip=0)]
    w = bench.linear_work(nonres, N)
    assert w["message_skip.L0"][0] == w["message_skip_bwd.L0"][0] == 2 * N * 16 * CC
    assert w["linear_prod.L0"][0] == 2 * N * 4 * CC


def _write_trace(path, names):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, ["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 0
        for n in names:
            w.writerow({"Kernel_Name": n, "Start_Timestamp": t, "End_Timestamp": t + 10})
            t += 20


def test_site_mapping_keeps_only_steady_steps(tmp_path):
    order = ["edge_fwd", "tp_fwd.L0", "tp_fwd.L0", "forces"]        # one site with two dispatches
    step = ["k_edge_fwd", "k_fill_zero", "k_tpx_fwd<1>", "k_forces"]
    rebuild = ["k_nl_bin", "k_nl_count", "k_edge_fwd", "k_embed", "k_fill_zero", "k_tpx_fwd<1>", "k_forces"]
    names = step + rebuild[:2] + step + step + ["k_edge_fwd", "k_embed"] + step[1:] + step
    _write_trace(tmp_path / "t.csv", names)
    rows = list(csv.DictReader(open(tmp_path / "t.csv")))
    acc, kname, n = rocprof_sites.site_durations(rows, order)
    assert n == 3   # the step followed by NL kernels and the one with an embed upload are dropped
    assert len(acc["tp_fwd.L0"]) == 6 and kname["forces"] == "k_forces"
