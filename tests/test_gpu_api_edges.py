"""GPU tests of the model-object API and of the reference's degenerate inputs.

* ``load_model`` returns a callable ``MACE`` / ``ScaleShiftMACE`` (`model.py:440-484,550-589,
  664-720`): energies per graph, node energies and the interaction energy against the float64
  oracle, for one structure and a batch of two.
* Overlapping atoms: two atoms at one position give a zero-length edge, whose length the
  reference clamps (`utils.py:79-83`) and whose spherical harmonics and Bessel features stay
  finite (`spherical_harmonics.py:113-117`, `radial.py:63-70`).
* ``skin <= 0`` rebuilds the neighbour list at every step (`calculators.py:278-279`).
"""

import numpy as np
import pytest

from gpu_helpers import Case, assert_parity, bruteforce_edges, edge_set
from mace_mlx_amd.model_io import random_init, save_model
from mace_mlx_amd.systems import System, arch_config, diamond_si, rattle
from oracle.model import OracleMACE
from oracle.neighbors import neighbor_list

pytestmark = pytest.mark.gpu


def _scaleshift_cfg():
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14], zbl=True)
    cfg.model_type = "ScaleShiftMACE"
    cfg.scale, cfg.shift = 1.7, -0.3
    cfg.atomic_energies = [-2.1, -4.6]
    return cfg


def test_load_model_callable(tmp_path):
    from mace_mlx_amd import ScaleShiftMACE, load_model
    cfg = _scaleshift_cfg()
    w = random_init(cfg, 21)
    save_model(tmp_path / "m", cfg, w)
    model = load_model(str(tmp_path / "m"))
    assert isinstance(model, ScaleShiftMACE)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 22)
    s.numbers = np.where(np.arange(len(s)) % 4 == 0, 8, 14)
    sp = (s.numbers == 14).astype(np.int64)
    onehot = np.eye(2)[sp]
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max + 0.5)
    ei = np.stack([i, j])
    out = model(s.positions, onehot, ei, S.astype(np.float64), cell=s.cell)
    ref = OracleMACE(cfg=cfg, weights=w)
    E, F, ne = ref.energy_forces(s.positions, sp, ei, S, s.cell)
    print(f"load_model: E {out['energy'][0]:.6f} ref {E:.6f}", flush=True)
    assert out["energy"].shape == (1,)
    assert abs(out["energy"][0] - E) <= 1e-6 * abs(E)
    assert np.abs(out["node_energy"] - ne).max() <= 1e-5 * max(1.0, np.abs(ne).max())
    e0 = np.array(cfg.atomic_energies)[sp].sum()
    assert abs(out["interaction_energy"][0] - (E - e0)) <= 1e-5 * max(1.0, abs(E))
    # energy and forces of the same call (calculators.py:440-476)
    e, ne2, f, _ = model.energy_forces(s.positions, onehot, ei, S, cell=s.cell)
    assert_parity({"E": e, "F": f, "ne": ne2}, {"E": E, "F": F, "ne": ne}, len(s))
    # a batch of two copies, the second translated: per-graph energies (utils.py:35-44)
    n = len(s)
    pos2 = np.concatenate([s.positions, s.positions + np.array([0.3, -0.2, 0.1])])
    ei2 = np.concatenate([ei, ei + n], axis=1)
    S2 = np.concatenate([S, S])
    batch = np.repeat([0, 1], n)
    out2 = model(pos2, np.concatenate([onehot, onehot]), ei2, S2, cell=s.cell, batch=batch, num_graphs=2)
    assert out2["energy"].shape == (2,)
    for g in range(2):
        assert abs(out2["energy"][g] - E) <= 1e-6 * abs(E), (g, out2["energy"])
        assert abs(out2["interaction_energy"][g] - (E - e0)) <= 1e-5 * max(1.0, abs(E))
    model.close()


def test_overlapping_atoms_zero_length_edge():
    """Atoms 4 and 5 of a 14-atom cluster share one position: the zero-length edges between them
    get r = 1e-12 (the clamp), Y = (1, 0, ..., 0) and the Bessel r -> 0 limit.  Energies and node
    energies match the oracle; the two atoms' forces carry the clamp's 1 / r factor through
    d(v / r) / dv (as the reference's autograd does) and match the oracle to 1e-5 of their size;
    every other atom's force meets the absolute bar."""
    case = Case(arch_config("medium"), seed=23)
    rng = np.random.default_rng(24)
    pos = rng.uniform(0.0, 5.0, size=(14, 3)) + 20.0
    pos[5] = pos[4]
    s = System(pos, np.full(14, 14), np.eye(3) * 50.0, np.array([False, False, False]))
    got = case.run(s)
    edges = case.edges()
    assert edge_set(*edges) == bruteforce_edges(s)
    snd, rcv, _ = edges
    assert np.count_nonzero((snd == 4) & (rcv == 5)) == 1 and np.count_nonzero((snd == 5) & (rcv == 4)) == 1
    ref = case.reference(s, got["sp"], edges)
    assert np.isfinite(got["E"]) and np.all(np.isfinite(got["F"])) and np.all(np.isfinite(got["ne"]))
    dE = abs(got["E"] - ref["E"])
    print(f"overlap: E {got['E']:.6f} ref {ref['E']:.6f}; |F4| {np.abs(ref['F'][4]).max():.3e}", flush=True)
    assert dE <= 1e-6 * abs(ref["E"])
    assert np.abs(got["ne"] - ref["ne"]).max() <= 1e-5 * max(1.0, np.abs(ref["ne"]).max())
    rest = np.setdiff1d(np.arange(14), [4, 5])
    assert np.abs(got["F"][rest] - ref["F"][rest]).max() <= 1e-4
    for a in (4, 5):
        scale = np.abs(ref["F"][a]).max()
        assert np.abs(got["F"][a] - ref["F"][a]).max() <= 1e-5 * scale, (a, got["F"][a], ref["F"][a])


def test_skin_zero_rebuilds_every_step():
    """skin = 0: every step rebuilds the list (`calculators.py:278-279`), also when no atom moved,
    and each step matches the oracle on its freshly built list (five builds on the same cell and
    buffers, each against the brute-force list)."""
    case = Case(arch_config("small"), seed=25)
    s = rattle(diamond_si((2, 2, 2)), 0.03, 26)
    sp = np.zeros(len(s), dtype=np.int32)
    case.eng.set_system(sp, s.cell, s.pbc, 0.0)
    for k in range(5):
        pos = s.positions + 0.004 * k
        E, ne, F, _ = case.eng.step(pos)
        assert case.eng.timings()[1] > 0, f"step {k} did not rebuild the neighbour list"
        moved = System(pos, s.numbers, s.cell, s.pbc)
        edges = case.edges()
        assert edge_set(*edges) == bruteforce_edges(moved, cutoff=6.0)   # r_max + skin
        assert_parity({"E": E, "F": F, "ne": ne}, case.reference(moved, sp, edges), len(s))
    # and with a positive skin a step that moves nothing does not rebuild
    case.eng.set_system(sp, s.cell, s.pbc, 0.5)
    case.eng.step(s.positions)
    case.eng.step(s.positions)
    assert case.eng.timings()[1] == 0


def test_mace_off_small_width_96():
    """A MACE-OFF-small-shaped model (96x0e, ten elements, r_max 5 A, non-residual first block,
    ScaleShiftMACE) runs as its zero-padded 128-channel equivalent; E, F and stress against the
    float64 oracle evaluating the original 96-channel model."""
    from mace_mlx_amd.systems import off_config, organic_cluster
    cfg = off_config("small")
    case = Case(cfg, seed=42)
    assert case.dm.dims["num_channels"] == 128
    s = organic_cluster()
    got = case.run(s)
    edges = case.edges()
    assert edge_set(*edges) == bruteforce_edges(s, cutoff=5.5)
    assert_parity(got, case.reference(s, got["sp"], edges), len(s))
    per = rattle(diamond_si((2, 2, 2)), 0.05, 43)
    per.positions *= 0.7                       # C-C distances of ~1.6 A
    per.cell *= 0.7
    per.numbers = np.full(len(per), 6)
    got = case.run(per, stress=True)
    edges = case.edges()
    assert_parity(got, case.reference(per, got["sp"], edges, stress=True), len(per), stress=True)


def test_mace_off_calculator_from_cache(tmp_path, monkeypatch):
    """``mace_off("small")`` resolves the converted model from the reference's cache layout
    (`<cache>/off-small/v2`) and evaluates it through the ASE calculator API."""
    from mace_mlx_amd import mace_off
    from mace_mlx_amd.systems import off_config, organic_cluster
    cfg = off_config("small")
    w = random_init(cfg, 44)
    save_model(tmp_path / "off-small" / "v2", cfg, w)
    monkeypatch.setenv("MACE_MLX_CACHE_DIR", str(tmp_path))
    calc = mace_off("small", device="cuda")
    s = organic_cluster(30, 45)
    calc.calculate(s, ["energy", "forces"])
    z = {int(v): k for k, v in enumerate(cfg.z_table)}
    sp = np.array([z[int(a)] for a in s.numbers])
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max + 0.5)
    E, F, ne = OracleMACE(cfg=cfg, weights=w).energy_forces(s.positions, sp, np.stack([i, j]), S, s.cell)
    assert_parity({"E": calc.results["energy"], "F": calc.results["forces"], "ne": calc.results["node_energy"]},
                  {"E": E, "F": F, "ne": ne}, len(s))


def test_mace_off_large_width_192():
    """A MACE-OFF-large-shaped model (192x0e + 192x1o + 192x2e: three input blocks, the l1 = 2
    CG paths) runs natively on the 192-channel engine (libmace_hip_c192.so: three 64-channel
    slices, grouped products whose output widths are not multiples of 128); E, F and stress
    against the float64 oracle.  That engine runs the default path only: the comparison paths
    raise before any launch."""
    from mace_mlx_amd.systems import off_config, organic_cluster
    cfg = off_config("large")
    case = Case(cfg, seed=46)
    assert case.dm.dims["num_channels"] == 192 and case.eng.channels == 192
    s = organic_cluster(40, 47)
    print("192-channel model on the 192-channel engine: organic cluster", flush=True)
    got = case.run(s)
    edges = case.edges()
    assert edge_set(*edges) == bruteforce_edges(s, cutoff=5.5)
    assert_parity(got, case.reference(s, got["sp"], edges), len(s))
    per = rattle(diamond_si((2, 2, 2)), 0.05, 48)
    per.positions *= 0.7
    per.cell *= 0.7
    per.numbers = np.full(len(per), 6)
    print("192-channel model on the 192-channel engine: periodic carbon with stress", flush=True)
    got = case.run(per, stress=True)
    assert_parity(got, case.reference(per, got["sp"], case.edges(), stress=True), len(per), stress=True)
    case.eng.set_split_products(False)
    with pytest.raises(NotImplementedError):
        case.run(per)
    case.eng.set_split_products(True)
    case.eng.set_fused_tp(False)
    with pytest.raises(NotImplementedError):
        case.run(per)
    case.eng.set_fused_tp(True)


def test_width_224_on_the_256_engine():
    """A medium-shaped model with 224 channels runs on the 256-channel engine as its zero-padded
    equivalent (model_io.pad_channels); E, F and stress against the float64 oracle evaluating the
    224-channel model."""
    cfg = arch_config("medium", zbl=True)
    cfg.hidden_irreps = "224x0e+224x1o"
    case = Case(cfg, seed=49)
    assert case.dm.dims["num_channels"] == 256 and case.eng.channels == 256
    s = rattle(diamond_si((2, 2, 2)), 0.04, 50)
    print("224-channel model on the 256-channel engine: Si64 with stress", flush=True)
    got = case.run(s, stress=True)
    edges = case.edges()
    assert edge_set(*edges) == bruteforce_edges(s)
    assert_parity(got, case.reference(s, got["sp"], edges, stress=True), len(s), stress=True)


def test_dense_rows_longer_than_recorded_hits():
    """A compressed diamond lattice (a = 3.6 A, about 190 neighbours per atom within r_max +
    skin): the count pass records at most 128 hits per receiver on the first build, so every row
    is written by a second full visit; the next build records them all (its capacity follows the
    first build's mean row) and writes the rows from the recorded hits.  Both builds give the
    brute-force edge set and oracle parity (the sender-side CSR comes from the same pass)."""
    case = Case(arch_config("small"), seed=27)
    s = rattle(diamond_si((2, 2, 2), a=3.6), 0.02, 28)
    for k in range(2):
        got = case.run(s, force_nl=True)
        edges = case.edges()
        n_e = len(edges[0])
        print(f"dense build {k}: {n_e} edges, {n_e / len(s):.1f} per atom", flush=True)
        assert n_e / len(s) > 128
        assert edge_set(*edges) == bruteforce_edges(s)
        assert_parity(got, case.reference(s, got["sp"], edges), len(s))
