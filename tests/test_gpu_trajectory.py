"""Trajectory-level checks through the calculator on the GPU, as the reference runs them
through its own calculator: NVE energy conservation over many steps with neighbour-list
rebuilds and graph re-captures (`tests/test_md_stability.py:50-101`), the equation of state
P = -dE/dV against the stress (`tests/test_stress_extended.py:185-224`), and the stress against
finite differences of the energy (`tests/test_stress.py:210-255`).  ASE is not installed here,
so velocity Verlet is written out (ASE units: eV, Angstrom, amu; one time unit is 10.18 fs)."""

import numpy as np
import pytest

from gpu_helpers import Case, assert_parity
from mace_mlx_amd.systems import System, arch_config, diamond_si, rattle, write_model_dir

pytestmark = pytest.mark.gpu

FS = 0.09822694788464063   # 1 fs in ASE time units
KB = 8.617330337217213e-05  # eV / K
M_SI = 28.0855


@pytest.fixture(scope="module")
def calc(tmp_path_factory):
    from mace_mlx_amd import MACECalculator
    d = write_model_dir(arch_config("medium", zbl=True), tmp_path_factory.mktemp("m") / "si-medium-zbl", seed=3)
    return MACECalculator(model_path=str(d), device="cuda", skin=0.2)


def test_nve_energy_conservation_with_rebuilds(calc):
    """200 velocity-Verlet steps of 0.5 fs at 1500 K on Si216 (skin 0.2: rebuilds every few tens of
    steps).  Total energy drift is bounded, several rebuilds happen, and at the end the calculator
    still matches the float64 oracle on the final positions and a freshly built neighbour list."""
    s = rattle(diamond_si((3, 3, 3)), 0.02, 31)
    n = len(s)
    rng = np.random.default_rng(32)
    v = rng.normal(size=(n, 3)) * np.sqrt(KB * 1500.0 / M_SI)
    v -= v.mean(0)
    dt = 0.5 * FS

    def forces(pos):
        s.positions = pos
        calc.calculate(s, ["energy", "forces"])
        return calc.results["energy"], calc.results["forces"], calc.last_timings()[1] > 0

    e, f, _ = forces(s.positions.copy())
    etot, rebuilds = [], 0
    for step in range(200):
        pos = s.positions + v * dt + 0.5 * f / M_SI * dt * dt
        e, f_new, rebuilt = forces(pos)
        v = v + 0.5 * (f + f_new) / M_SI * dt
        f = f_new
        rebuilds += int(rebuilt)
        etot.append(e + 0.5 * M_SI * (v * v).sum())
    etot = np.array(etot)
    drift = (etot.max() - etot.min()) / n
    print(f"NVE: {rebuilds} rebuilds, drift {drift:.3e} eV/atom, E_pot {e:.4f}, max|F| {np.abs(f).max():.3f}",
          flush=True)
    assert rebuilds >= 2
    assert drift < 1e-4, drift   # measured 9e-6 eV/atom
    # the state after many rebuilds and re-captured graphs: oracle parity on the final geometry
    case = Case(arch_config("medium", zbl=True), seed=3)
    fresh = case.run(s, force_nl=True)
    assert abs(fresh["E"] - e) <= 1e-6 * abs(e) and np.abs(fresh["F"] - f).max() <= 1e-4
    ref = case.reference(s, fresh["sp"], case.edges())
    assert_parity({"E": e, "F": f, "ne": calc.results["node_energy"]}, ref, n)


def test_equation_of_state_pressure(calc):
    """P = -tr(stress)/3 against -dE/dV (np.gradient over 11 volumes within +-5 %, inner points), as
    `tests/test_stress_extended.py:185-224`; and against the float64 oracle's stress at each volume."""
    base = rattle(diamond_si((2, 2, 2)), 0.02, 33)
    V, E, P = [], [], []
    case = Case(arch_config("medium", zbl=True), seed=3)
    for k, sc in enumerate(np.linspace(0.95, 1.05, 11)):
        a = System(base.positions * sc, base.numbers, base.cell * sc, base.pbc)
        calc.calculate(a, ["energy", "stress"])
        st = calc.results["stress"]
        V.append(abs(np.linalg.det(a.cell)))
        E.append(calc.results["energy"])
        P.append(-(st[0] + st[1] + st[2]) / 3)
        if k % 5 == 0:
            got = case.run(a, stress=True)
            ref = case.reference(a, got["sp"], case.edges(), stress=True)
            voigt = np.array(ref["vir"])[[0, 1, 2, 1, 0, 0], [0, 1, 2, 2, 2, 1]] / V[-1]
            assert np.abs(st - voigt).max() <= 1e-5 * max(1e-3, np.abs(voigt).max()), (st, voigt)
    V, E, P = map(np.array, (V, E, P))
    Pn = -np.gradient(E, V)
    print(f"EOS: P_stress {P[2:-2]}, -dE/dV {Pn[2:-2]}", flush=True)
    np.testing.assert_allclose(P[2:-2], Pn[2:-2], atol=0.05 * max(1e-3, np.abs(P).max()) + 1e-4)


def test_stress_matches_energy_finite_differences(calc):
    """Every Voigt component of the calculator's stress against (E(+h) - E(-h)) / (2 h V) under a
    symmetric strain of a triclinic cell (`tests/test_stress.py:210-255`)."""
    cell = np.array([[7.1, 0.0, 0.0], [2.3, 6.8, 0.0], [-1.4, 1.9, 7.4]])
    g = np.stack(np.meshgrid(*[np.arange(k) for k in (3, 3, 4)], indexing="ij"), -1).reshape(-1, 3)
    frac = (g + 0.5) / np.array([3, 3, 4]) + np.random.default_rng(34).normal(scale=0.02, size=(36, 3))
    s = System(frac @ cell, np.full(36, 14), cell, np.array([True, True, True]))
    calc.calculate(s, ["energy", "stress"])
    st = np.array(calc.results["stress"])
    vol = abs(np.linalg.det(cell))
    h = 2e-3
    fd = []
    for a, b in ((0, 0), (1, 1), (2, 2), (1, 2), (0, 2), (0, 1)):
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h if a == b else h / 2
        es = []
        for sign in (1, -1):
            T = np.eye(3) + sign * eps
            calc.calculate(System(s.positions @ T, s.numbers, cell @ T, s.pbc), ["energy"])
            es.append(calc.results["energy"])
        fd.append((es[0] - es[1]) / (2 * h * vol))
    fd = np.array(fd)
    print(f"stress {st}\nFD     {fd}", flush=True)
    np.testing.assert_allclose(st, fd, atol=1e-3 * np.abs(st).max() + 2e-5)
