"""Pins the CPU oracle against closed forms, reference-held numbers and invariants.

Nothing here compares the oracle with itself: each check is a closed form
(e3nn's l<=2 harmonics, the SH addition theorem, Bessel / envelope formulas), a
number the reference recorded (edge counts of `docs/prototypes/profile_results.json`),
or a physical invariant the reference tests through its calculator
(`tests/test_forces.py`, `tests/test_stress.py`, `tests/test_materials.py`).
"""

import math

import numpy as np
import pytest
import torch

from mace_mlx_amd.model_io import COVALENT_RADII, random_init, weight_shapes
from mace_mlx_amd.systems import arch_config, diamond_si, make_config, rattle
from oracle import model as om
from oracle.neighbors import neighbor_list


def _unit(n, seed=0):
    v = np.random.default_rng(seed).normal(size=(n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def test_sh_low_orders_closed_form():
    """l=0,1 (spherical_harmonics.py:125-140) and e3nn's closed l=2 forms."""
    u = _unit(50)
    Y = om.spherical_harmonics(torch.tensor(u * 2.7), 3).numpy()
    x, y, z = u.T
    np.testing.assert_allclose(Y[:, 0], 1.0, atol=1e-14)
    np.testing.assert_allclose(Y[:, 1:4], math.sqrt(3) * u, atol=1e-14)
    s15 = math.sqrt(15)
    l2 = np.stack([s15 * x * z, s15 * x * y, math.sqrt(5) * (y ** 2 - 0.5 * (x ** 2 + z ** 2)),
                   s15 * y * z, s15 / 2 * (z ** 2 - x ** 2)], axis=1)
    np.testing.assert_allclose(Y[:, 4:9], l2, atol=1e-12)


@pytest.mark.parametrize("l", [0, 1, 2, 3])
def test_sh_addition_theorem(l):
    """sum_m Y_lm(a) Y_lm(b) = (2l+1) P_l(a.b) in component normalisation."""
    a, b = _unit(40, 1), _unit(40, 2)
    Ya = om.spherical_harmonics(torch.tensor(a), 3).numpy()[:, l * l:(l + 1) ** 2]
    Yb = om.spherical_harmonics(torch.tensor(b), 3).numpy()[:, l * l:(l + 1) ** 2]
    c = (a * b).sum(1)
    P = np.polynomial.legendre.legval(c, [0] * l + [1])
    np.testing.assert_allclose((Ya * Yb).sum(1), (2 * l + 1) * P, atol=1e-12)


def test_sh_zero_vector_finite():
    Y = om.spherical_harmonics(torch.zeros(1, 3, dtype=torch.float64), 3)
    assert torch.isfinite(Y).all()


def test_bessel_and_envelope_closed_form():
    r_max, p = 6.0, 5
    w = torch.arange(1, 9, dtype=torch.float64) * math.pi / r_max
    r = torch.tensor([0.0, 0.5, 2.35, 5.9], dtype=torch.float64)
    B = om.bessel(r, w, r_max).numpy()
    for i, rv in enumerate(r.tolist()):
        for n in range(8):
            want = math.sqrt(2 / r_max) * (w[n].item() if rv == 0 else math.sin(w[n].item() * rv) / rv)
            assert abs(B[i, n] - want) < 1e-12
    u = torch.tensor([0.0, 0.3, 0.999999, 1.0, 1.5], dtype=torch.float64)
    env = om.poly_envelope(u, p).numpy()
    assert env[0] == 1.0 and env[3] == 0.0 and env[4] == 0.0
    assert abs(env[2]) < 1e-9  # vanishes like (1-u)^3
    # C1 continuity at u = 1: derivative of the polynomial vanishes there
    uu = torch.tensor([1.0 - 1e-6], dtype=torch.float64, requires_grad=True)
    (g,) = torch.autograd.grad(om.poly_envelope(uu, p).sum(), uu)
    assert abs(g.item()) < 1e-8


def test_zbl_limits():
    """phi(0) = sum c_k and V -> 14.3996 Z^2 / r * 0.5 at short range."""
    r = torch.tensor([1e-8], dtype=torch.float64)
    z = torch.tensor([14])
    e = om.zbl_node_energy(r, z, z, torch.tensor([0]), 1, {"p": 6})
    assert abs(e.item() / (0.5 * 14.3996 * 14 * 14 / 1e-8) - (0.1818 + 0.5099 + 0.2802 + 0.02817)) < 1e-6
    far = om.zbl_node_energy(torch.tensor([2.3], dtype=torch.float64), z, z, torch.tensor([0]), 1, {"p": 6})
    assert far.item() == 0.0  # beyond 2 * r_cov(Si) = 2.22 A


def test_neighbor_counts_match_reference():
    """n_edges 2944 (Si64) and 46000 (Si1000) of profile_results.json; diamond shells."""
    s = diamond_si((2, 2, 2))
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    assert len(i) == 2944
    s = diamond_si((5, 5, 5))
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    assert len(i) == 46000
    d = np.linalg.norm(s.positions[j] - s.positions[i] + S @ s.cell, axis=1)
    shells = np.unique(np.round(d, 3), return_counts=True)
    np.testing.assert_allclose(shells[0], [2.351, 3.840, 4.502, 5.430, 5.917], atol=2e-3)
    assert (shells[1] == np.array([4, 12, 12, 6, 12]) * 1000).all()


def test_neighbor_pairing_and_unwrapped_positions():
    s = rattle(diamond_si((2, 2, 2)), 0.05, 3)
    shift = np.array([[1, -2, 0]]) @ s.cell   # unwrap a few atoms by lattice vectors
    pos = s.positions.copy()
    pos[::5] += shift
    i, j, S = neighbor_list(pos, s.cell, s.pbc, 6.5)
    d = np.linalg.norm(pos[j] - pos[i] + S @ s.cell, axis=1)
    assert (d < 6.5).all()
    fw = set(zip(i.tolist(), j.tolist(), map(tuple, S.tolist())))
    bw = set(zip(j.tolist(), i.tolist(), map(tuple, (-S).tolist())))
    assert fw == bw
    i0, j0, S0 = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    assert len(i0) == len(i)


# ---------------------------------------------------------------------------
# whole-model invariants (float64)
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def si64():
    cfg = arch_config("medium", zbl=True)
    w = random_init(cfg, 0)
    m = om.OracleMACE(cfg=cfg, weights=w)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 11)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    return m, s, np.stack([i, j]), S


def test_forces_match_finite_differences(si64):
    m, s, ei, S = si64
    sp = np.zeros(len(s), int)
    E, F, _ = m.energy_forces(s.positions, sp, ei, S, s.cell)
    h = 1e-4
    for a, k in [(0, 0), (5, 1), (17, 2), (40, 0)]:
        p1, p2 = s.positions.copy(), s.positions.copy()
        p1[a, k] += h
        p2[a, k] -= h
        fd = -(m.energy(p1, sp, ei, S, s.cell)[0] - m.energy(p2, sp, ei, S, s.cell)[0]) / (2 * h)
        assert abs(fd - F[a, k]) < 1e-6 * max(1.0, abs(F[a, k]))
    np.testing.assert_allclose(F.sum(0), 0.0, atol=1e-10)


def test_translation_rotation_invariance(si64):
    m, s, ei, S = si64
    sp = np.zeros(len(s), int)
    E, F, _ = m.energy_forces(s.positions, sp, ei, S, s.cell)
    Et, Ft, _ = m.energy_forces(s.positions + np.array([0.3, -1.7, 2.2]), sp, ei, S, s.cell)
    assert abs(Et - E) < 1e-9 * abs(E)
    np.testing.assert_allclose(Ft, F, atol=1e-9)
    q = np.linalg.qr(np.random.default_rng(5).normal(size=(3, 3)))[0]
    R = q * np.sign(np.linalg.det(q))
    Er, Fr, _ = m.energy_forces(s.positions @ R.T, sp, ei, S, s.cell @ R.T)
    assert abs(Er - E) < 1e-9 * abs(E)
    np.testing.assert_allclose(Fr, F @ R.T, atol=1e-9)


def test_permutation_invariance(si64):
    m, s, ei, S = si64
    sp = np.zeros(len(s), int)
    E, F, _ = m.energy_forces(s.positions, sp, ei, S, s.cell)
    perm = np.random.default_rng(2).permutation(len(s))
    inv = np.argsort(perm)
    Ep, Fp, _ = m.energy_forces(s.positions[perm], sp, inv[ei], S, s.cell)
    assert abs(Ep - E) < 1e-9 * abs(E)
    np.testing.assert_allclose(Fp, F[perm], atol=1e-9)


def test_stress_finite_differences_and_forces(si64):
    m, s, ei, S = si64
    sp = np.zeros(len(s), int)
    E, F, st, ne, vir = m.energy_forces_stress(s.positions, sp, ei, S, s.cell)
    E2, F2, _ = m.energy_forces(s.positions, sp, ei, S, s.cell)
    np.testing.assert_allclose(F, F2, atol=1e-12)  # test_stress.py:118-146
    np.testing.assert_allclose(vir, vir.T, atol=1e-10)
    # symmetric strain eps(t): pos' = pos (1 + eps), cell' = cell (1 + eps); dE/dt = vir[a, b]
    h = 1e-5
    vol = abs(np.linalg.det(s.cell))
    for a, b in [(0, 0), (1, 2), (2, 1), (0, 1)]:
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h if a == b else h / 2

        def e_at(sg):
            T = np.eye(3) + sg * eps
            return m.energy(s.positions @ T, sp, ei, S, s.cell @ T)[0]

        fd = (e_at(1) - e_at(-1)) / (2 * h)
        assert abs(fd - vir[a, b]) < 1e-5 * max(1.0, abs(fd))
    np.testing.assert_allclose(st, (vir / vol)[[0, 1, 2, 1, 0, 0], [0, 1, 2, 2, 2, 1]])


def test_single_atom_and_far_pair():
    """test_materials.py:250-265: isolated atoms feel no force."""
    cfg = arch_config("small")
    m = om.OracleMACE(cfg=cfg, weights=random_init(cfg, 0))
    pos = np.array([[0.0, 0.0, 0.0]])
    E, F, ne = m.energy_forces(pos, np.zeros(1, int), np.zeros((2, 0), int), np.zeros((0, 3)), np.eye(3) * 20)
    assert np.abs(F).max() == 0.0 and np.isfinite(E)
    pos2 = np.array([[0.0, 0.0, 0.0], [10.0, 0.0, 0.0]])
    E2, F2, ne2 = m.energy_forces(pos2, np.zeros(2, int), np.zeros((2, 0), int), np.zeros((0, 3)), np.eye(3) * 30)
    assert np.abs(F2).max() == 0.0
    assert abs(E2 - 2 * E) < 1e-12


def test_symmetric_contraction_equals_dense_definition():
    """Row-compressed main step == einsum strings of symmetric_contraction.py:95-121."""
    from mace_mlx_amd.cg import u_matrix
    from mace_mlx_amd.irreps import Irrep, Irreps
    rng = np.random.default_rng(0)
    b, c, nel = 3, 4, 2
    coupling = Irreps("0e+1o+2e+3o")
    for lout in ("0e", "1o", "2e"):
        U3, U2, U1 = (u_matrix(coupling, lout, nu) for nu in (3, 2, 1))
        W3, W2, W1 = (torch.tensor(rng.normal(size=(nel, U.shape[-1], c))) for U in (U3, U2, U1))
        f = torch.tensor(rng.normal(size=(b, c, 16)))
        sp = torch.tensor([0, 1, 1])
        con = om.Contraction(coupling, Irrep.parse(lout), 3, W3, [W2, W1], torch.float64)
        got = con(f, sp).numpy()
        oh = np.eye(nel)[sp.numpy()]
        pre = "" if lout == "0e" else "w"
        main = np.einsum(f"{pre}xyik,ekc,bci,be->bc{pre}xy", U3, W3.numpy(), f.numpy(), oh)
        c2 = np.einsum(f"{pre}xyk,ekc,be->bc{pre}xy", U2, W2.numpy(), oh) + main
        out = np.einsum(f"bc{pre}xi,bci->bc{pre}x", c2, f.numpy())
        c1 = np.einsum(f"{pre}xk,ekc,be->bc{pre}x", U1, W1.numpy(), oh) + out
        out = np.einsum(f"bc{pre}i,bci->bc{pre}", c1, f.numpy())
        want = out.reshape(b, -1)
        np.testing.assert_allclose(got, want, atol=1e-10)


# ---------------------------------------------------------------------------
# trained-model topology (Agnesi transform, density normalisation, non-residual
# first interaction)
# ---------------------------------------------------------------------------

def test_agnesi_transform_closed_form():
    """radial.py:231-262: t(x) = 1 / (1 + a x^q / (1 + x^(q-p))), x = r / r0."""
    prm = {"q": 0.9183, "p": 4.5791, "a": 1.0805}
    radii = torch.tensor(COVALENT_RADII, dtype=torch.float64)
    r0 = 0.5 * (COVALENT_RADII[14] + COVALENT_RADII[8])
    r = torch.tensor([r0, 0.5 * r0, 2.0 * r0, 1e-9, 50.0], dtype=torch.float64)
    z1, z2 = torch.full((5,), 14), torch.full((5,), 8)
    t = om.agnesi(r, z1, z2, prm, radii).numpy()
    assert abs(t[0] - 1.0 / (1.0 + prm["a"] / 2.0)) < 1e-14          # x = 1
    x = 0.5
    assert abs(t[1] - 1.0 / (1.0 + prm["a"] * x ** prm["q"] / (1.0 + x ** (prm["q"] - prm["p"])))) < 1e-14
    assert t[3] > 1.0 - 1e-6                                          # r -> 0: t -> 1
    xl = 50.0 / r0                                                    # r -> inf: t ~ 1 / (1 + a x^q)
    assert abs(t[4] * (1.0 + prm["a"] * xl ** prm["q"]) - 1.0) < 1e-4
    assert np.all(np.diff(t[[3, 1, 0, 2, 4]]) < 0)                    # decreasing in r


@pytest.fixture(scope="module")
def mpa():
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14], trained_topology=True)
    w = random_init(cfg, 3)
    m = om.OracleMACE(cfg=cfg, weights=w)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 12)
    s.numbers = np.where(np.arange(len(s)) % 3 == 0, 8, 14)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    sp = (s.numbers == 14).astype(int)
    return cfg, w, m, s, np.stack([i, j]), S, sp


def test_trained_topology_forces_stress_and_invariance(mpa):
    cfg, w, m, s, ei, S, sp = mpa
    E, F, st, ne, vir = m.energy_forces_stress(s.positions, sp, ei, S, s.cell)
    h = 1e-4
    for a, k in [(0, 0), (7, 1), (33, 2)]:
        p1, p2 = s.positions.copy(), s.positions.copy()
        p1[a, k] += h
        p2[a, k] -= h
        fd = -(m.energy(p1, sp, ei, S, s.cell)[0] - m.energy(p2, sp, ei, S, s.cell)[0]) / (2 * h)
        assert abs(fd - F[a, k]) < 1e-6 * max(1.0, abs(F[a, k]))
    np.testing.assert_allclose(F.sum(0), 0.0, atol=1e-10)
    q = np.linalg.qr(np.random.default_rng(7).normal(size=(3, 3)))[0]
    R = q * np.sign(np.linalg.det(q))
    Er, Fr, _ = m.energy_forces(s.positions @ R.T, sp, ei, S, s.cell @ R.T)
    assert abs(Er - E) < 1e-9 * abs(E)
    np.testing.assert_allclose(Fr, F @ R.T, atol=1e-9)


def test_density_normalisation_reduces_to_unit_average(mpa):
    """With density_fn = 0 every edge density is tanh(0) = 0, so dividing by (density + 1)
    is the plain block with avg_num_neighbors = 1 (blocks.py:372-380 vs 262-264)."""
    cfg, w, m, s, ei, S, sp = mpa
    w0 = {k: (np.zeros_like(v) if k.endswith("density_fn.weight") else v) for k, v in w.items()}
    cfg_plain = arch_config("medium", num_elements=2, z_table=[8, 14], trained_topology=True)
    cfg_plain.use_density_normalization = False
    w_plain = {k: v for k, v in w.items() if not k.endswith("density_fn.weight")}
    E0 = om.OracleMACE(cfg=cfg, weights=w0).energy(s.positions, sp, ei, S, s.cell)[0]
    E1 = om.OracleMACE(cfg=cfg_plain, weights=w_plain).energy(s.positions, sp, ei, S, s.cell)[0]
    assert abs(E0 - E1) < 1e-10 * abs(E1)


def test_nonresidual_first_block_with_identity_skip():
    """blocks.py:68-176: the non-residual block applies its skip FCTP to the message.
    With W[u, z, w] = delta_uw sqrt(C n_el) (path weight 1/sqrt(C n_el), 3j = I/sqrt(2l+1))
    that FCTP is the identity, so the model equals the residual layout with a zero
    first-layer skip."""
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14])
    cfg.first_interaction_nonresidual = True
    w = random_init(cfg, 4)
    C, nel = 128, 2
    eye = np.zeros((C, nel, C))
    for z in range(nel):
        eye[:, z, :] = np.eye(C) * math.sqrt(C * nel)
    w_id = {k: (eye if k.startswith("interactions.0.skip_tp.") else v) for k, v in w.items()}
    cfg_res = arch_config("medium", num_elements=2, z_table=[8, 14])
    w_res = {k: v for k, v in w.items() if not k.startswith("interactions.0.skip_tp.")}
    for k, shp in weight_shapes(cfg_res).items():
        if k.startswith("interactions.0.skip_tp."):
            w_res[k] = np.zeros(shp)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 13)
    sp = (np.arange(len(s)) % 2).astype(int)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    ei = np.stack([i, j])
    Ea = om.OracleMACE(cfg=cfg, weights=w_id).energy(s.positions, sp, ei, S, s.cell)[0]
    Eb = om.OracleMACE(cfg=cfg_res, weights=w_res).energy(s.positions, sp, ei, S, s.cell)[0]
    assert abs(Ea - Eb) < 1e-9 * max(1.0, abs(Eb))


@pytest.mark.parametrize("lin_irreps", ["8x0e", "8x0e+8x1o", "8x0e+8x1o+8x2e"])
def test_gemm_form_tp_equals_loop_form(lin_irreps):
    """The x2-first GEMM form of the conv TP (the reference's CPU path, `tensor_product.py:545-575`,
    used to time the CPU baseline) equals the per-instruction loop form."""
    import torch
    from mace_mlx_amd.irreps import Irreps
    from oracle.model import ConvTP, ConvTPGemm, spherical_harmonics
    irr = Irreps(lin_irreps)
    sh = Irreps.spherical_harmonics(3)
    target = Irreps([(8, b.ir) for b in sh])
    g = torch.Generator().manual_seed(1)
    loop, gemm = ConvTP(irr, sh, target), ConvTPGemm(irr, sh, target)
    E = 11
    x1 = torch.randn(E, irr.dim, dtype=torch.float64, generator=g)
    Y = spherical_harmonics(torch.randn(E, 3, dtype=torch.float64, generator=g), 3)
    w = torch.randn(E, loop.weight_numel, dtype=torch.float64, generator=g)
    assert torch.allclose(gemm(x1, Y, w), loop(x1, Y, w), rtol=1e-12, atol=1e-12)
