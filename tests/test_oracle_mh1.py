"""Pins of the oracle's mh-1 family restatement (`blocks.py:611-807`, `radial.py:344-357`,
`gate.py:19-164`, `blocks.py:493-537`), each against something other than a second
restatement: torch's own LayerNorm / Linear / SiLU modules, e3nn's normalize2mom constant,
equivariance, finite differences and the special cases the block reduces to."""

import math

import numpy as np
import pytest
import torch

from mace_mlx_amd.model_io import NONLINEAR_BLOCK, SIGMOID_NORM_FACTOR, SILU_NORM_FACTOR, random_init
from mace_mlx_amd.systems import arch_config, diamond_si, rattle
from oracle.model import Gate, OracleMACE, RadialMLPLN, layer_norm, spherical_harmonics
from oracle.neighbors import neighbor_list
from mace_mlx_amd.irreps import Irreps


def mh1_config(apply_cutoff=False, agnostic=True, edge="128x0e+128x1o", nel=3):
    c = arch_config("medium", num_elements=nel, z_table=[1, 6, 14][:nel])
    c.interaction_cls = NONLINEAR_BLOCK
    c.edge_irreps = edge
    c.apply_cutoff = apply_cutoff
    c.use_agnostic_product = agnostic
    return c


def _system(seed=3):
    s = rattle(diamond_si((1, 1, 1)), 0.05, seed)
    sp = np.array([0, 1, 2, 0, 1, 2, 2, 1])
    return s, sp


def test_layer_norm_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 64, generator=g, dtype=torch.float64) * 3 + 1
    w = torch.randn(64, generator=g, dtype=torch.float64)
    b = torch.randn(64, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.layer_norm(x, (64,), w, b, eps=1e-5)
    assert torch.allclose(layer_norm(x, w, b), ref, rtol=1e-12, atol=1e-12)
    y = layer_norm(x, torch.ones(64, dtype=torch.float64), torch.zeros(64, dtype=torch.float64))
    assert torch.allclose(y.mean(-1), torch.zeros(7, dtype=torch.float64), atol=1e-12)


def test_radial_mlp_layernorm_matches_torch_sequential():
    cfg = mh1_config()
    W = {k: torch.as_tensor(np.asarray(v, np.float64)) for k, v in random_init(cfg, seed=1).items()}
    pre = "interactions.1.conv_tp_weights"
    mlp = RadialMLPLN(W, pre)
    dims = [W[f"{pre}.layers.{3 * k}.weight"].shape for k in range(4)]
    mods = []
    for k, (o, i) in enumerate(dims):
        lin = torch.nn.Linear(i, o, dtype=torch.float64)
        lin.weight.data, lin.bias.data = W[f"{pre}.layers.{3 * k}.weight"], W[f"{pre}.layers.{3 * k}.bias"]
        mods.append(lin)
        if k < 3:
            ln = torch.nn.LayerNorm(o, dtype=torch.float64)
            ln.weight.data, ln.bias.data = W[f"{pre}.layers.{3 * k + 1}.weight"], W[f"{pre}.layers.{3 * k + 1}.bias"]
            mods += [ln, torch.nn.SiLU()]
    seq = torch.nn.Sequential(*mods)
    x = torch.randn(5, dims[0][1], dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    assert torch.allclose(mlp(x), seq(x), rtol=1e-12, atol=1e-12)


def test_sigmoid_norm_factor_is_e3nn_normalize2mom():
    g = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=g, dtype=torch.float64)
    assert abs(SIGMOID_NORM_FACTOR - torch.sigmoid(z).pow(2).mean().pow(-0.5).item()) < 1e-7


def test_gate_scalars_and_equivariance():
    irr = Irreps("4x0e+4x1o+4x2e+4x3o")
    gate = Gate(irr)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 4 + 12 + irr.dim - 4, dtype=torch.float64, generator=g)
    y = gate(x)
    assert y.shape == (6, irr.dim)
    # scalars: normalised SiLU; first gated block: normalised sigmoid of gate scalar k times vector k
    assert torch.allclose(y[:, :4], SILU_NORM_FACTOR * torch.nn.functional.silu(x[:, :4]))
    v = x[:, 16:28].reshape(6, 4, 3)
    want = SIGMOID_NORM_FACTOR * torch.sigmoid(x[:, 4:8])[:, :, None] * v
    assert torch.allclose(y[:, 4:16].reshape(6, 4, 3), want)
    # a rotation of the gated blocks commutes with the gate (gate scalars are invariant)
    R = torch.linalg.qr(torch.randn(3, 3, dtype=torch.float64, generator=g))[0]
    if torch.det(R) < 0:
        R = -R
    # D_l(R) of the real SH basis, fitted from Y(R v) = D Y(v) on random directions
    v = torch.randn(64, 3, dtype=torch.float64, generator=g)
    Yv, Yr = spherical_harmonics(v, 3), spherical_harmonics(v @ R.T, 3)

    def dmat(l):
        a, b = l * l, (l + 1) * (l + 1)
        return torch.linalg.lstsq(Yv[:, a:b], Yr[:, a:b]).solution.T

    def rot(t, off_in):
        out, off = [t[:, :off_in]], off_in
        for l in (1, 2, 3):
            D = dmat(l)
            blk = t[:, off:off + 4 * (2 * l + 1)].reshape(6, 4, 2 * l + 1)
            out.append((blk @ D.T).reshape(6, -1))
            off += 4 * (2 * l + 1)
        return torch.cat(out, -1)
    assert torch.allclose(gate(rot(x, 16)), rot(y, 4), atol=1e-12)


def _fd_forces(o, s, sp, ei, S, h=1e-5, atoms=(0, 3, 5)):
    out = []
    for k in atoms:
        for a in range(3):
            p = s.positions.copy()
            p[k, a] += h
            ep, _ = o.energy(p, sp, ei, S, s.cell)
            p[k, a] -= 2 * h
            em, _ = o.energy(p, sp, ei, S, s.cell)
            out.append(-(ep - em) / (2 * h))
    return np.array(out)


@pytest.mark.parametrize("apply_cutoff,agnostic", [(False, True), (True, False)])
def test_mh1_model_forces_stress_and_invariance(apply_cutoff, agnostic):
    cfg = mh1_config(apply_cutoff, agnostic)
    w = random_init(cfg, seed=5)
    o = OracleMACE(cfg=cfg, weights=w)
    s, sp = _system()
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max)
    ei = np.stack([i, j])
    E, F, voigt, ne, _ = o.energy_forces_stress(s.positions, sp, ei, S, s.cell)
    assert 0.05 < np.abs(F).max() < 500
    np.testing.assert_allclose(F.sum(0), 0, atol=1e-10)
    np.testing.assert_allclose(_fd_forces(o, s, sp, ei, S), F[[0, 3, 5]].reshape(-1), rtol=1e-6, atol=1e-8)
    # rotation (positions and cell), translation: same energy
    R = np.linalg.qr(np.random.default_rng(0).standard_normal((3, 3)))[0]
    Er, _ = o.energy(s.positions @ R.T + 0.37, sp, ei, S, s.cell @ R.T)
    assert abs(Er - E) < 1e-10 * max(1, abs(E))
    # stress: finite difference of the energy under a symmetric strain
    vol = abs(np.linalg.det(s.cell))
    h = 1e-6
    for a, b, v in ((0, 0, 0), (1, 2, 3)):
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h
        def en(e):
            T = np.eye(3) + e
            return o.energy(s.positions @ T, sp, ei, S, s.cell @ T)[0]
        d = (en(eps) - en(-eps)) / (2 * h) / vol
        want = d if a == b else d / 2
        assert abs(voigt[v] - want) < 1e-6 * max(1.0, abs(want)), (v, voigt[v], want)


def test_beta_zero_switches_the_density_off():
    cfg = mh1_config()
    w = random_init(cfg, seed=6)
    s, sp = _system(4)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max)
    ei = np.stack([i, j])
    w0 = dict(w)
    for li in range(2):
        w0[f"interactions.{li}.beta"] = np.asarray(0.0)
    w1 = dict(w0)
    for k in w1:
        if ".density_fn." in k:
            w1[k] = w1[k] * 3.0 + 0.5
    e0, _ = OracleMACE(cfg=cfg, weights=w0).energy(s.positions, sp, ei, S, s.cell)
    e1, _ = OracleMACE(cfg=cfg, weights=w1).energy(s.positions, sp, ei, S, s.cell)
    e2, _ = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, ei, S, s.cell)
    assert abs(e0 - e1) < 1e-12 * abs(e0) and abs(e0 - e2) > 1e-6 * abs(e0)


def test_agnostic_product_equals_copied_element_weights():
    """use_agnostic_product evaluates the contraction with all-ones attributes on one weight set
    (`blocks.py:510-533`): the same as an element-resolved product whose every element holds
    that set."""
    cfg = mh1_config(agnostic=True)
    w = random_init(cfg, seed=7)
    cfg2 = mh1_config(agnostic=False)
    w2 = dict(w)
    for k, v in w.items():
        if ".symmetric_contractions." in k:
            w2[k] = np.repeat(v, cfg.num_elements, axis=0)
    s, sp = _system(5)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max)
    ei = np.stack([i, j])
    e1, _ = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, ei, S, s.cell)
    e2, _ = OracleMACE(cfg=cfg2, weights=w2).energy(s.positions, sp, ei, S, s.cell)
    assert abs(e1 - e2) < 1e-12 * abs(e1)


def test_cutoff_applied_to_weights_and_density():
    """apply_cutoff=False (`radial.py:316-318`, `blocks.py:782-788`): an edge at r >= r_max
    contributes nothing even though its Bessel features are not zero."""
    cfg = mh1_config(apply_cutoff=False)
    w = random_init(cfg, seed=8)
    o = OracleMACE(cfg=cfg, weights=w)
    pos = np.array([[0.0, 0.0, 0.0], [1.9, 0.3, 0.2], [0.0, 6.05, 0.0]])
    sp = np.array([0, 2, 1])
    cell = np.eye(3) * 30
    i, j, S = neighbor_list(pos, cell, [False] * 3, 2 * cfg.r_max)   # includes pairs beyond r_max
    e_all, _ = o.energy(pos, sp, np.stack([i, j]), S, cell)
    keep = np.linalg.norm(pos[j] - pos[i], axis=1) < cfg.r_max
    e_in, _ = o.energy(pos, sp, np.stack([i[keep], j[keep]]), S[keep], cell)
    assert (~keep).any() and abs(e_all - e_in) < 1e-12 * abs(e_in)
