"""Pins the architecture bookkeeping (instruction lists, slot order, path weights)
against answers the reference itself holds, and the normalisations against the
second-moment property they are defined by.

* The layer-1 conv-TP instruction table of the medium architecture recorded in the
  reference (`docs/prototypes/teamA_convtp_batch.md:18-29`: i_in1, i_in2, i_out,
  (d1, d2, do), path weights 1 / 1.7321 / 2.2361 / 2.6458), its derived sizes
  (weight_numel 1280, K0 = 16, K1 = 24, OUTDIM = 5120:
  `docs/prototypes/team_metal_proto_mul21.py:4-15`, `teamA_convtp_batch.md:31-33`),
  checked for all three generators: the oracle's restatement, the product's
  `model_io.conv_tp_instructions` and the kernel-table generator `gen_tables`.
* The EquivariantLinear known answer of the reference's own test
  (`tests/test_linear.py:194-226`): `2x0e + 3x0e -> 1x0e` has two instructions with
  path weight 1/sqrt(5) and y = pw (x0 . w0 + x1 . w1).
* Component normalisation: with unit-variance inputs, component-normalised spherical
  harmonics and N(0, 1) weights every output component of a Linear, an FCTP and a
  conv TP has unit second moment (that is what the path weights are chosen for,
  `linear.py:46-74`, `tensor_product.py:1080-1098`, `utils.py:143-154`).  A dropped
  or misplaced path-weight factor moves some slot's moment by a factor 3/5/7 or
  its inverse and fails.
"""

import math

import numpy as np
import pytest
import torch

import gen_tables
from mace_mlx_amd import model_io
from mace_mlx_amd.irreps import Irreps
from oracle import model as om

# teamA_convtp_batch.md:18-29 -- (i_in1, i_in2, i_out, (d1, d2, do), path_weight)
REF_TABLE = [
    (0, 0, 0, (1, 1, 1), 1.0000),
    (1, 1, 1, (3, 3, 1), 1.0000),
    (0, 1, 2, (1, 3, 3), 1.7321),
    (1, 0, 3, (3, 1, 3), 1.7321),
    (1, 2, 4, (3, 5, 3), 1.7321),
    (0, 2, 5, (1, 5, 5), 2.2361),
    (1, 1, 6, (3, 3, 5), 2.2361),
    (1, 3, 7, (3, 7, 5), 2.2361),
    (0, 3, 8, (1, 7, 7), 2.6458),
    (1, 2, 9, (3, 5, 7), 2.6458),
]

IN1 = Irreps("128x0e+128x1o")
SH = Irreps("0e+1o+2e+3o")
TARGET = Irreps("128x0e+128x1o+128x2e+128x3o")


def _check_table(mid, inst):
    assert len(inst) == len(REF_TABLE)
    for (i1, i2, io, pw), (ri1, ri2, rio, dims, rpw) in zip(inst, REF_TABLE):
        assert (i1, i2, io) == (ri1, ri2, rio)
        assert (IN1[i1].ir.dim, SH[i2].ir.dim, mid[io].ir.dim) == dims
        assert abs(pw - rpw) < 5e-5
    # uvu with one weight per (instruction, channel): weight_numel = n_instr * 128
    assert sum(IN1[i1].mul * SH[i2].mul for i1, i2, _, _ in inst) == 1280
    assert mid.dim == 5120
    # scalar group (l1 = 0) output components K0 and l1 = 1 group K1
    assert sum(mid[io].ir.dim for i1, _, io, _ in inst if i1 == 0) == 16
    assert sum(mid[io].ir.dim for i1, _, io, _ in inst if i1 == 1) == 24
    assert sum(SH[i2].ir.dim * mid[io].ir.dim for i1, i2, io, _ in inst if i1 == 1) == 106


def test_convtp_table_oracle():
    mid, inst = om.conv_tp_instructions(IN1, SH, TARGET)
    _check_table(mid, inst)
    tp = om.ConvTP(IN1, SH, TARGET)
    assert tp.weight_numel == 1280


def test_convtp_table_product():
    mid, inst = model_io.conv_tp_instructions(IN1, SH, TARGET)
    _check_table(mid, inst)


def test_convtp_table_kernel_generator():
    slots = gen_tables.tp_layout(2)
    assert len(slots) == len(REF_TABLE)
    for slot, (i1, i2, io, dims, pw) in zip(slots, REF_TABLE):
        l1, l2, l3 = slot
        # blocks 0e, 1o of the input and 0e, 1o, 2e, 3o of the SH: index = degree
        assert (l1, l2) == (i1, i2)
        assert (2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1) == dims
        assert abs(gen_tables.tp_path_weight(slot) - pw) < 5e-5
    assert 128 * sum(2 * s[2] + 1 for s in slots) == 5120
    # the one-block layout (layer 0) is the l1 = 0 rows of the same table, in order
    assert gen_tables.tp_layout(1) == [s for s in slots if s[0] == 0]


def test_convtp_large_has_17_instructions():
    """Large layer 1 (`utils.py:118-124` with sources 0e / 1o / 2e): 4 + 6 + 7."""
    big = Irreps("128x0e+128x1o+128x2e")
    for gen in (om.conv_tp_instructions, model_io.conv_tp_instructions):
        mid, inst = gen(big, SH, TARGET)
        assert [sum(1 for t in inst if t[0] == b) for b in range(3)] == [4, 6, 7]
        assert 128 * len(inst) == 2176 and mid.dim == 9088
    slots = gen_tables.tp_layout(3)
    mid, inst = model_io.conv_tp_instructions(big, SH, TARGET)
    assert [(big[i1].ir.l, SH[i2].ir.l, mid[io].ir.l) for i1, i2, io, _ in inst] == slots


def test_linear_known_answer():
    """`tests/test_linear.py:194-226` of the reference."""
    ii, io = Irreps("2x0e+3x0e"), Irreps("1x0e")
    inst = model_io.linear_instructions(ii, io)
    assert [(a, b) for a, b, *_ in inst] == [(0, 0), (1, 0)]
    for t in inst:
        assert abs(t[-1] - 1.0 / math.sqrt(5.0)) < 1e-12
    rng = np.random.default_rng(0)
    w0, w1 = rng.normal(size=(2, 1)), rng.normal(size=(3, 1))
    lin = om.Linear(ii, io, [torch.tensor(w0), torch.tensor(w1)])
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0, 5.0]], dtype=torch.float64)
    y = lin(x).numpy()
    pw = 1.0 / math.sqrt(5.0)
    want = pw * (np.array([1.0, 2.0]) @ w0) + pw * (np.array([3.0, 4.0, 5.0]) @ w1)
    np.testing.assert_allclose(y[0], want, atol=1e-12)


# ---------------------------------------------------------------------------
# second moments
# ---------------------------------------------------------------------------

def _unit_sh(n, lmax, seed):
    v = torch.as_tensor(np.random.default_rng(seed).normal(size=(n, 3)))
    return om.spherical_harmonics(v, lmax)


def _moments(y, irreps):
    """Mean square per output block (averaged over samples, channels, components).
    Shared weight matrices make each block's moment a chi-square over its K x M
    weights; the multiplicities below keep that spread near 2-3 %."""
    out = []
    for b, off in zip(irreps, irreps.offsets):
        out.append(float((y[:, off:off + b.dim] ** 2).mean()))
    return np.array(out)


@pytest.mark.parametrize("spec_in,spec_out", [
    ("48x0e+32x0e+40x1o+24x1o+64x2e", "64x0e+48x1o+56x2e"),
    ("128x0e+128x1o", "128x0e+128x1o"),
])
def test_linear_unit_second_moment(spec_in, spec_out):
    ii, io = Irreps(spec_in), Irreps(spec_out)
    g = torch.Generator().manual_seed(1)
    ws = [torch.randn(a[2], a[3], generator=g, dtype=torch.float64)
          for a in model_io.linear_instructions(ii, io)]
    lin = om.Linear(ii, io, ws)
    x = torch.randn(4000, ii.dim, generator=g, dtype=torch.float64)
    m = _moments(lin(x), io)
    np.testing.assert_allclose(m, 1.0, rtol=0.06)


def test_fctp_unit_second_moment():
    """FCTP (uvw) with a generic second input: every output block has unit moment."""
    i1, n2 = Irreps("40x0e+32x1o+24x2e"), 5
    io = Irreps("48x0e+40x1o+32x2e")
    inst = model_io.fctp_instructions(i1, Irreps(f"{n2}x0e"), io)
    g = torch.Generator().manual_seed(2)
    ws = [torch.randn(i1[i].mul, n2, io[k].mul, generator=g, dtype=torch.float64)
          for i, _, k, _ in inst]
    fc = om.SkipFCTP(i1, n2, io, ws)
    x1 = torch.randn(6000, i1.dim, generator=g, dtype=torch.float64)
    x2 = torch.randn(6000, n2, generator=g, dtype=torch.float64)
    m = _moments(fc(x1, x2), io)
    np.testing.assert_allclose(m, 1.0, rtol=0.06)


@pytest.mark.parametrize("spec_in", ["32x0e", "32x0e+32x1o", "32x0e+32x1o+32x2e"])
def test_convtp_unit_second_moment(spec_in):
    """uvu conv TP: x ~ N(0,1), Y component-normalised over random directions,
    w ~ N(0,1) -> every output slot has unit second moment."""
    i1 = Irreps(spec_in)
    tgt = Irreps("32x0e+32x1o+32x2e+32x3o")
    tp = om.ConvTP(i1, SH, tgt)
    n = 6000
    g = torch.Generator().manual_seed(3)
    x1 = torch.randn(n, i1.dim, generator=g, dtype=torch.float64)
    Y = _unit_sh(n, 3, 4)
    w = torch.randn(n, tp.weight_numel, generator=g, dtype=torch.float64)
    m = _moments(tp(x1, Y, w), tp.mid)
    np.testing.assert_allclose(m, 1.0, rtol=0.07)


# ---------------------------------------------------------------------------
# ZBL pair repulsion against the published universal potential
# ---------------------------------------------------------------------------

# Ziegler, Biersack & Littmark, "The Stopping and Range of Ions in Solids" (1985), eq. 2-73:
# universal screening function with the published five-digit coefficients, universal
# screening length a_U = 0.8854 a0 / (Z1^0.23 + Z2^0.23).  a0 and e^2 / (4 pi eps0) from the
# CODATA 2018 constants (e, eps0, a0 in metres), not from the reference.
ZBL_PUBLISHED = ((0.18175, 3.19980), (0.50986, 0.94229), (0.28022, 0.40290), (0.028171, 0.20162))
_E_CHARGE, _EPS0, _A0_M = 1.602176634e-19, 8.8541878128e-12, 5.29177210903e-11
KE_EV_A = _E_CHARGE / (4.0 * math.pi * _EPS0) * 1e10      # eV * Angstrom
A0_A = _A0_M * 1e10


def _zbl_published(r, z1, z2):
    a = 0.8854 * A0_A / (z1 ** 0.23 + z2 ** 0.23)
    phi = sum(c * np.exp(-d * r / a) for c, d in ZBL_PUBLISHED)
    return KE_EV_A * z1 * z2 / r * phi


def _oracle_pair_energy(r, z1, z2):
    """Total ZBL energy of an isolated pair (both directed edges) from the oracle, with the
    universal screening parameters, and the envelope it applies."""
    r_t = torch.as_tensor(r, dtype=torch.float64)
    n = len(r)
    # edge k: atom 2k -> 2k+1 and back; each pair is its own system of two nodes
    zs = torch.tensor([z1, z2] * n)
    zr = torch.tensor([z2, z1] * n)
    rr = r_t.repeat_interleave(2)
    recv = torch.arange(2 * n).view(n, 2).flip(1).reshape(-1)
    e = om.zbl_node_energy(rr, zs, zr, recv, 2 * n, {"p": 6, "a_exp": 0.23, "a_prefactor": 0.8854})
    pair = e.view(n, 2).sum(1).numpy()
    rc = model_io.COVALENT_RADII[z1] + model_io.COVALENT_RADII[z2]
    env = om.poly_envelope(r_t / rc, 6).numpy()
    return pair, env


ZBL_PAIRS = [(14, 14), (6, 8), (26, 28), (1, 1), (1, 8), (8, 8)]


def _zbl_max_rel_dev():
    worst = 0.0
    for z1, z2 in ZBL_PAIRS:
        rc = model_io.COVALENT_RADII[z1] + model_io.COVALENT_RADII[z2]
        r = np.geomspace(0.05, min(2.0, 0.9 * rc), 50)
        pair, env = _oracle_pair_energy(r, z1, z2)
        assert np.all(env > 1e-3)
        worst = max(worst, float(np.abs(pair / env / _zbl_published(r, z1, z2) - 1.0).max()))
    return worst


def test_zbl_matches_published_universal_potential():
    """`radial.py:127-201` (oracle `zbl_node_energy`) at the universal screening parameters
    (a_exp 0.23, a_prefactor 0.8854) against the ZBL universal potential, r in [0.05, 2] A,
    envelope divided out.  The reference rounds the coefficients to four digits (0.4028
    for 0.40290, 3.2 for 3.1998) and a0 to 0.529 A: over these pairs and distances that
    moves V by at most 8.7e-4 relative (4.3e-4 for r <= 1 A), hence the 1.5e-3 bar.  Each
    pair's two directed edges carry half the energy each (0.5 factor)."""
    assert _zbl_max_rel_dev() < 1.5e-3


@pytest.mark.parametrize("mistake", ["swap_c01", "swap_d23", "a0_bohr_1", "coulomb_x2", "drop_c3"])
def test_zbl_pin_detects_planted_mistakes(monkeypatch, mistake):
    """The same comparison with a plausible misreading planted in the oracle fails by more than 1 %."""
    c, d = list(om.ZBL_C), list(om.ZBL_D)
    if mistake == "swap_c01":
        c[0], c[1] = c[1], c[0]
    elif mistake == "swap_d23":
        d[2], d[3] = d[3], d[2]
    elif mistake == "a0_bohr_1":
        monkeypatch.setattr(om, "ZBL_BOHR", 1.0)
    elif mistake == "coulomb_x2":
        monkeypatch.setattr(om, "ZBL_COULOMB", 2 * 14.3996)
    elif mistake == "drop_c3":
        c[3] = 0.0
    monkeypatch.setattr(om, "ZBL_C", tuple(c))
    monkeypatch.setattr(om, "ZBL_D", tuple(d))
    assert _zbl_max_rel_dev() > 1e-2


def test_zbl_screening_function_at_origin():
    """phi(0) = sum c_k = 1 up to the published rounding (the potential is unscreened Coulomb
    at r -> 0), and -phi'(0) = sum c_k d_k of the published set."""
    assert abs(sum(c for c, _ in ZBL_PUBLISHED) - 1.0) < 5e-6
    assert abs(sum(om.ZBL_C) - 1.0) < 2e-4          # four coefficients, each rounded by <= 5e-5
    slope_ref = sum(c * d for c, d in ZBL_PUBLISHED)
    assert abs(sum(c * d for c, d in zip(om.ZBL_C, om.ZBL_D)) / slope_ref - 1.0) < 1e-3


# ---------------------------------------------------------------------------
# plain radial MLP against torch's own modules
# ---------------------------------------------------------------------------

def test_radial_mlp_matches_torch_sequential():
    """`make_radial_mlp` (`radial.py:329-341`): nn.Sequential of Linear(bias=False) with
    SiLU between layers and none after the last.  The model file's keys
    `conv_tp_weights.layers.{k}.weight` index that Sequential (Linear at k = 0, 2, 4, 6),
    so the file's tensors load strictly into a torch.nn.Sequential built the same way;
    its output must equal the oracle's RadialMLP fed from the same file."""
    from mace_mlx_amd.systems import arch_config
    cfg = arch_config("medium")
    w = model_io.random_init(cfg, 5)
    m = om.OracleMACE(cfg=cfg, weights=w)
    x = torch.as_tensor(np.random.default_rng(0).normal(size=(257, cfg.num_bessel)), dtype=torch.float64)
    for li in range(cfg.num_interactions):
        p = f"interactions.{li}.conv_tp_weights.layers."
        keys = sorted((k for k in w if k.startswith(p)), key=lambda k: int(k[len(p):].split(".")[0]))
        idx = [int(k[len(p):].split(".")[0]) for k in keys]
        assert idx == [0, 2, 4, 6]
        sizes = [cfg.num_bessel] + list(cfg.radial_MLP) + [w[keys[-1]].shape[0]]
        mods = []
        for a in range(len(sizes) - 1):
            mods.append(torch.nn.Linear(sizes[a], sizes[a + 1], bias=False))
            if a < len(sizes) - 2:
                mods.append(torch.nn.SiLU())
        seq = torch.nn.Sequential(*mods).double()
        seq.load_state_dict({f"{k[len(p):]}": torch.as_tensor(w[k], dtype=torch.float64) for k in keys},
                            strict=True)
        with torch.no_grad():
            want = seq(x)
        got = m.layers[li]["mlp"](x)
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
        # not the identity-activation chain, and not SiLU after the last layer
        lin_only = x
        for k in keys:
            lin_only = lin_only @ torch.as_tensor(w[k], dtype=torch.float64).T
        assert (got - lin_only).abs().max() > 1e-2 * got.abs().max()


# ---------------------------------------------------------------------------
# density normalisation away from zero density
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("c", [0.35, 0.8, 1.6])
def test_density_normalisation_nonzero_density(c):
    """`blocks.py:366-380`: rho_i = sum over i's edges of tanh((ef . w)^2), message / (rho + 1).
    On an unrattled single-species diamond lattice with a first-shell neighbour list, every
    receiver has k = 4 edges of one length, so every edge has the same radial features ef;
    density weights w = c ef / |ef|^2 give ef . w = c on every edge, rho = 4 tanh(c^2) on every
    node, and the block must equal the plain block with avg_num_neighbors = 1 + 4 tanh(c^2).
    (tanh(c) in place of tanh(c^2), a dropped + 1, or a sum over senders of another shell
    would all move the energy.)"""
    from mace_mlx_amd.systems import arch_config, diamond_si
    from oracle.neighbors import neighbor_list
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14], trained_topology=True)
    w = model_io.random_init(cfg, 3)
    s = diamond_si((1, 1, 1))
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 3.0)
    assert len(i) == 4 * len(s)
    ei = np.stack([i, j])
    sp = np.ones(len(s), dtype=int)                       # all Si (z_table index 1)
    m0 = om.OracleMACE(cfg=cfg, weights=w)
    r = np.linalg.norm(s.positions[j] - s.positions[i] + S @ s.cell, axis=1)
    assert np.ptp(r) < 1e-12
    # the radial features of that length (the oracle's pinned Agnesi / Bessel / envelope)
    rt = torch.as_tensor(r[:1])
    z = torch.tensor([14])
    rb = om.agnesi(rt, z, z, m0.agnesi, m0.radii)
    ef = (om.bessel(rb, m0.bw, cfg.r_max)
          * om.poly_envelope(rt / cfg.r_max, cfg.num_polynomial_cutoff)[:, None])[0].numpy()
    dens = (c * ef / (ef @ ef))[None, :]
    wd = dict(w)
    for li in range(cfg.num_interactions):
        wd[f"interactions.{li}.density_fn.weight"] = dens
    E_dens = om.OracleMACE(cfg=cfg, weights=wd).energy(s.positions, sp, ei, S, s.cell)[0]
    cfg_plain = arch_config("medium", num_elements=2, z_table=[8, 14], trained_topology=True)
    cfg_plain.use_density_normalization = False
    cfg_plain.avg_num_neighbors = 1.0 + 4.0 * math.tanh(c * c)
    w_plain = {k: v for k, v in w.items() if not k.endswith("density_fn.weight")}
    E_plain = om.OracleMACE(cfg=cfg_plain, weights=w_plain).energy(s.positions, sp, ei, S, s.cell)[0]
    assert abs(E_dens - E_plain) < 1e-10 * max(1.0, abs(E_plain))
    # the same model at tanh(c) would differ
    cfg_plain.avg_num_neighbors = 1.0 + 4.0 * math.tanh(c)
    E_wrong = om.OracleMACE(cfg=cfg_plain, weights=w_plain).energy(s.positions, sp, ei, S, s.cell)[0]
    assert abs(E_dens - E_wrong) > 1e-4 * max(1.0, abs(E_plain))
