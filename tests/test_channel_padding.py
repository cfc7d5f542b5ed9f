"""Channel padding (model_io.pad_channels): a model of C channels, zero-padded to C' with the
path-weight compensation, gives the same energies and forces in the float64 oracle as the
original model evaluated directly (the oracle derives every path weight from the config's
irreps, so this pins the padding rule against the reference's normalisations,
`linear.py:46-74`, `tensor_product.py:1080-1098`)."""

import numpy as np
import pytest

from mace_mlx_amd.model_io import pad_channels, random_init, weight_shapes
from mace_mlx_amd.systems import arch_config, diamond_si, rattle
from oracle import model as om
from oracle.neighbors import neighbor_list


def _cfg(arch, C, **kw):
    cfg = arch_config(arch, **kw)
    cfg.hidden_irreps = "+".join(f"{C}x{b.ir}" for b in cfg.hidden)
    return cfg


@pytest.mark.parametrize("arch,C,kw", [
    ("small", 96, {}),
    ("medium", 96, {"zbl": True}),
    ("medium", 48, {"num_elements": 2, "z_table": [8, 14], "trained_topology": True}),
    ("large", 32, {}),
])
def test_padded_model_equals_original(arch, C, kw):
    cfg = _cfg(arch, C, **kw)
    w = random_init(cfg, 7)
    cfg2, w2 = pad_channels(cfg, w, 128)
    assert cfg2.num_features == 128
    assert {k: v.shape for k, v in w2.items()} == {k: tuple(s) for k, s in weight_shapes(cfg2).items()}
    s = rattle(diamond_si((1, 1, 1)), 0.05, 8)
    nel = cfg.num_elements
    sp = (np.arange(len(s)) % nel).astype(int)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max + 0.5)
    ei = np.stack([i, j])
    E1, F1, _ = om.OracleMACE(cfg=cfg, weights=w).energy_forces(s.positions, sp, ei, S, s.cell)
    E2, F2, _ = om.OracleMACE(cfg=cfg2, weights=w2).energy_forces(s.positions, sp, ei, S, s.cell)
    assert abs(E1 - E2) <= 1e-10 * max(1.0, abs(E1)), (E1, E2)
    np.testing.assert_allclose(F2, F1, atol=1e-9)


def test_padding_without_compensation_differs():
    """The sqrt(C'/C) factor matters: dropping it from the linears moves the energy."""
    cfg = _cfg("medium", 96)
    w = random_init(cfg, 9)
    cfg2, w2 = pad_channels(cfg, w, 128)
    bad = {k: (v / np.sqrt(128 / 96) if ".linear.weights." in k and k.startswith("interactions.1") else v)
           for k, v in w2.items()}
    s = rattle(diamond_si((1, 1, 1)), 0.05, 10)
    sp = np.zeros(len(s), dtype=int)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    ei = np.stack([i, j])
    E1 = om.OracleMACE(cfg=cfg2, weights=w2).energy(s.positions, sp, ei, S, s.cell)[0]
    E2 = om.OracleMACE(cfg=cfg2, weights=bad).energy(s.positions, sp, ei, S, s.cell)[0]
    assert abs(E1 - E2) > 1e-6 * max(1.0, abs(E1))


def test_padding_refuses_unequal_and_shrinking():
    cfg = _cfg("medium", 96)
    with pytest.raises(ValueError):
        pad_channels(cfg, random_init(cfg, 0), 64)
    cfg.hidden_irreps = "96x0e+64x1o"
    with pytest.raises(NotImplementedError):
        pad_channels(cfg, {}, 128)
