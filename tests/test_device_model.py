"""Host-side folding of the reference model into the engine's tensors.

The tensors handed to the HIP library (path weights, CG factors, 1/avg_num_neighbors
and ScaleShift folded in; component-major block layouts) and the generated TP /
symmetric-contraction tables are re-evaluated in float64 on the CPU
(tests/kernel_model.py) and compared with the oracle, for every architecture.
"""

import numpy as np
import pytest
import torch

import kernel_model
from mace_mlx_amd.device_model import UnsupportedModel, build_device_model, round_weights_bf16
from mace_mlx_amd.model_io import ModelConfig, random_init, weight_shapes
from mace_mlx_amd.systems import arch_config, diamond_si, lattice, rattle, _FCC
from oracle.model import OracleMACE
from oracle.neighbors import neighbor_list


@pytest.fixture(scope="module")
def si64():
    s = rattle(diamond_si((2, 2, 2)), 0.05, 1)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    return s, i, j, S


@pytest.mark.parametrize("arch", ["small", "medium", "large"])
@pytest.mark.parametrize("zbl", [False, True])
def test_kernel_formulation_matches_oracle(si64, arch, zbl):
    s, i, j, S = si64
    cfg = arch_config(arch, zbl=zbl)
    w = random_init(cfg, 3)
    sp = np.zeros(len(s), int)
    Eo, neo = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, np.stack([i, j]), S, s.cell)
    Ek, nek = kernel_model.energy(build_device_model(cfg, w), s.positions, sp, i, j, S.astype(float), s.cell)
    np.testing.assert_allclose(nek, neo, atol=5e-6)
    assert abs(Ek - Eo) < 1e-6 * max(1.0, abs(Eo)) * len(s)


def test_scaleshift_and_multielement():
    """ScaleShiftMACE (model.py:550-589) folded into readouts / ZBL / e0; 3 species."""
    base = lattice(_FCC, 3.6, (2, 2, 2), 26)
    rng = np.random.default_rng(0)
    base.numbers = np.array([26, 28, 24])[rng.integers(0, 3, len(base))]
    s = rattle(base, 0.05, 2)
    cfg = arch_config("medium", num_elements=3, z_table=[24, 26, 28], zbl=True,
                      atomic_energies=[-3.0, -1.5, 0.25])
    cfg.model_type = "ScaleShiftMACE"
    cfg.scale, cfg.shift = 1.7, -0.3
    w = random_init(cfg, 5)
    zmap = {24: 0, 26: 1, 28: 2}
    sp = np.array([zmap[z] for z in s.numbers])
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    Ek, nek = kernel_model.energy(build_device_model(cfg, w), s.positions, sp, i, j, S.astype(float), s.cell)
    # oracle: plain MACE energy terms, then scale/shift applied as in ScaleShiftMACE
    plain = arch_config("medium", num_elements=3, z_table=[24, 26, 28], zbl=True,
                        atomic_energies=[0.0, 0.0, 0.0])
    m = OracleMACE(cfg=plain, weights={**w, "atomic_energies_fn.atomic_energies": np.zeros(3, np.float32)})
    _, ne_inter = m.energy(s.positions, sp, np.stack([i, j]), S, s.cell)
    e0 = np.array([-3.0, -1.5, 0.25])[sp]
    want = e0 + 1.7 * ne_inter - 0.3
    np.testing.assert_allclose(nek, want, atol=1e-5)


def test_weight_inventory_matches_reference_layout():
    cfg = arch_config("medium", zbl=True)
    shapes = weight_shapes(cfg)
    # key names of converter.py / the MLX module tree
    for key in ["interactions.1.conv_tp_weights.layers.6.weight",
                "products.0.symmetric_contractions.contractions.1.weights_max",
                "products.0.symmetric_contractions.contractions.1.weights.1",
                "interactions.0.skip_tp.tp.weights.0", "readouts.1.linear_2.weights.0"]:
        assert key in shapes
    assert shapes["interactions.1.conv_tp_weights.layers.6.weight"] == (1280, 64)
    assert shapes["products.0.symmetric_contractions.contractions.1.weights_max"] == (1, 51, 128)
    assert shapes["interactions.1.linear.weights.0"] == (128, 128)
    assert sum(k.startswith("interactions.1.linear.weights") for k in shapes) == 10


def test_unsupported_topologies_raise():
    cfg = arch_config("medium")
    w = random_init(cfg, 0)
    bad = ModelConfig.from_dict({**cfg.to_dict(), "hidden_irreps": "128x0e+64x1o"})
    with pytest.raises((UnsupportedModel, NotImplementedError, KeyError)):
        build_device_model(bad, w)
    # a separate cutoff exists only in the non-linear (mh-1) block here; the non-linear block
    # with the density / non-residual layout of the 0b2 family is not a reference topology
    for upd in ({"apply_cutoff": False},
                {"interaction_cls": "RealAgnosticResidualNonLinearInteractionBlock",
                 "first_interaction_nonresidual": True}):
        bad2 = ModelConfig.from_dict({**cfg.to_dict(), **upd})
        with pytest.raises(NotImplementedError):
            build_device_model(bad2, w)


def test_float16_policy_rounds_all_but_pinned_weights():
    """float16 models (`model.py:705-711`): every weight array becomes fp16 except the
    atomic energies and the Bessel frequencies (`_pin_float32`, `model.py:627-647`)."""
    from mace_mlx_amd.device_model import FP32_PINNED, round_weights_fp16
    cfg = arch_config("medium")
    w = random_init(cfg, 0)
    w16 = round_weights_fp16(w)
    assert set(w16) == set(w)
    for k, v in w16.items():
        v = np.asarray(v, dtype=np.float64)
        if k in FP32_PINNED:
            np.testing.assert_array_equal(v, np.asarray(w[k], dtype=np.float64))
        else:
            np.testing.assert_array_equal(v, v.astype(np.float16).astype(np.float64))
    bessel = "radial_embedding.bessel_fn.bessel_weights"
    assert not np.array_equal(np.asarray(w[bessel]).astype(np.float16).astype(np.float64), np.asarray(w[bessel]))
    dm16 = build_device_model(cfg, w, dtype="float16")
    dm_r = build_device_model(cfg, w16, dtype="float32")
    assert dm16.dims["feature_half"] == 1 and dm_r.dims["feature_half"] == 0
    for k in dm16.tensors:   # the half model is the float32 fold of the rounded weights
        np.testing.assert_array_equal(dm16.tensors[k], dm_r.tensors[k])
    with pytest.raises(UnsupportedModel):
        build_device_model(cfg, w, dtype="float64")


def test_bf16_rounding_matches_torch():
    """to_bf16 against torch's own float32 -> bfloat16 conversion (round to nearest, ties to
    even): random magnitudes across the exponent range, exact ties, values next to ties,
    subnormals, signed zeros, infinities and the largest finite bf16 neighbourhood."""
    import torch
    from mace_mlx_amd.device_model import to_bf16
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-140, 120, 20000))).astype(np.float32)
    base = rng.integers(0, 1 << 16, 4000, dtype=np.uint64) << 16
    ties = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001]).astype(np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, 1e-45, -1e-40, np.inf, -np.inf, 3.3895314e38, 3.38e38, 1.0, -1.00390625],
                       np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)], special])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float64).numpy()
    np.testing.assert_array_equal(to_bf16(x), want)
    assert np.array_equal(np.signbit(to_bf16(x)), np.signbit(want))
    # NaNs stay NaN with their sign, including the patterns the 0x7fff carry would turn into
    # -0.0 (0x7fffffff), +0.0 (0xffffffff) or an infinity (0x7f800001)
    nans = np.array([0x7FFFFFFF, 0xFFFFFFFF, 0x7F800001, 0xFF800001, 0x7FC00000, 0x7FBFFFFF, 0xFFC12345],
                    np.uint32).view(np.float32)
    got = to_bf16(nans)
    assert np.isnan(got).all()
    assert np.array_equal(np.signbit(got), np.signbit(nans))
    assert np.isnan(torch.from_numpy(nans).to(torch.bfloat16).to(torch.float64).numpy()).all()


def test_bfloat16_policy_rounds_all_but_pinned_weights():
    """bfloat16 models (`model.py:592-596,705-711`): every weight array becomes bf16 except the
    pinned ones; the device model is the float32 fold of those rounded weights with feature
    policy 2, and the non-linear block stays float32-only."""
    from mace_mlx_amd.device_model import FP32_PINNED, round_weights_bf16, to_bf16
    cfg = arch_config("medium")
    w = random_init(cfg, 0)
    wb = round_weights_bf16(w)
    for k, v in wb.items():
        v = np.asarray(v, dtype=np.float64)
        if k in FP32_PINNED:
            np.testing.assert_array_equal(v, np.asarray(w[k], dtype=np.float64))
        else:
            np.testing.assert_array_equal(v, to_bf16(v))
    up = "interactions.0.linear_up.weights.0"
    assert not np.array_equal(wb[up], np.asarray(w[up], np.float64))
    dmb = build_device_model(cfg, w, dtype="bfloat16")
    dm_r = build_device_model(cfg, wb, dtype="float32")
    assert dmb.dims["feature_half"] == 2
    for k in dmb.tensors:
        np.testing.assert_array_equal(dmb.tensors[k], dm_r.tensors[k])
    # mh-1 models take the bf16 policy too: their fold is the float32 fold of the rounded weights
    from test_oracle_mh1 import mh1_config
    c1 = mh1_config()
    w1 = random_init(c1, 0)
    d1, d1r = build_device_model(c1, w1, dtype="bfloat16"), build_device_model(c1, round_weights_bf16(w1))
    assert d1.dims["feature_half"] == 2
    for k in d1.tensors:
        np.testing.assert_array_equal(d1.tensors[k], d1r.tensors[k])


def _multihead_cfg(heads, **kw):
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14], zbl=True, **kw)
    cfg.heads = list(heads)
    return cfg


def test_multi_head_oracle_pinned_by_embedding():
    """The oracle's multi-head readouts (every head evaluated, the non-linear readout's
    features masked to the active head, the active column taken; `model.py:302-326`,
    `blocks.py:553-608`) pinned by embedding a single-head model as head "b" of a two-head
    model: the single-head weights become head b's columns, `linear_2`'s rows scaled by
    sqrt(2) because its path weight drops from 1/sqrt(16) to 1/sqrt(32) (`linear.py:46-74`).
    Head b must then reproduce the single-head energies exactly, and head a must not."""
    s, i, j, S = _two_species_system()
    one = arch_config("medium", num_elements=2, z_table=[8, 14], zbl=True, atomic_energies=[-2.0, -1.0])
    w1 = random_init(one, 7)
    two = _multihead_cfg(["a", "b"], atomic_energies=[[0.5, 0.25], [-2.0, -1.0]])
    w2 = {k: v.astype(np.float64) for k, v in random_init(two, 8).items()}
    last = f"readouts.{one.num_interactions - 1}"
    w2["atomic_energies_fn.atomic_energies"] = np.array([[0.5, 0.25], [-2.0, -1.0]], np.float32)
    for k, v in w1.items():
        if k.startswith("readouts.") and ".linear.weights." in k:
            w2[k][:, 1:2] = v
        elif k.startswith(f"{last}.linear_1."):
            w2[k][:, 16:32] = v
        elif k.startswith(f"{last}.linear_2."):
            w2[k][16:32, 1:2] = v * np.sqrt(2.0)
        elif k != "atomic_energies_fn.atomic_energies":
            w2[k] = v
    sp = np.array([0 if z == 8 else 1 for z in s.numbers])
    ei = np.stack([i, j])
    E1, ne1 = OracleMACE(cfg=one, weights=w1).energy(s.positions, sp, ei, S, s.cell)
    Eb, neb = OracleMACE(cfg=two, weights=w2, head="b").energy(s.positions, sp, ei, S, s.cell)
    Ea, nea = OracleMACE(cfg=two, weights=w2, head="a").energy(s.positions, sp, ei, S, s.cell)
    np.testing.assert_allclose(neb, ne1, rtol=0, atol=1e-10)
    assert abs(Ea - E1) > 1e-3
    with pytest.raises(ValueError):
        OracleMACE(cfg=two, weights=w2, head="nope")


def _two_species_system():
    s = rattle(diamond_si((2, 2, 2)), 0.05, 11)
    s.numbers = np.where(np.arange(len(s)) % 4 == 0, 8, 14)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, 6.5)
    return s, i, j, S


@pytest.mark.parametrize("head", ["pbe", "r2scan", "third"])
def test_multi_head_selection_matches_oracle(head):
    """build_device_model(head=...) keeps one head's readouts, E0 row and ScaleShift
    entry (`model_io.select_head`); the folded tensors, re-evaluated in float64, equal the
    oracle's evaluation of the full three-head ScaleShiftMACE.  The shift list is shorter
    than the head list, so head "third" takes entry 0 (`model.py:530-548`)."""
    s, i, j, S = _two_species_system()
    cfg = _multihead_cfg(["pbe", "r2scan", "third"],
                         atomic_energies=[[-3.0, -1.5], [0.5, 0.25], [1.0, -0.75]])
    cfg.model_type = "ScaleShiftMACE"
    cfg.scale, cfg.shift = [1.7, 0.8, 1.1], [-0.3, 0.2]
    w = random_init(cfg, 9)
    sp = np.array([0 if z == 8 else 1 for z in s.numbers])
    Eo, neo = OracleMACE(cfg=cfg, weights=w, head=head).energy(s.positions, sp, np.stack([i, j]), S, s.cell)
    dm = build_device_model(cfg, w, head=head)
    Ek, nek = kernel_model.energy(dm, s.positions, sp, i, j, S.astype(float), s.cell)
    np.testing.assert_allclose(nek, neo, atol=5e-6)
    assert abs(Ek - Eo) < 1e-6 * max(1.0, abs(Eo)) * len(s)


def test_scaleshift_oracle_matches_definition():
    """The oracle's ScaleShiftMACE (`model.py:550-589`: e0 + scale x (pair + readouts) +
    shift per atom) against the plain-MACE terms of the same weights."""
    s, i, j, S = _two_species_system()
    cfg = arch_config("medium", num_elements=2, z_table=[8, 14], zbl=True, atomic_energies=[-3.0, 0.5])
    w = random_init(cfg, 4)
    sp = np.array([0 if z == 8 else 1 for z in s.numbers])
    ei = np.stack([i, j])
    _, ne_plain = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, ei, S, s.cell)
    cfg.model_type = "ScaleShiftMACE"
    cfg.scale, cfg.shift = 1.3, -0.4
    _, ne_ss = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, ei, S, s.cell)
    e0 = np.array([-3.0, 0.5])[sp]
    np.testing.assert_allclose(ne_ss, e0 + 1.3 * (ne_plain - e0) - 0.4, atol=1e-10)


def test_head_selection_errors_and_single_head():
    cfg = _multihead_cfg(["a", "b"])
    w = random_init(cfg, 0)
    with pytest.raises(ValueError):
        build_device_model(cfg, w, head="c")
    one = arch_config("medium")
    one.heads = ["Default"]
    w1 = random_init(one, 0)
    dm_a = build_device_model(one, w1, head="anything")   # single-head models ignore head
    dm_b = build_device_model(arch_config("medium"), w1)
    for k in dm_b.tensors:
        np.testing.assert_array_equal(dm_a.tensors[k], dm_b.tensors[k])


@pytest.mark.parametrize("apply_cutoff,agnostic,edge", [(False, True, "128x0e+128x1o"), (True, False, "128x0e+128x1o"),
                                                        (False, True, "128x0e+128x1o+128x2e")])
def test_mh1_kernel_formulation_matches_oracle(apply_cutoff, agnostic, edge):
    """mh-1 family: the engine's folded tensors (per-species first-layer tables, gate-input
    column layout, path weights) re-evaluated on the CPU equal the oracle's energy."""
    from test_oracle_mh1 import _system, mh1_config
    cfg = mh1_config(apply_cutoff, agnostic, edge)
    w = random_init(cfg, seed=9)
    s, sp = _system(6)
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cfg.r_max)
    E, ne = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, np.stack([i, j]), S, s.cell)
    Ek, nek = kernel_model.energy(build_device_model(cfg, w), s.positions, sp, i, j, S.astype(float), s.cell)
    # the engine's tensors are float32 (folded in float64, then rounded): ~1e-8 relative
    assert abs(Ek - E) < 1e-6 * max(1.0, abs(E)), (Ek, E)
    np.testing.assert_allclose(nek, ne, rtol=0, atol=1e-6 * max(1.0, np.abs(ne).max()))


@pytest.mark.parametrize("arch,C,width", [("small", 96, 128), ("medium", 96, 128), ("large", 64, 128),
                                          ("small", 192, 192), ("large", 192, 192), ("medium", 160, 192),
                                          ("small", 224, 256), ("medium", 256, 256)])
def test_model_padded_to_engine_width_in_the_fold(si64, arch, C, width):
    """A model runs on the narrowest compiled engine width that holds its channels (128, 192 or
    256): MACE-OFF small (96x0e) as its zero-padded 128-channel equivalent, MACE-OFF large
    (192x0e + 192x1o + 192x2e) natively at 192, 160 and 224 channels padded to 192 and 256.
    The kernel formulation of the folded tensors matches the oracle evaluating the original
    model."""
    s, i, j, S = si64
    cfg = arch_config(arch, zbl=True)
    cfg.hidden_irreps = "+".join(f"{C}x{b.ir}" for b in cfg.hidden)
    w = random_init(cfg, 4)
    dm = build_device_model(cfg, w)
    assert dm.dims["num_channels"] == width
    sp = np.zeros(len(s), int)
    Eo, neo = OracleMACE(cfg=cfg, weights=w).energy(s.positions, sp, np.stack([i, j]), S, s.cell)
    Ek, nek = kernel_model.energy(dm, s.positions, sp, i, j, S.astype(float), s.cell)
    np.testing.assert_allclose(nek, neo, atol=5e-6)
    assert abs(Ek - Eo) < 1e-6 * max(1.0, abs(Eo)) * len(s)


def test_wider_than_every_engine_raises():
    wide = arch_config("small")
    wide.hidden_irreps = "320x0e"
    with pytest.raises(UnsupportedModel):
        build_device_model(wide, random_init(wide, 0))
