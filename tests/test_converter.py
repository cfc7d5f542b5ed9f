"""The converter's weight-layout rules (mace_mlx_amd/converter.py, reference
`converter.py:369-506,578-646,660-675,797-824,887-929`), pinned by what they are for:
the converted module computes the same map as the e3nn module it comes from.

No mace-torch checkpoint can be read here, so the e3nn side is written from e3nn's
documented forward formulas (o3.Linear path normalisation, FullyConnectedNet layers
with the unit-second-moment SiLU, whose constant is recomputed here the way e3nn computes
it rather than taken from the product).  Parity against a real checkpoint stays unpinned."""

import math

import numpy as np
import pytest
import torch
from scipy import integrate

from mace_mlx_amd import converter as cv
from mace_mlx_amd.irreps import Irreps
from mace_mlx_amd.model_io import SILU_NORM_FACTOR, ModelConfig, conv_tp_instructions, linear_instructions, random_init
from oracle.model import Linear


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _silu_second_moment():
    f = lambda z: _silu(z) ** 2 * math.exp(-z * z / 2) / math.sqrt(2 * math.pi)
    return integrate.quad(f, -40, 40, epsabs=1e-13, epsrel=1e-13)[0]


def _normalize2mom(f):
    """e3nn's normalize2mom constant: E[f(z)^2]^(-1/2) estimated on 10^6 float64 normals
    drawn from torch's CPU generator seeded with 0 (a sample, not the integral)."""
    g = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=g, dtype=torch.float64)
    return f(z).pow(2).mean().pow(-0.5).item()


def test_silu_norm_factor_is_unit_second_moment():
    # e3nn normalize2mom(silu): silu scaled so that E[act(z)^2] = 1 for z ~ N(0, 1); the
    # reference keeps its float32 value (`utils.py:17`)
    assert abs(SILU_NORM_FACTOR - _normalize2mom(torch.nn.functional.silu)) < 2e-7
    # and it is the sampled estimate of the exact second moment (within the sample's 0.2 %)
    assert abs(SILU_NORM_FACTOR * math.sqrt(_silu_second_moment()) - 1.0) < 2e-3


def _pack_linear(weights, torch_in, torch_out):
    return np.concatenate([w.reshape(-1) for w in weights])


def test_e3nn_linear_order_and_roundtrip():
    t_in, t_out = Irreps("16x0e+8x1o+4x0e+2x2e"), Irreps("6x0e+3x1o+5x2e")
    ins = cv.e3nn_linear_instructions(t_in, t_out)
    # input blocks outer, output blocks inner (o3.Linear default instructions)
    assert [(i, o) for i, o, _, _ in ins] == [(0, 0), (1, 1), (2, 0), (3, 2)]
    rng = np.random.default_rng(0)
    ws = [rng.standard_normal((mi, mo)) for _, _, mi, mo in ins]
    got = cv.split_e3nn_linear(_pack_linear(ws, t_in, t_out), t_in, t_out)
    assert len(got) == len(ws) and all(np.array_equal(a, b) for a, b in zip(got, ws))
    with pytest.raises(ValueError):
        cv.split_e3nn_linear(np.zeros(3), t_in, t_out)


@pytest.mark.parametrize("lin_irreps", ["32x0e+32x1o", "32x0e+32x1o+32x2e"])
def test_message_linear_split_is_the_same_map(lin_irreps):
    """mace-torch feeds the message linear the simplified conv-TP irreps; the reference keeps
    them unsimplified (`converter.py:407-506`).  The split weights must give the same linear
    map (including the 1/sqrt(fan-in) path weights) on the same flat feature vector."""
    irr_in = Irreps(lin_irreps)
    sh = Irreps.spherical_harmonics(3)
    target = Irreps([(32, b.ir) for b in sh])
    mid, _ = conv_tp_instructions(irr_in, sh, target)
    simp = mid.simplify()
    assert len(simp) < len(mid) and simp.dim == mid.dim
    rng = np.random.default_rng(1)
    tw = [torch.from_numpy(rng.standard_normal((mi, mo))) for _, _, mi, mo in cv.e3nn_linear_instructions(simp, target)]
    flat = np.concatenate([w.numpy().reshape(-1) for w in tw])
    ref_w = [torch.from_numpy(w) for w in cv.split_e3nn_linear(flat, simp, target, mid, target)]
    assert len(ref_w) == len(linear_instructions(mid, target))
    x = torch.from_numpy(rng.standard_normal((5, mid.dim)))
    y_e3nn = Linear(simp, target, tw)(x)
    y_ref = Linear(mid, target, ref_w)(x)
    assert torch.allclose(y_e3nn, y_ref, rtol=1e-12, atol=1e-12)


def test_gate_input_split_columns():
    """Output split (`converter.py:432-453`): an e3nn Linear into the simplified gate input
    '96x0e+...' equals the reference's unsimplified '32x0e+64x0e+...' one."""
    t_in, r_out = Irreps("32x0e+32x1o"), Irreps("32x0e+64x0e+32x1o")
    t_out = r_out.simplify()
    rng = np.random.default_rng(2)
    tw = [torch.from_numpy(rng.standard_normal((mi, mo))) for _, _, mi, mo in cv.e3nn_linear_instructions(t_in, t_out)]
    flat = np.concatenate([w.numpy().reshape(-1) for w in tw])
    rw = [torch.from_numpy(w) for w in cv.split_e3nn_linear(flat, t_in, t_out, t_in, r_out)]
    x = torch.from_numpy(rng.standard_normal((4, t_in.dim)))
    # the reference's path weight is 1/sqrt(fan-in) per output block: unchanged by the split
    assert torch.allclose(Linear(t_in, t_out, tw)(x), Linear(t_in, r_out, rw)(x), rtol=1e-12, atol=1e-12)


def _e3nn_fcn(x, ws, var_in, var_out, c):
    """e3nn FullyConnectedNet: act(x @ W / sqrt(h_in var_in)) sqrt(var_out) per hidden layer,
    x @ W / sqrt(h_in var_in / var_out) for the last; act = c silu."""
    n = len(ws)
    for k, w in enumerate(ws):
        h_in = w.shape[0]
        if k < n - 1:
            x = c * _silu(x @ (w / math.sqrt(h_in * var_in[k]))) * math.sqrt(var_out[k])
        else:
            x = x @ (w / math.sqrt(h_in * var_in[k] / var_out[k]))
    return x


@pytest.mark.parametrize("variances", [None, ([1.0, 1.0, 1.0, 1.0], [1.0, 1.0, 1.0, 1.0]),
                                       ([1.3, 0.7, 1.1, 0.9], [0.8, 1.2, 0.6, 1.4])])
def test_fcn_baking_is_the_same_map(variances):
    rng = np.random.default_rng(3)
    dims = [8, 64, 64, 64, 40]
    ws = [rng.standard_normal((a, b)) for a, b in zip(dims, dims[1:])]
    vi, vo = variances if variances else ([1.0] * 4, [1.0] * 4)
    baked = cv.bake_fcn(ws, *(variances or (None, None)))
    assert [w.shape for w in baked] == [(b, a) for a, b in zip(dims, dims[1:])]
    x = rng.standard_normal((7, 8))
    c = _normalize2mom(torch.nn.functional.silu)
    want = _e3nn_fcn(x, ws, vi, vo, c)
    y = x
    for k, w in enumerate(baked):  # the reference's chain: Linear (x @ W.T), plain SiLU between
        y = y @ w.T
        if k < len(baked) - 1:
            y = _silu(y)
    # the product's constant is the float32 value of e3nn's (5e-9 relative apart)
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-9)


def test_density_fn_weight():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((8, 1))
    x = rng.standard_normal((6, 8))
    got = x @ cv.density_fn_weight(w).T
    np.testing.assert_allclose(got, _e3nn_fcn(x, [w], [1.0], [1.0], 1.0), rtol=1e-12)


def test_readout_silu_factor():
    """e3nn's non-linear readout uses the unit-second-moment SiLU; the reference's plain SiLU
    with linear_2 scaled by the constant gives the same energy (`converter.py:909-929`)."""
    rng = np.random.default_rng(5)
    w1, w2 = rng.standard_normal((32, 16)), rng.standard_normal((16, 1))
    x = rng.standard_normal((9, 32))
    c = _normalize2mom(torch.nn.functional.silu)
    h = x @ w1 / math.sqrt(32)
    e3nn = (c * _silu(h)) @ w2 / math.sqrt(16)
    ref = _silu(h) @ cv.readout_linear_2([w2])[0] / math.sqrt(16)
    np.testing.assert_allclose(ref, e3nn, rtol=1e-7)


def test_fctp_split_order():
    i1, i2, io = Irreps("4x0e+2x1o"), Irreps("3x0e"), Irreps("5x0e+6x1o")
    rng = np.random.default_rng(6)
    shapes = [(4, 3, 5), (2, 3, 6)]  # (0e x 0e -> 0e), (1o x 0e -> 1o)
    ws = [rng.standard_normal(s) for s in shapes]
    got = cv.split_e3nn_fctp(np.concatenate([w.reshape(-1) for w in ws]), i1, i2, io)
    assert [g.shape for g in got] == shapes and all(np.array_equal(a, b) for a, b in zip(got, ws))


def _to_mace_torch(cfg: ModelConfig, w: dict) -> dict:
    """A mace-torch state dict holding the same model as the reference-layout weights `w`:
    e3nn flat weights (the message linear over the simplified irreps), FullyConnectedNet
    layers with the normalisation taken back out, linear_2 without the SiLU constant."""
    sd = {}
    attrs = Irreps(f"{cfg.num_elements}x0e")
    scal = Irreps([b for b in cfg.hidden if b.ir.l == 0])
    inter = cfg.interaction_irreps

    def flat(prefix, n):
        return np.concatenate([np.asarray(w[f"{prefix}.weights.{k}"], np.float64).reshape(-1) for k in range(n)])

    def cnt(prefix):
        return sum(1 for k in w if k.startswith(prefix + ".weights."))

    sd["atomic_energies_fn.atomic_energies"] = w["atomic_energies_fn.atomic_energies"]
    sd["radial_embedding.bessel_fn.bessel_weights"] = w["radial_embedding.bessel_fn.bessel_weights"]
    sd["node_embedding.linear.weight"] = flat("node_embedding.linear", cnt("node_embedding.linear"))

    def merged_linear(prefix, r_in, r_out, t_in):
        """e3nn flat weight over the simplified input irreps t_in from the reference's
        per-instruction weights over the unsimplified r_in"""
        paths = {}
        for (ji, jo, mi, mo, _), k in zip(linear_instructions(r_in, r_out), range(10 ** 6)):
            paths.setdefault((r_in[ji].ir, jo), []).append(np.asarray(w[f"{prefix}.weights.{k}"], np.float64))
        return np.concatenate([np.concatenate(paths[(t_in[i].ir, o)], axis=0).reshape(-1)
                               for i, o, _, _ in cv.e3nn_linear_instructions(t_in, r_out)])

    for li, (irr_in, hid) in enumerate(zip(cfg.layer_inputs(), cfg.hidden_per_layer())):
        p = f"interactions.{li}"
        if cfg.nonlinear:
            for name in ("source_embedding", "target_embedding", "skip_tp", "linear_up", "linear_res", "linear_2"):
                sd[f"{p}.{name}.weight"] = flat(f"{p}.{name}", cnt(f"{p}.{name}"))
            for name in ("conv_tp_weights", "density_fn"):
                for k, v in w.items():
                    if k.startswith(f"{p}.{name}.layers."):
                        sd[k.replace(".layers.", ".net.")] = v
            sd[f"{p}.alpha"], sd[f"{p}.beta"] = w[f"{p}.alpha"], w[f"{p}.beta"]
            edge = cfg.edge_irreps_per_layer()[li]
            mid, _ = conv_tp_instructions(edge, cfg.sh_irreps, cfg.interaction_irreps)
            sd[f"{p}.linear_1.weight"] = merged_linear(f"{p}.linear_1", mid, cfg.nonlin_irreps(), mid.simplify())
        if cfg.nonlinear:
            q = f"products.{li}"
            for k, v in w.items():
                if k.startswith(f"{q}.symmetric_contractions."):
                    sd[k] = v
            sd[f"{q}.linear.weight"] = flat(f"{q}.linear", cnt(f"{q}.linear"))
            r = f"readouts.{li}"
            if li < cfg.num_interactions - 1:
                sd[f"{r}.linear.weight"] = flat(f"{r}.linear", cnt(f"{r}.linear"))
            else:
                sd[f"{r}.linear_1.weight"] = flat(f"{r}.linear_1", cnt(f"{r}.linear_1"))
                sd[f"{r}.linear_2.weight"] = flat(f"{r}.linear_2", cnt(f"{r}.linear_2")) / SILU_NORM_FACTOR
            continue
        sd[f"{p}.linear_up.weight"] = flat(f"{p}.linear_up", cnt(f"{p}.linear_up"))
        ks = sorted(int(k.split(".layers.")[1].split(".")[0]) for k in w if k.startswith(f"{p}.conv_tp_weights."))
        n = len(ks)
        for j, k in enumerate(ks):
            m = np.asarray(w[f"{p}.conv_tp_weights.layers.{k}.weight"], np.float64).T  # (h_in, h_out)
            m = m * math.sqrt(m.shape[0])
            if j > 0:
                m = m / SILU_NORM_FACTOR
            sd[f"{p}.conv_tp_weights.layer{j}.weight"] = m
        mid, _ = conv_tp_instructions(irr_in, cfg.sh_irreps, inter)
        simp = mid.simplify()
        paths = {}
        for (ji, jo, mi, mo, _), k in zip(linear_instructions(mid, inter), range(10 ** 6)):
            paths.setdefault((mid[ji].ir, jo), []).append(np.asarray(w[f"{p}.linear.weights.{k}"], np.float64))
        sd[f"{p}.linear.weight"] = np.concatenate(
            [np.concatenate(paths[(simp[i].ir, o)], axis=0).reshape(-1) for i, o, _, _ in cv.e3nn_linear_instructions(simp, inter)])
        sd[f"{p}.skip_tp.weight"] = flat(f"{p}.skip_tp.tp", cnt(f"{p}.skip_tp.tp"))
        if cfg.use_density_normalization:
            d = np.asarray(w[f"{p}.density_fn.weight"], np.float64).T
            sd[f"{p}.density_fn.layer0.weight"] = d * math.sqrt(d.shape[0])
        q = f"products.{li}"
        for k, v in w.items():
            if k.startswith(f"{q}.symmetric_contractions."):
                sd[k] = v
        sd[f"{q}.linear.weight"] = flat(f"{q}.linear", cnt(f"{q}.linear"))
        r = f"readouts.{li}"
        if li < cfg.num_interactions - 1:
            sd[f"{r}.linear.weight"] = flat(f"{r}.linear", cnt(f"{r}.linear"))
        else:
            sd[f"{r}.linear_1.weight"] = flat(f"{r}.linear_1", cnt(f"{r}.linear_1"))
            sd[f"{r}.linear_2.weight"] = flat(f"{r}.linear_2", cnt(f"{r}.linear_2")) / SILU_NORM_FACTOR
    return sd


@pytest.mark.parametrize("kind", ["medium", "mpa0_like", "mh1"])
def test_convert_state_dict_roundtrip(kind):
    from mace_mlx_amd.systems import arch_config
    cfg = arch_config("medium", zbl=True)
    if kind == "mpa0_like":
        cfg.first_interaction_nonresidual = True
        cfg.use_density_normalization = True
    if kind == "mh1":
        from test_oracle_mh1 import mh1_config
        cfg = mh1_config()
    w = random_init(cfg, seed=11)
    got = cv.convert_state_dict(_to_mace_torch(cfg, w), cfg)
    assert set(got) == set(w)
    for k in w:
        np.testing.assert_allclose(got[k], w[k], rtol=2e-6, atol=1e-6, err_msg=k)


def test_convert_npz_writes_a_loadable_model(tmp_path):
    from mace_mlx_amd.model_io import load_config, load_weights
    from mace_mlx_amd.systems import arch_config
    cfg = arch_config("small")
    w = random_init(cfg, seed=3)
    np.savez(tmp_path / "sd.npz", **_to_mace_torch(cfg, w))
    out = cv.convert_npz(str(tmp_path / "sd.npz"), cfg.to_dict(), str(tmp_path / "model"))
    assert load_config(out).to_dict() == cfg.to_dict()
    got = load_weights(out)
    assert set(got) == set(w) and all(np.allclose(got[k], w[k], rtol=2e-6, atol=1e-6) for k in w)
