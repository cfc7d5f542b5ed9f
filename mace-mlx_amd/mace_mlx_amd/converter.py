"""Weight-layout rules from an e3nn / mace-torch state dict to the reference's layout.

The reference converts a mace-torch checkpoint with torch and mace-torch installed
(`converter.py:125-158`); neither exists here, so this module restates only the
*layout rules* (`converter.py:369-506,578-646,660-675,764-794,797-824,887-929`) as
numpy transforms on a state dict that has already been read into arrays (for
example an ``.npz`` written by ``torch.save``-free tooling elsewhere).  The module
metadata the reference reads off the torch modules (instruction lists, path shapes,
FullyConnectedNet variances) is derived here from the model configuration with
e3nn's conventions:

* ``o3.Linear(irreps_in, irreps_out)`` holds one flat weight; its instructions run
  over input blocks (outer) and output blocks (inner) with equal irreps, each a
  row-major ``(mul_in, mul_out)`` slice, concatenated in instruction order.
* ``o3.FullyConnectedTensorProduct`` likewise, with ``(mul_1, mul_2, mul_out)``
  slices over (block 1, block 2, output block) with an allowed coupling.
* ``nn.FullyConnectedNet`` layer k computes ``act(x @ (W / sqrt(h_in var_in))) *
  sqrt(var_out)`` (hidden layers) or ``x @ (W / sqrt(h_in var_in / var_out))`` (last
  layer), with ``act`` = SiLU scaled to unit second moment; W is ``(h_in, h_out)``.
* mace-torch hands the interaction's message linear the *simplified* irreps of the
  conv-TP output, while the reference keeps them unsimplified (sorted); its linear
  then has more instructions, and each one takes a row block of the merged weight.

Parity unpinned against a real checkpoint (none can be loaded here); the tests pin
every rule by functional equivalence instead (the converted module computes the
same map as the e3nn one on random inputs).
"""

from __future__ import annotations

import math
from typing import Dict, Iterable, List, Mapping, Sequence, Tuple

import numpy as np

from .irreps import Irreps
from .model_io import (SILU_NORM_FACTOR, ModelConfig, conv_tp_instructions, fctp_instructions,
                       linear_instructions)


def e3nn_linear_instructions(irreps_in: Irreps, irreps_out: Irreps) -> List[Tuple[int, int, int, int]]:
    """(i_in, i_out, mul_in, mul_out) of ``o3.Linear``'s default instructions, in the
    order its flat weight stores them."""
    return [(i, o, bi.mul, bo.mul)
            for i, bi in enumerate(irreps_in)
            for o, bo in enumerate(irreps_out) if bi.ir == bo.ir]


def _block_map(ref: Irreps, src: Irreps) -> Dict[int, Tuple[int, int]]:
    """For every block of ``ref``, the block of ``src`` holding its channels and the
    channel offset inside it (`converter.py:432-474`).  Equal block counts map one to
    one; otherwise a block maps into the first ``src`` block of its irrep, after the
    channels of the earlier ``ref`` blocks of that irrep."""
    if len(ref) == len(src):
        return {i: (i, 0) for i in range(len(ref))}
    out, seen = {}, {}
    for i, b in enumerate(ref):
        key = (b.ir.l, b.ir.p)
        first = next((k for k, s in enumerate(src) if (s.ir.l, s.ir.p) == key), None)
        if first is not None:
            out[i] = (first, seen.get(key, 0))
        seen[key] = seen.get(key, 0) + b.mul
    return out


def split_e3nn_linear(flat: np.ndarray, torch_in: Irreps, torch_out: Irreps,
                      ref_in: Irreps | None = None, ref_out: Irreps | None = None) -> List[np.ndarray]:
    """Per-instruction weights of the reference's EquivariantLinear(ref_in, ref_out)
    from the flat weight of e3nn's Linear(torch_in, torch_out) (`converter.py:369-506`).

    With the same instruction count the slices are taken in order.  Otherwise each
    reference instruction takes the (row, column) block of the e3nn path weight its
    input and output blocks map to; paths e3nn does not have stay zero."""
    ref_in = torch_in if ref_in is None else ref_in
    ref_out = torch_out if ref_out is None else ref_out
    flat = np.asarray(flat).reshape(-1)
    tins = e3nn_linear_instructions(torch_in, torch_out)
    need = sum(mi * mo for _, _, mi, mo in tins)
    if flat.size != need:
        raise ValueError(f"e3nn Linear {torch_in} -> {torch_out}: {flat.size} weights, expected {need}")
    paths, off = {}, 0
    for i, o, mi, mo in tins:
        paths[(i, o)] = flat[off:off + mi * mo].reshape(mi, mo)
        off += mi * mo
    rins = linear_instructions(ref_in, ref_out)
    if len(rins) == len(tins):
        return [paths[(i, o)].copy() for i, o, _, _ in tins]
    rows, cols = _block_map(ref_in, torch_in), _block_map(ref_out, torch_out)
    out = []
    for ji, jo, mi, mo, _ in rins:
        if ji not in rows or jo not in cols or (rows[ji][0], cols[jo][0]) not in paths:
            out.append(np.zeros((mi, mo), dtype=flat.dtype))
            continue
        (ti, r0), (to, c0) = rows[ji], cols[jo]
        out.append(paths[(ti, to)][r0:r0 + mi, c0:c0 + mo].copy())
    return out


def split_e3nn_fctp(flat: np.ndarray, irreps1: Irreps, irreps2: Irreps, irreps_out: Irreps) -> List[np.ndarray]:
    """Per-instruction ``(mul_1, mul_2, mul_out)`` weights of a FullyConnectedTensorProduct
    from e3nn's flat weight (`converter.py:797-824`)."""
    flat = np.asarray(flat).reshape(-1)
    out, off = [], 0
    for i, j, k, _ in fctp_instructions(irreps1, irreps2, irreps_out):
        shp = (irreps1[i].mul, irreps2[j].mul, irreps_out[k].mul)
        n = shp[0] * shp[1] * shp[2]
        out.append(flat[off:off + n].reshape(shp).copy())
        off += n
    if off != flat.size:
        raise ValueError(f"FCTP flat weight has {flat.size} entries, instructions need {off}")
    return out


def bake_fcn(weights: Sequence[np.ndarray], var_in: Sequence[float] | None = None,
             var_out: Sequence[float] | None = None) -> List[np.ndarray]:
    """``nn.Linear`` weights ``(h_out, h_in)`` of the plain Linear -> SiLU -> ... -> Linear
    chain computing the same map as e3nn's FullyConnectedNet with layer weights
    ``(h_in, h_out)`` (`converter.py:578-646`).  Every layer but the last has the
    normalised SiLU; its scale ``SILU_NORM_FACTOR sqrt(var_out)`` is folded into the
    next layer's weight."""
    n = len(weights)
    var_in = [1.0] * n if var_in is None else list(var_in)
    var_out = [1.0] * n if var_out is None else list(var_out)
    out = []
    for k, w in enumerate(weights):
        w = np.asarray(w, dtype=np.float64)
        h_in = w.shape[0]
        last = k == n - 1
        eff = w / math.sqrt(h_in * var_in[k] / (var_out[k] if last else 1.0))
        if k > 0:  # the previous layer's activation was act(.) * sqrt(var_out)
            eff = eff * (SILU_NORM_FACTOR * math.sqrt(var_out[k - 1]))
        out.append(eff.T.copy())
    return out


def density_fn_weight(w: np.ndarray, var_in: float = 1.0, var_out: float = 1.0) -> np.ndarray:
    """``density_fn.weight`` ``(1, num_radial)`` of a density block from e3nn's one-layer
    FullyConnectedNet ``(num_radial, 1)`` without activation (`converter.py:660-675`)."""
    w = np.asarray(w, dtype=np.float64)
    return (w / math.sqrt(w.shape[0] * var_in / var_out)).T.copy()


def readout_linear_2(weights: Iterable[np.ndarray]) -> List[np.ndarray]:
    """The non-linear readout's ``linear_2`` weights with e3nn's unit-second-moment SiLU
    folded in (the reference's gate is plain SiLU; `converter.py:887-929`)."""
    return [np.asarray(w, dtype=np.float64) * SILU_NORM_FACTOR for w in weights]


def radial_mlp_layernorm(sd: Mapping[str, np.ndarray], torch_prefix: str, ref_prefix: str) -> Dict[str, np.ndarray]:
    """mace-torch ``RadialMLP`` (``net.{k}`` Linear / LayerNorm / SiLU) -> the reference's
    ``layers.{k}``: the same parameters under new names (`converter.py:764-794`)."""
    out = {}
    pre = torch_prefix + ".net."
    for key, v in sd.items():
        if key.startswith(pre):
            idx, _, name = key[len(pre):].partition(".")
            if idx.isdigit() and name in ("weight", "bias"):
                out[f"{ref_prefix}.layers.{idx}.{name}"] = np.asarray(v)
    return out


def convert_state_dict(sd: Mapping[str, np.ndarray], cfg: ModelConfig) -> Dict[str, np.ndarray]:
    """A mace-torch ``MACE`` / ``ScaleShiftMACE`` state dict (as numpy arrays) in the
    reference's weight layout for ``cfg`` (`converter.py:315-366`).

    mace-torch key names: ``interactions.{i}.linear_up.weight``,
    ``interactions.{i}.conv_tp_weights.layer{k}.weight``, ``interactions.{i}.linear.weight``,
    ``interactions.{i}.skip_tp.weight``, ``interactions.{i}.density_fn.layer0.weight``,
    ``products.{i}.symmetric_contractions.contractions.{c}.weights_max`` /
    ``.weights.{k}``, ``products.{i}.linear.weight``, ``readouts.{i}.linear.weight`` or
    ``.linear_1.weight`` / ``.linear_2.weight``, ``node_embedding.linear.weight``,
    ``atomic_energies_fn.atomic_energies``, ``radial_embedding.bessel_fn.bessel_weights``."""
    cfg.check_supported()
    res: Dict[str, np.ndarray] = {}
    nel, H = cfg.num_elements, cfg.num_heads
    attrs = Irreps(f"{nel}x0e")
    scal = Irreps([b for b in cfg.hidden if b.ir.l == 0])
    inter = cfg.interaction_irreps

    def lin(torch_key, ref_key, t_in, t_out, r_in=None, r_out=None):
        for n, w in enumerate(split_e3nn_linear(sd[torch_key], t_in, t_out, r_in, r_out)):
            res[f"{ref_key}.weights.{n}"] = w

    res["atomic_energies_fn.atomic_energies"] = np.asarray(sd["atomic_energies_fn.atomic_energies"])
    lin("node_embedding.linear.weight", "node_embedding.linear", attrs, scal)
    res["radial_embedding.bessel_fn.bessel_weights"] = np.asarray(sd["radial_embedding.bessel_fn.bessel_weights"])
    edges = cfg.edge_irreps_per_layer()
    for li, (irr_in, hid) in enumerate(zip(cfg.layer_inputs(), cfg.hidden_per_layer())):
        p = f"interactions.{li}"
        if cfg.nonlinear:  # converter.py:679-762
            nsc = Irreps(f"{irr_in.count('0e')}x0e")
            edge, nonlin = edges[li], cfg.nonlin_irreps()
            mid, _ = conv_tp_instructions(edge, cfg.sh_irreps, inter)
            lin(f"{p}.source_embedding.weight", f"{p}.source_embedding", attrs, nsc)
            lin(f"{p}.target_embedding.weight", f"{p}.target_embedding", attrs, nsc)
            lin(f"{p}.skip_tp.weight", f"{p}.skip_tp", irr_in, hid)
            lin(f"{p}.linear_up.weight", f"{p}.linear_up", irr_in, edge)
            res.update(radial_mlp_layernorm(sd, f"{p}.conv_tp_weights", f"{p}.conv_tp_weights"))
            res.update(radial_mlp_layernorm(sd, f"{p}.density_fn", f"{p}.density_fn"))
            res[f"{p}.alpha"] = np.asarray(sd[f"{p}.alpha"])
            res[f"{p}.beta"] = np.asarray(sd[f"{p}.beta"])
            # e3nn's Gate concatenates its input irreps (scalars + gates + gated) unsimplified, as
            # the reference does; the message enters linear_1 simplified, as in the other blocks
            lin(f"{p}.linear_res.weight", f"{p}.linear_res", edge, nonlin)
            lin(f"{p}.linear_1.weight", f"{p}.linear_1", mid.simplify(), nonlin, mid, nonlin)
            lin(f"{p}.linear_2.weight", f"{p}.linear_2", inter, inter)
            _convert_product_readout(sd, cfg, li, hid, res, lin)
            continue
        lin(f"{p}.linear_up.weight", f"{p}.linear_up", irr_in, irr_in)
        k, ws = 0, []
        while f"{p}.conv_tp_weights.layer{k}.weight" in sd:
            ws.append(sd[f"{p}.conv_tp_weights.layer{k}.weight"])
            k += 1
        for n, w in enumerate(bake_fcn(ws)):
            res[f"{p}.conv_tp_weights.layers.{2 * n}.weight"] = w
        mid, _ = conv_tp_instructions(irr_in, cfg.sh_irreps, inter)
        lin(f"{p}.linear.weight", f"{p}.linear", mid.simplify(), inter, mid, inter)
        s_in, s_out = (irr_in, hid) if cfg.residual(li) else (inter, inter)
        for n, w in enumerate(split_e3nn_fctp(sd[f"{p}.skip_tp.weight"], s_in, attrs, s_out)):
            res[f"{p}.skip_tp.tp.weights.{n}"] = w
        if cfg.use_density_normalization:
            res[f"{p}.density_fn.weight"] = density_fn_weight(sd[f"{p}.density_fn.layer0.weight"])
        _convert_product_readout(sd, cfg, li, hid, res, lin)
    return {k: np.asarray(v, dtype=np.float32) for k, v in res.items()}


def _convert_product_readout(sd, cfg: ModelConfig, li: int, hid: Irreps, res: dict, lin) -> None:
    """Symmetric-contraction weights (same layout), product linear, readouts with the SiLU
    constant folded into the non-linear readout's linear_2 (`converter.py:836-929`)."""
    H = cfg.num_heads
    q = f"products.{li}"
    for key, v in sd.items():
        if key.startswith(f"{q}.symmetric_contractions."):
            res[key] = np.asarray(v)
    lin(f"{q}.linear.weight", f"{q}.linear", hid, hid)
    r = f"readouts.{li}"
    out = Irreps(f"{H}x0e")
    if li < cfg.num_interactions - 1:
        lin(f"{r}.linear.weight", f"{r}.linear", hid, out)
    else:
        mlp = Irreps(f"{16 * H}x0e")
        lin(f"{r}.linear_1.weight", f"{r}.linear_1", hid, mlp)
        for n, w in enumerate(readout_linear_2(split_e3nn_linear(sd[f"{r}.linear_2.weight"], mlp, out))):
            res[f"{r}.linear_2.weights.{n}"] = w


def convert_npz(state_npz: str, config: dict | ModelConfig, out_dir: str):
    """Write ``config.json`` + ``weights.npz`` (the reference's model directory, loadable by
    ``MACECalculator(model_path=out_dir)``) from a mace-torch state dict saved as an
    ``.npz`` of arrays under mace-torch key names, and the model's configuration."""
    from .model_io import save_model

    cfg = config if isinstance(config, ModelConfig) else ModelConfig.from_dict(config)
    with np.load(state_npz, allow_pickle=False) as z:
        sd = {k: np.asarray(z[k]) for k in z.files}
    return save_model(out_dir, cfg, convert_state_dict(sd, cfg))
