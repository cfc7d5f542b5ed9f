"""Reference-layout model -> named tensors for the HIP engine.

Reads a model in the reference's format (`model.py:664-720`: config.json +
weights.npz, key names of `converter.py`) and produces the dims struct and the
tensors `mace_model_set_tensor` expects.  All normalisation constants of the
reference (path weights, CG factors, 1/avg_num_neighbors, ScaleShift scale and
shift) are folded in here, once, in float64, and the per-block matrices are laid
out for the kernels' component-major node layout (element (u, m) of a block at
``m * C + u``).

Tensor names (C = channels, n_el = elements, per layer prefix ``L{l}.``):

  e0 [n_el]                       atomic energies (+ shift for ScaleShiftMACE)
  bessel_w [nb]                   Bessel frequencies
  zbl_z, zbl_cov [n_el]           atomic number and covalent radius per element
  embed [n_el][C]                 node embedding (one-hot linear, pw folded)
  L.up.b [C][C]                   linear_up, block l=b
  agnesi_cov [n_el]               covalent radius per element (Agnesi transform only)
  L.skip.b [n_el][C][C]           skip FCTP for hidden block b (CG * pw folded; residual blocks)
  L.mskip.l [n_el][C][C]          message skip FCTP, interaction block l (non-residual first block)
  L.dens [nb]                     density_fn weights (density-normalised blocks)
  L.mlp.k                         radial MLP layer k, [in][out]
  L.lin.l [nslots(l)*C][C]        message linear for output l (pw folded; / avg unless density)
  L.sc.b [n_el][K3+K2+K1][C]      symmetric-contraction weights, output block b
  L.plin.b [C][C]                 product linear
  L.ro [C] | L.ro1 [C][16], L.ro2 [16]   readouts (scale folded)
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from .cg import u_matrix, wigner_3j
from .irreps import Irrep, Irreps
from .model_io import (COVALENT_RADII, ModelConfig, conv_tp_instructions, linear_instructions, pad_channels,
                       select_head)

# channel multiplicities the HIP engine is compiled for (csrc/common.h NC, one library each);
# a model runs on the smallest one that holds its channels, zero-padded up to it
from ._ffi import ENGINE_WIDTHS  # noqa: E402


class UnsupportedModel(NotImplementedError):
    pass


def _blocks(irreps: Irreps, C: int) -> int:
    """Number of leading blocks 0e, 1o, 2e, ... (all multiplicity C)."""
    for b, blk in enumerate(irreps):
        if blk.mul != C or blk.ir != Irrep(b, (-1) ** b):
            raise UnsupportedModel(f"irreps {irreps}: blocks must be {C}x0e+{C}x1o+{C}x2e...")
    if len(irreps) > 3:
        raise UnsupportedModel(f"irreps {irreps}: at most l=2 hidden features are compiled in")
    return len(irreps)


@dataclass
class DeviceModel:
    dims: dict
    tensors: Dict[str, np.ndarray]
    z_table: List[int]
    r_max: float


# Arrays the reference keeps in float32 when the model runs in float16 or bfloat16
# (`model.py:642-661` _pin_float32): baseline energies and Bessel frequencies
# (covalent radii are tables, never model weights).
FP32_PINNED = ("atomic_energies_fn.atomic_energies", "radial_embedding.bessel_fn.bessel_weights")


def round_weights_fp16(w: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """The weights of a float16 model (`model.py:705-711`: set_dtype, then re-pin): every
    floating array rounded to fp16 except FP32_PINNED."""
    return {k: (np.asarray(v) if k in FP32_PINNED else
                np.asarray(v, dtype=np.float32).astype(np.float16).astype(np.float64))
            for k, v in w.items()}


def to_bf16(x) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 value (ties to even), returned as float64:
    the upper 16 bits of the float32 pattern after adding 0x7fff plus the lowest kept bit; a NaN
    becomes the quiet NaN of its upper bits (the addition could carry it into the sign or the
    exponent).  The device's round_bf16 is the same bit operation."""
    shape = np.shape(x)
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    u = np.where(nan, (u | 0x00400000) & 0xFFFF0000, (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000)
    return u.astype(np.uint32).view(np.float32).astype(np.float64).reshape(shape)


def round_weights_bf16(w: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """The weights of a bfloat16 model (`model.py:705-711`): every floating array rounded to
    bf16 except FP32_PINNED."""
    return {k: (np.asarray(v) if k in FP32_PINNED else to_bf16(v)) for k, v in w.items()}


def round_weights(w: Dict[str, np.ndarray], dtype: str) -> Dict[str, np.ndarray]:
    """The weights a model of dtype ("float32", "float16", "bfloat16") computes with."""
    return {"float16": round_weights_fp16, "bfloat16": round_weights_bf16}.get(dtype, dict)(w)


# mace_model_dims.feature_half per dtype (the rounding mode of the stored activations)
FEATURE_POLICY = {"float32": 0, "float16": 1, "bfloat16": 2}


def build_device_model(cfg: ModelConfig, w: Dict[str, np.ndarray], dtype: str = "float32",
                       head: Optional[str] = None) -> DeviceModel:
    """Fold a model (config + reference-layout weights) into the engine's tensors.  dtype
    "float16" / "bfloat16" select the reference's half-precision feature policies (`model.py:1-15,
    592-596, 705-711`); ``head`` the readout head of a multi-head model (default: the first, as
    `calculators.py:128-137`)."""
    if dtype not in FEATURE_POLICY:
        raise UnsupportedModel(f"dtype={dtype!r} (float32, float16 and bfloat16 are implemented)")
    w = round_weights(w, dtype)
    cfg.check_supported()
    cfg, w = select_head(cfg, w, head)
    if cfg.model_type not in ("MACE", "ScaleShiftMACE"):
        raise UnsupportedModel(f"model_type={cfg.model_type}")
    width = min((c for c in ENGINE_WIDTHS if c >= cfg.num_features), default=None)
    if width is None:
        raise UnsupportedModel(f"{cfg.num_features} channels (the engine is compiled for at most "
                               f"{max(ENGINE_WIDTHS)})")
    if cfg.num_features != width:
        # a width between the compiled ones (MACE-OFF small 96, large 192): the same model with
        # zero channels appended and the path weights compensated (model_io.pad_channels)
        try:
            cfg, w = pad_channels(cfg, w, width)
        except NotImplementedError as exc:
            raise UnsupportedModel(str(exc)) from exc
    C = cfg.num_features
    nel = cfg.num_elements
    if cfg.max_ell != 3:
        raise UnsupportedModel("max_ell must be 3")
    if list(cfg.radial_MLP) != [64, 64, 64]:
        raise UnsupportedModel(f"radial_MLP={cfg.radial_MLP}")
    scale = float(cfg.scale) if cfg.model_type == "ScaleShiftMACE" else 1.0
    shift = float(cfg.shift) if cfg.model_type == "ScaleShiftMACE" else 0.0
    z_table = list(cfg.z_table) if cfg.z_table else list(range(nel))
    T: Dict[str, np.ndarray] = {}
    f64 = lambda k: np.asarray(w[k], dtype=np.float64)

    T["e0"] = f64("atomic_energies_fn.atomic_energies").reshape(-1) + shift
    T["bessel_w"] = f64("radial_embedding.bessel_fn.bessel_weights").reshape(-1)
    T["zbl_z"] = np.asarray(z_table, dtype=np.float64)
    T["zbl_cov"] = COVALENT_RADII[np.asarray(z_table)]
    attrs = Irreps(f"{nel}x0e")
    scal = Irreps([b for b in cfg.hidden if b.ir.l == 0])
    (inst,) = linear_instructions(attrs, scal)
    T["embed"] = f64("node_embedding.linear.weights.0") * inst[4]

    ins, hids = cfg.layer_inputs(), cfg.hidden_per_layer()
    n_layers = cfg.num_interactions
    dims = dict(num_elements=nel, num_channels=C, max_ell=cfg.max_ell, num_bessel=cfg.num_bessel,
                num_poly_cutoff=cfg.num_polynomial_cutoff, num_layers=n_layers, radial_hidden=64,
                radial_depth=3, layer_in_blocks=[0] * 4, layer_hid_blocks=[0] * 4, correlation=[0] * 4,
                has_zbl=int(bool(cfg.pair_repulsion)), zbl_p=6, r_max=float(cfg.r_max),
                zbl_a_exp=0.3, zbl_a_prefactor=0.4543, zbl_scale=scale,
                feature_half=FEATURE_POLICY[dtype],
                density_norm=int(bool(cfg.use_density_normalization)),
                first_nonresidual=int(bool(cfg.first_interaction_nonresidual)),
                agnesi=int(cfg.agnesi() is not None), agnesi_q=0.0, agnesi_p=0.0, agnesi_a=0.0,
                nonlinear=int(cfg.nonlinear), separate_cutoff=int(not cfg.apply_cutoff),
                agnostic_product=int(bool(cfg.use_agnostic_product)), layer_edge_blocks=[0] * 4)
    ag = cfg.agnesi()
    if ag is not None:
        dims.update(agnesi_q=ag["q"], agnesi_p=ag["p"], agnesi_a=ag["a"])
        T["agnesi_cov"] = cfg.agnesi_radii()[np.asarray(z_table)]
    if cfg.pair_repulsion:
        dims["zbl_p"] = int(cfg.pair_repulsion.get("p", 6))
        dims["zbl_a_exp"] = float(cfg.pair_repulsion.get("a_exp", 0.3))
        dims["zbl_a_prefactor"] = float(cfg.pair_repulsion.get("a_prefactor", 0.4543))
    inter = cfg.interaction_irreps
    coupling = Irreps([(1, b.ir) for b in inter])
    edges = cfg.edge_irreps_per_layer()
    for l in range(n_layers):
        p = f"L{l}."
        q = f"interactions.{l}"
        irr_in, hid = ins[l], hids[l]
        lin, lhid = _blocks(irr_in, C), _blocks(hid, C)
        dims["layer_in_blocks"][l] = lin
        dims["layer_hid_blocks"][l] = lhid
        dims["correlation"][l] = int(cfg.correlation[l])
        if cfg.nonlinear:
            dims["layer_edge_blocks"][l] = _blocks(edges[l], C)
            _fold_nonlinear(cfg, w, l, irr_in, hid, edges[l], T)
            _fold_product_readout(cfg, w, l, hid, T, scale, coupling)
            continue
        # linear_up
        for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(irr_in, irr_in)):
            assert ji == jo
            T[f"{p}up.{ji}"] = f64(f"{q}.linear_up.weights.{n}") * pw
        # skip FCTP with one-hot attributes: out[w,k] = pw * sum_u W[u,z,w] x[u,i] cg[i,0,k];
        # residual blocks: input -> hidden ("skip"); non-residual first block: message ->
        # message ("mskip", blocks.py:68-176)
        from .model_io import fctp_instructions
        resid = cfg.residual(l)
        s_in, s_out, s_name = (irr_in, hid, "skip") if resid else (inter, inter, "mskip")
        for n, (i1, i2, io, pw) in enumerate(fctp_instructions(s_in, attrs, s_out)):
            l1, lo = s_in[i1].ir.l, s_out[io].ir.l
            cg = wigner_3j(l1, 0, lo)[:, 0, :]
            c = cg[0, 0]
            if l1 != lo or not np.allclose(cg, c * np.eye(2 * l1 + 1), atol=1e-12):
                raise UnsupportedModel("skip connection with non-diagonal coupling")
            W = f64(f"{q}.skip_tp.tp.weights.{n}")          # (C, n_el, C)
            T[f"{p}{s_name}.{io}"] = np.transpose(W, (1, 0, 2)) * (pw * c)
        if cfg.use_density_normalization:
            T[f"{p}dens"] = f64(f"{q}.density_fn.weight").reshape(-1)
        # radial MLP, nn.Linear (out, in) -> [in][out]
        for k in range(4):
            T[f"{p}mlp.{k}"] = f64(f"{q}.conv_tp_weights.layers.{2 * k}.weight").T
        # message linear (irreps_mid -> interaction irreps) / avg_num_neighbors
        mid, _ = conv_tp_instructions(irr_in, cfg.sh_irreps, inter)
        per_out = {}
        norm = 1.0 if cfg.use_density_normalization else 1.0 / cfg.avg_num_neighbors
        for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(mid, inter)):
            per_out.setdefault(jo, []).append(f64(f"{q}.linear.weights.{n}") * pw * norm)
        for jo in range(len(inter)):
            T[f"{p}lin.{jo}"] = np.concatenate(per_out[jo], axis=0)
        _fold_product_readout(cfg, w, l, hid, T, scale, coupling)
    return DeviceModel(dims=dims, tensors={k: np.ascontiguousarray(v, dtype=np.float32) for k, v in T.items()},
                       z_table=z_table, r_max=float(cfg.r_max))


def _fold_product_readout(cfg: ModelConfig, w, l: int, hid: Irreps, T: Dict[str, np.ndarray], scale: float,
                          coupling: Irreps) -> None:
    """Symmetric contraction (one weight set when the product is element-agnostic), product
    linear and readout of layer l."""
    p = f"L{l}."
    f64 = lambda k: np.asarray(w[k], dtype=np.float64)
    r = f"products.{l}.symmetric_contractions.contractions"
    corr = int(cfg.correlation[l])
    for b, blk in enumerate(hid):
        parts = []
        keys = [f"{r}.{b}.weights_max"] + [f"{r}.{b}.weights.{i}" for i in range(corr - 1)]
        for key, nu in zip(keys, range(corr, 0, -1)):
            Wn = f64(key)
            if not np.any(np.abs(u_matrix(coupling, blk.ir, nu)) > 1e-15):
                Wn = np.zeros_like(Wn)   # symmetric_contraction.py:255-262
            parts.append(Wn)
        T[f"{p}sc.{b}"] = np.concatenate(parts, axis=1)   # (n_el or 1, KT, C)
    for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(hid, hid)):
        T[f"{p}plin.{jo}"] = f64(f"products.{l}.linear.weights.{n}") * pw
    ro = f"readouts.{l}"
    if l < cfg.num_interactions - 1:
        (ji, jo, mi, mo, pw), = linear_instructions(hid, Irreps("0e"))
        T[f"{p}ro"] = f64(f"{ro}.linear.weights.0").reshape(-1) * pw * scale
    else:
        (i1,) = linear_instructions(hid, Irreps("16x0e"))
        (i2,) = linear_instructions(Irreps("16x0e"), Irreps("0e"))
        T[f"{p}ro1"] = f64(f"{ro}.linear_1.weights.0") * i1[4]
        T[f"{p}ro2"] = f64(f"{ro}.linear_2.weights.0").reshape(-1) * i2[4] * scale


def _fold_nonlinear(cfg: ModelConfig, w, l: int, irr_in: Irreps, hid: Irreps, edge: Irreps,
                    T: Dict[str, np.ndarray]) -> None:
    """The non-linear interaction block's tensors (`blocks.py:611-807`): path weights folded in,
    the species parts of both MLPs' first Linear turned into per-species tables (the one-hot
    embedding is a row lookup), linear_1 / linear_res output columns laid out as the gate input
    [scalars | gates of 1o, 2e, 3o | 1o | 2e | 3o] with the four 0e blocks side by side."""
    p, q = f"L{l}.", f"interactions.{l}"
    f64 = lambda k: np.asarray(w[k], dtype=np.float64)
    nel, nb = cfg.num_elements, cfg.num_bessel
    attrs = Irreps(f"{nel}x0e")
    nsc = irr_in.count("0e")
    inter, nonlin = cfg.interaction_irreps, cfg.nonlin_irreps()
    for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(irr_in, edge)):
        assert ji == jo
        T[f"{p}up.{ji}"] = f64(f"{q}.linear_up.weights.{n}") * pw
    for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(irr_in, hid)):
        assert ji == jo
        T[f"{p}skip.{ji}"] = f64(f"{q}.skip_tp.weights.{n}") * pw
    (es,) = linear_instructions(attrs, Irreps(f"{nsc}x0e"))
    src = f64(f"{q}.source_embedding.weights.0") * es[4]   # (n_el, nsc)
    tgt = f64(f"{q}.target_embedding.weights.0") * es[4]
    mp = f"{q}.conv_tp_weights.layers"
    W0 = f64(f"{mp}.0.weight")                            # (64, nb + 2 nsc)
    T[f"{p}rmlp.w0"] = W0[:, :nb].T
    T[f"{p}rmlp.ts"] = src @ W0[:, nb:nb + nsc].T
    T[f"{p}rmlp.tt"] = tgt @ W0[:, nb + nsc:].T + f64(f"{mp}.0.bias")
    T[f"{p}rmlp.w1"] = f64(f"{mp}.3.weight").T
    T[f"{p}rmlp.w2"] = f64(f"{mp}.6.weight").T
    T[f"{p}rmlp.ln"] = np.stack([np.stack([f64(f"{mp}.{k}.weight"), f64(f"{mp}.{k}.bias")]) for k in (1, 4, 7)])
    T[f"{p}rmlp.bias"] = np.stack([f64(f"{mp}.3.bias"), f64(f"{mp}.6.bias")])
    T[f"{p}mlp.3"] = f64(f"{mp}.9.weight").T
    T[f"{p}rmlp.b3"] = f64(f"{mp}.9.bias")
    dp = f"{q}.density_fn.layers"
    D0 = f64(f"{dp}.0.weight")
    T[f"{p}dmlp.w0"] = D0[:, :nb].T
    T[f"{p}dmlp.ts"] = src @ D0[:, nb:nb + nsc].T
    T[f"{p}dmlp.tt"] = tgt @ D0[:, nb + nsc:].T + f64(f"{dp}.0.bias")
    T[f"{p}dmlp.ln"] = np.stack([f64(f"{dp}.1.weight"), f64(f"{dp}.1.bias")])
    T[f"{p}dmlp.w1"] = np.concatenate([f64(f"{dp}.3.weight").reshape(-1), f64(f"{dp}.3.bias").reshape(-1)])
    T[f"{p}ab"] = np.array([float(f64(f"{q}.alpha")), float(f64(f"{q}.beta"))])

    def by_degree(instrs, prefix):
        """{output degree: [C * rows][columns]} with the 0e outputs side by side"""
        cols = {}
        for n, (ji, jo, mi, mo, pw) in enumerate(instrs):
            cols.setdefault(jo, []).append(f64(f"{prefix}.{n}") * pw)
        out = {}
        for jo, mats in cols.items():
            lo = nonlin[jo].ir.l
            out.setdefault(lo, []).append((jo, np.concatenate(mats, axis=0)))
        return {lo: np.concatenate([m for _, m in sorted(v)], axis=1) for lo, v in out.items()}

    mid, _ = conv_tp_instructions(edge, cfg.sh_irreps, inter)
    for lo, m in by_degree(linear_instructions(mid, nonlin), f"{q}.linear_1.weights").items():
        T[f"{p}lin.{lo}"] = m
    for lo, m in by_degree(linear_instructions(edge, nonlin), f"{q}.linear_res.weights").items():
        T[f"{p}res.{lo}"] = m
    for n, (ji, jo, mi, mo, pw) in enumerate(linear_instructions(inter, inter)):
        T[f"{p}lin2.{jo}"] = f64(f"{q}.linear_2.weights.{n}") * pw
