"""Model files in the reference layout: ``config.json`` + ``weights.npz``.

The on-disk format is the one the reference loads in `model.py:664-720`: a JSON
dict of `MACE.__init__` keyword arguments (`model.py:59-82`) plus ``model_type``,
``scale``, ``shift`` and ``z_table``, and an ``.npz`` of float arrays keyed by the
MLX module path (key names as written by `converter.py:315-366,636`, e.g.
``interactions.1.conv_tp_weights.layers.4.weight``).

This module also builds *random-init* models of the BASELINE architectures with
the reference's own initialisation distributions (the reference draws them from
MLX's RNG, which cannot be reproduced here, so models are exchanged as files):

* EquivariantLinear weights ~ N(0, 1)                       (`linear.py:70`)
* FullyConnectedTensorProduct weights ~ N(0, 1)             (`tensor_product.py:286`)
* SymmetricContraction weights ~ N(0, 1) / n_params         (`symmetric_contraction.py:240-252`)
* radial-MLP ``nn.Linear`` weights, stored (out, in): the distribution a
  converted e3nn ``FullyConnectedNet`` has after `converter.py:578-646` folds its
  normalisation into the weights -- N(0, 1) / sqrt(fan_in), times the SiLU
  second-moment factor 1.6791768 (`utils.py:17`) for every layer that follows a
  SiLU.  (MLX's own default, U(+-1/sqrt(fan_in)), shrinks the signal ~3x per
  layer and leaves random models with forces ~1e-4 eV/A, too small to test.)
* Bessel frequencies n*pi/r_max                             (`radial.py:49-51`)
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field, replace
from pathlib import Path
from typing import Dict, List, Optional

import numpy as np

from .irreps import Irrep, Irreps

# 1 / sqrt(E[silu(x)^2]) for x ~ N(0, 1) (`utils.py:17`)
SILU_NORM_FACTOR = 1.6791768074035645
# the same for the sigmoid gate of the non-linear interaction block (`blocks.py:708-717`)
SIGMOID_NORM_FACTOR = 1.8467055569904827
NONLINEAR_BLOCK = "RealAgnosticResidualNonLinearInteractionBlock"

# Published covalent radii (Cordero et al., Dalton Trans. 2008, 2832), in
# Angstrom, indexed by atomic number (index 0 is a placeholder).  The reference
# reads the same table from ase.data.covalent_radii (`radial.py:145-154`).
COVALENT_RADII = np.array([
    0.20, 0.31, 0.28, 1.28, 0.96, 0.84, 0.76, 0.71, 0.66, 0.57, 0.58,  # 0-10
    1.66, 1.41, 1.21, 1.11, 1.07, 1.05, 1.02, 1.06, 2.03, 1.76,        # 11-20
    1.70, 1.60, 1.53, 1.39, 1.39, 1.32, 1.26, 1.24, 1.32, 1.22,        # 21-30
    1.22, 1.20, 1.19, 1.20, 1.20, 1.16, 2.20, 1.95, 1.90, 1.75,        # 31-40
    1.64, 1.54, 1.47, 1.46, 1.42, 1.39, 1.45, 1.44, 1.42, 1.39,        # 41-50
    1.39, 1.38, 1.39, 1.40, 2.44, 2.15, 2.07, 2.04, 2.03, 2.01,        # 51-60
    1.99, 1.98, 1.98, 1.96, 1.94, 1.92, 1.92, 1.89, 1.90, 1.87,        # 61-70
    1.87, 1.75, 1.70, 1.62, 1.51, 1.44, 1.41, 1.36, 1.36, 1.32,        # 71-80
    1.45, 1.46, 1.48, 1.40, 1.50, 1.50, 2.60, 2.21, 2.15, 2.06,        # 81-90
    2.00, 1.96, 1.90, 1.87, 1.80, 1.69,                                # 91-96
], dtype=np.float64)


@dataclass
class ModelConfig:
    """Subset of `MACE.__init__` arguments (`model.py:59-82`) this engine runs."""

    r_max: float
    num_bessel: int = 10
    num_polynomial_cutoff: int = 5
    max_ell: int = 3
    num_interactions: int = 2
    hidden_irreps: str = "128x0e"
    correlation: List[int] = field(default_factory=lambda: [3, 3])
    num_elements: int = 89
    atomic_energies: Optional[List[float]] = None
    avg_num_neighbors: float = 1.0
    radial_MLP: List[int] = field(default_factory=lambda: [64, 64, 64])
    gate: str = "silu"
    model_type: str = "MACE"
    scale: float = 1.0
    shift: float = 0.0
    z_table: Optional[List[int]] = None
    pair_repulsion: Optional[dict] = None
    heads: Optional[List[str]] = None
    first_interaction_nonresidual: bool = False
    use_density_normalization: bool = False
    distance_transform: Optional[dict] = None
    interaction_cls: str = "RealAgnosticResidualInteractionBlock"
    apply_cutoff: bool = True
    use_agnostic_product: bool = False
    edge_irreps: Optional[str] = None

    @staticmethod
    def from_dict(d: dict) -> "ModelConfig":
        d = dict(d)
        # load_model's default when the key is missing (model.py:680)
        d.setdefault("model_type", "ScaleShiftMACE")
        corr = d.get("correlation", 3)
        n_int = int(d.get("num_interactions", 2))
        if isinstance(corr, int):
            corr = [corr] * n_int
        d["correlation"] = [int(c) for c in corr]
        known = set(ModelConfig.__dataclass_fields__)
        unknown = sorted(set(d) - known)
        if unknown:
            raise ValueError(f"unsupported config keys: {unknown}")
        return ModelConfig(**d)

    def to_dict(self) -> dict:
        out = {k: getattr(self, k) for k in self.__dataclass_fields__}
        return {k: v for k, v in out.items() if v is not None}

    def agnesi(self) -> Optional[dict]:
        """AgnesiTransform parameters (`radial.py:207-229` defaults), or None."""
        if self.distance_transform is None:
            return None
        d = {"q": 0.9183, "p": 4.5791, "a": 1.0805}
        d.update({k: float(self.distance_transform[k]) for k in ("q", "p", "a") if k in self.distance_transform})
        return d

    def agnesi_radii(self) -> np.ndarray:
        """Covalent radii (Å) by atomic number used by the distance transform."""
        cov = (self.distance_transform or {}).get("covalent_radii")
        return np.asarray(cov if cov is not None else COVALENT_RADII, dtype=np.float64)

    def residual(self, layer: int) -> bool:
        """Interaction `layer` adds the skip FCTP of its input (`model.py:213-247`)."""
        return not (layer == 0 and self.first_interaction_nonresidual)

    @property
    def nonlinear(self) -> bool:
        """mh-1 family: every interaction is the non-linear block (`model.py:175-211`,
        `blocks.py:611-807`)."""
        return self.interaction_cls == NONLINEAR_BLOCK

    def edge_irreps_per_layer(self) -> List[Irreps]:
        """Output irreps of linear_up in the non-linear block: ``edge_irreps`` (its scalar part
        in the first layer), else the layer's input irreps (`model.py:192-211`,
        `blocks.py:646-657`)."""
        out = []
        for i, irr_in in enumerate(self.layer_inputs()):
            if self.edge_irreps is None:
                out.append(irr_in)
            elif i == 0:
                out.append(Irreps([b for b in Irreps(self.edge_irreps) if b.ir.l == 0]))
            else:
                out.append(Irreps(self.edge_irreps))
        return out

    def nonlin_irreps(self) -> Irreps:
        """Input irreps of the non-linear block's gate: activated scalars, one gate scalar
        block per gated block, then the gated blocks (`blocks.py:700-733`, `gate.py:57-60`)."""
        inter = self.interaction_irreps
        scal = [b for b in inter if b.ir.l == 0]
        gated = [b for b in inter if b.ir.l > 0]
        return Irreps(scal + [(b.mul, Irrep(0, 1)) for b in gated] + gated)

    # --- derived architecture (model.py:96-145) -----------------------------
    @property
    def hidden(self) -> Irreps:
        return Irreps(self.hidden_irreps)

    @property
    def num_heads(self) -> int:
        """Readout heads (`model.py:89-91`): one per entry of ``heads``, else one."""
        return len(self.heads) if self.heads else 1

    @property
    def num_features(self) -> int:
        return self.hidden[0].mul

    @property
    def sh_irreps(self) -> Irreps:
        return Irreps.spherical_harmonics(self.max_ell)

    @property
    def interaction_irreps(self) -> Irreps:
        return Irreps([(self.num_features, b.ir) for b in self.sh_irreps])

    def hidden_per_layer(self) -> List[Irreps]:
        scal = Irreps([b for b in self.hidden if b.ir.l == 0])
        return [self.hidden if i < self.num_interactions - 1 else scal
                for i in range(self.num_interactions)]

    def layer_inputs(self) -> List[Irreps]:
        scal = Irreps([b for b in self.hidden if b.ir.l == 0])
        hid = self.hidden_per_layer()
        return [scal] + hid[:-1]

    def check_supported(self) -> None:
        """Raise NotImplementedError for topology options outside this engine."""
        if self.interaction_cls not in ("RealAgnosticResidualInteractionBlock", NONLINEAR_BLOCK):
            raise NotImplementedError(f"interaction_cls={self.interaction_cls}")
        if self.nonlinear and (self.first_interaction_nonresidual or self.use_density_normalization):
            raise NotImplementedError("non-linear interaction blocks with the density / non-residual layout")
        if self.distance_transform is not None:
            unknown = set(self.distance_transform) - {"q", "p", "a", "covalent_radii"}
            if unknown:
                raise NotImplementedError(f"distance_transform keys {sorted(unknown)}")
        if not self.apply_cutoff and not self.nonlinear:
            raise NotImplementedError("apply_cutoff=False outside the non-linear interaction block")
        if self.gate != "silu":
            raise NotImplementedError(f"gate={self.gate}")
        if any(b.ir.l == 0 and b.ir.p != 1 for b in self.hidden):
            raise NotImplementedError("pseudoscalar hidden irreps")


def load_config(model_dir: str | Path) -> ModelConfig:
    with open(Path(model_dir) / "config.json") as f:
        return ModelConfig.from_dict(json.load(f))


def load_weights(model_dir: str | Path) -> Dict[str, np.ndarray]:
    with np.load(Path(model_dir) / "weights.npz", allow_pickle=False) as z:
        return {k: np.asarray(z[k]) for k in z.files}


def save_model(model_dir: str | Path, cfg: ModelConfig, weights: Dict[str, np.ndarray]) -> Path:
    p = Path(model_dir)
    p.mkdir(parents=True, exist_ok=True)
    with open(p / "config.json", "w") as f:
        json.dump(cfg.to_dict(), f, indent=1)
    np.savez(p / "weights.npz", **{k: np.asarray(v, dtype=np.float32) for k, v in weights.items()})
    return p


# ---------------------------------------------------------------------------
# Weight-key inventory (shapes) for a config, in the reference's module layout
# ---------------------------------------------------------------------------


def linear_instructions(irreps_in: Irreps, irreps_out: Irreps):
    """EquivariantLinear instruction list (`linear.py:46-74`): outer loop over
    input blocks, inner over output blocks; path weight 1/sqrt(sum of input
    multiplicities feeding the output block)."""
    tot = {}
    for jo, bo in enumerate(irreps_out):
        tot[jo] = sum(bi.mul for bi in irreps_in if bi.ir == bo.ir)
    out = []
    for ji, bi in enumerate(irreps_in):
        for jo, bo in enumerate(irreps_out):
            if bi.ir != bo.ir:
                continue
            pw = 1.0 / math.sqrt(tot[jo]) if tot[jo] > 0 else 1.0
            out.append((ji, jo, bi.mul, bo.mul, pw))
    return out


def conv_tp_instructions(irreps1: Irreps, irreps2: Irreps, target: Irreps):
    """`tp_out_irreps_with_instructions` (`utils.py:87-156`): returns the sorted
    mid irreps and [(i1, i2, i_out, path_weight)] sorted by i_out."""
    outs, inst = [], []
    for i, b1 in enumerate(irreps1):
        for j, b2 in enumerate(irreps2):
            for ir in b1.ir.couple(b2.ir):
                if ir in target:
                    inst.append((i, j, len(outs), b2.mul))
                    outs.append((b1.mul, ir))
    alpha = {}
    for (_, _, k, m2) in inst:
        alpha[k] = alpha.get(k, 0.0) + m2
    mid = Irreps(outs)
    mid_sorted, _, inv = mid.sorted_with_perm()
    res = []
    for (i, j, k, _) in inst:
        pw = math.sqrt(outs[k][1].dim / alpha[k]) if alpha[k] > 0 else 1.0
        res.append((i, j, inv[k], pw))
    res.sort(key=lambda t: t[2])
    return mid_sorted, res


def fctp_instructions(irreps1: Irreps, irreps2: Irreps, irreps_out: Irreps):
    """FullyConnectedTensorProduct instructions (`tensor_product.py:1068-1098`):
    [(i1, i2, i_out, path_weight)] in (i1, i2, i_out) loop order."""
    inst = []
    for i, b1 in enumerate(irreps1):
        for j, b2 in enumerate(irreps2):
            for k, bo in enumerate(irreps_out):
                if b1.ir.p * b2.ir.p != bo.ir.p:
                    continue
                if not (abs(b1.ir.l - b2.ir.l) <= bo.ir.l <= b1.ir.l + b2.ir.l):
                    continue
                inst.append((i, j, k))
    alpha = {}
    for (i, j, k) in inst:
        alpha[k] = alpha.get(k, 0.0) + irreps1[i].mul * irreps2[j].mul
    return [(i, j, k, math.sqrt(irreps_out[k].ir.dim / alpha[k])) for (i, j, k) in inst]


def weight_shapes(cfg: ModelConfig) -> Dict[str, tuple]:
    """Key -> shape for every array the reference's MACE module tree holds."""
    from .cg import u_matrix  # local import: scipy-free callers stay light

    cfg.check_supported()
    shapes: Dict[str, tuple] = {}
    nel = cfg.num_elements
    C = cfg.num_features
    attrs = Irreps(f"{nel}x0e")
    H = cfg.num_heads
    # (num_elements,) single-head, (num_heads, num_elements) multi-head (converter.py:175-185)
    shapes["atomic_energies_fn.atomic_energies"] = (H, nel) if H > 1 else (nel,)
    scal = Irreps([b for b in cfg.hidden if b.ir.l == 0])
    for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(attrs, scal)):
        shapes[f"node_embedding.linear.weights.{n}"] = (mi, mo)
    shapes["radial_embedding.bessel_fn.bessel_weights"] = (cfg.num_bessel,)
    inter = cfg.interaction_irreps
    if cfg.nonlinear:
        _nonlinear_shapes(cfg, shapes)
    for li, (irr_in, hid) in enumerate(zip(cfg.layer_inputs(), cfg.hidden_per_layer())):
        p = f"interactions.{li}"
        if cfg.nonlinear:
            _product_readout_shapes(cfg, li, hid, shapes)
            continue
        # residual blocks skip from the layer input to the hidden irreps; the non-residual
        # first block (blocks.py:68-176) applies its skip FCTP to the message
        s_in, s_out = (irr_in, hid) if cfg.residual(li) else (inter, inter)
        for n, (i, j, k, _) in enumerate(fctp_instructions(s_in, attrs, s_out)):
            shapes[f"{p}.skip_tp.tp.weights.{n}"] = (s_in[i].mul, attrs[j].mul, s_out[k].mul)
        if cfg.use_density_normalization:  # nn.Linear(num_radial, 1, bias=False), blocks.py:331-332
            shapes[f"{p}.density_fn.weight"] = (1, cfg.num_bessel)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(irr_in, irr_in)):
            shapes[f"{p}.linear_up.weights.{n}"] = (mi, mo)
        mid, tpi = conv_tp_instructions(irr_in, cfg.sh_irreps, inter)
        wnum = sum(irr_in[i].mul * cfg.sh_irreps[j].mul for (i, j, _, _) in tpi)
        dims = [cfg.num_bessel] + list(cfg.radial_MLP) + [wnum]
        for n in range(len(dims) - 1):
            shapes[f"{p}.conv_tp_weights.layers.{2 * n}.weight"] = (dims[n + 1], dims[n])
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(mid, inter)):
            shapes[f"{p}.linear.weights.{n}"] = (mi, mo)
        _product_readout_shapes(cfg, li, hid, shapes)
    return shapes


def _product_readout_shapes(cfg: ModelConfig, li: int, hid: Irreps, shapes: Dict[str, tuple]) -> None:
    from .cg import u_matrix

    C, H, inter = cfg.num_features, cfg.num_heads, cfg.interaction_irreps
    # the element-agnostic product has one set of weights (`model.py:250-258`)
    nel = 1 if cfg.use_agnostic_product else cfg.num_elements
    q = f"products.{li}"
    coupling = Irreps([(1, b.ir) for b in inter])
    for ci, b in enumerate(hid):
        cp = f"{q}.symmetric_contractions.contractions.{ci}"
        corr = cfg.correlation[li]
        shapes[f"{cp}.weights_max"] = (nel, u_matrix(coupling, b.ir, corr).shape[-1], C)
        for wi, nu in enumerate(range(corr - 1, 0, -1)):
            shapes[f"{cp}.weights.{wi}"] = (nel, u_matrix(coupling, b.ir, nu).shape[-1], C)
    for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(hid, hid)):
        shapes[f"{q}.linear.weights.{n}"] = (mi, mo)
    r = f"readouts.{li}"
    # readouts give num_heads x 0e; the last one's MLP has 16 x num_heads scalars
    # (model.py:135-139)
    out = Irreps(f"{H}x0e")
    if li < cfg.num_interactions - 1:
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(hid, out)):
            shapes[f"{r}.linear.weights.{n}"] = (mi, mo)
    else:
        mlp = Irreps(f"{16 * H}x0e")
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(hid, mlp)):
            shapes[f"{r}.linear_1.weights.{n}"] = (mi, mo)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(mlp, out)):
            shapes[f"{r}.linear_2.weights.{n}"] = (mi, mo)


def _nonlinear_shapes(cfg: ModelConfig, shapes: Dict[str, tuple]) -> None:
    """Arrays of the non-linear interaction block (`blocks.py:611-733`): source / target
    species embeddings, plain-linear skip, linear_up, LayerNorm radial MLP and density MLP
    (``layers.{k}``: Linear at 0, 3, 6, ..., LayerNorm at 1, 4, 7, ...; `radial.py:344-357`),
    alpha / beta, linear_res, linear_1, linear_2."""
    nel = cfg.num_elements
    attrs = Irreps(f"{nel}x0e")
    inter = cfg.interaction_irreps
    nonlin = cfg.nonlin_irreps()
    for li, (irr_in, hid, edge) in enumerate(zip(cfg.layer_inputs(), cfg.hidden_per_layer(),
                                                 cfg.edge_irreps_per_layer())):
        p = f"interactions.{li}"
        nsc = irr_in.count("0e")
        for name in ("source_embedding", "target_embedding"):
            for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(attrs, Irreps(f"{nsc}x0e"))):
                shapes[f"{p}.{name}.weights.{n}"] = (mi, mo)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(irr_in, hid)):
            shapes[f"{p}.skip_tp.weights.{n}"] = (mi, mo)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(irr_in, edge)):
            shapes[f"{p}.linear_up.weights.{n}"] = (mi, mo)
        mid, tpi = conv_tp_instructions(edge, cfg.sh_irreps, inter)
        wnum = sum(edge[i].mul * cfg.sh_irreps[j].mul for (i, j, _, _) in tpi)
        aug = cfg.num_bessel + 2 * nsc
        for name, dims in (("conv_tp_weights", [aug] + list(cfg.radial_MLP) + [wnum]),
                           ("density_fn", [aug, 64, 1])):
            for k in range(len(dims) - 1):
                shapes[f"{p}.{name}.layers.{3 * k}.weight"] = (dims[k + 1], dims[k])
                shapes[f"{p}.{name}.layers.{3 * k}.bias"] = (dims[k + 1],)
                if k < len(dims) - 2:
                    shapes[f"{p}.{name}.layers.{3 * k + 1}.weight"] = (dims[k + 1],)
                    shapes[f"{p}.{name}.layers.{3 * k + 1}.bias"] = (dims[k + 1],)
        shapes[f"{p}.alpha"] = ()
        shapes[f"{p}.beta"] = ()
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(edge, nonlin)):
            shapes[f"{p}.linear_res.weights.{n}"] = (mi, mo)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(mid, nonlin)):
            shapes[f"{p}.linear_1.weights.{n}"] = (mi, mo)
        for n, (ji, jo, mi, mo, _) in enumerate(linear_instructions(inter, inter)):
            shapes[f"{p}.linear_2.weights.{n}"] = (mi, mo)


def random_init(cfg: ModelConfig, seed: int = 0) -> Dict[str, np.ndarray]:
    """Random-init weights with the reference's initialisation distributions.

    Keys are drawn in sorted order from one ``np.random.default_rng(seed)``
    stream, so the result depends only on (cfg, seed)."""
    rng = np.random.default_rng(seed)
    shapes = weight_shapes(cfg)
    w: Dict[str, np.ndarray] = {}
    for key in sorted(shapes):
        shp = shapes[key]
        if key == "atomic_energies_fn.atomic_energies":
            ae = cfg.atomic_energies
            w[key] = np.zeros(shp) if ae is None else np.asarray(ae, dtype=np.float64).reshape(shp)
        elif key == "radial_embedding.bessel_fn.bessel_weights":
            w[key] = np.arange(1, shp[0] + 1, dtype=np.float64) * math.pi / cfg.r_max
        elif cfg.nonlinear and (".conv_tp_weights." in key or ".density_fn." in key):
            # nn.Linear's U(+-1/sqrt(fan_in)) for weights and biases (MLX default); LayerNorm
            # scale / shift drawn around MLX's 1 / 0 so that a test exercises them
            k = int(key.split(".layers.")[1].split(".")[0])
            if k % 3 == 1:
                w[key] = (1.0 if key.endswith(".weight") else 0.0) + 0.1 * rng.standard_normal(shp)
            else:
                fan_in = shapes[key.rsplit(".", 1)[0] + ".weight"][1]
                w[key] = rng.uniform(-1.0, 1.0, shp) / math.sqrt(fan_in)
        elif key.endswith(".alpha") or key.endswith(".beta"):
            # the block starts from alpha = 20, beta = 0 (blocks.py:697-698): the density off and
            # every message damped 20x, which leaves a random model with forces ~0.01 eV/A;
            # a random model takes alpha in [1.5, ~4.5] and beta in [0.1, ~0.4] instead, which
            # keeps its forces at O(1-10) eV/A on bulk, ragged and three-species systems (the
            # correlation-3 product makes them scale roughly with alpha^-3)
            a0, sc = (1.5, 1.5) if key.endswith(".alpha") else (0.1, 0.1)
            w[key] = np.asarray(a0 + sc * abs(rng.standard_normal()))
        elif ".conv_tp_weights." in key:
            layer = int(key.split(".layers.")[1].split(".")[0])
            scale = 1.0 / math.sqrt(shp[1]) * (SILU_NORM_FACTOR if layer > 0 else 1.0)
            w[key] = rng.standard_normal(shp) * scale
        elif key.endswith(".density_fn.weight"):
            w[key] = rng.standard_normal(shp) / math.sqrt(shp[1])
        elif ".symmetric_contractions." in key:
            w[key] = rng.standard_normal(shp) / shp[1]
        else:
            w[key] = rng.standard_normal(shp)
    return {k: v.astype(np.float32) for k, v in w.items()}


def head_index(cfg: ModelConfig, head: Optional[str] = None) -> int:
    """Index of the active head: the named one, else the first (`calculators.py:128-137`);
    single-head models ignore ``head``."""
    if cfg.num_heads == 1:
        return 0
    name = cfg.heads[0] if head is None else head
    if name not in cfg.heads:
        raise ValueError(f"Head '{name}' not found in model heads: {cfg.heads}")
    return cfg.heads.index(name)


def select_head(cfg: ModelConfig, w: Dict[str, np.ndarray],
                head: Optional[str] = None) -> tuple:
    """The single-head model whose energy equals head ``head`` of ``cfg``.

    The reference evaluates every head and then picks one column: E0 and the readouts
    give (N, num_heads) and `_e0_select_head` / `_readout_select_head` take the active
    column (`model.py:302-326`); the non-linear readout multiplies its 16 x num_heads
    gated features by a mask that keeps the active head's 16 (`blocks.py:583-608`)
    before `linear_2`, whose path weight is 1/sqrt(16 x num_heads) (`linear.py:46-74`);
    ScaleShiftMACE takes the active entry of per-head scale / shift lists, falling back
    to entry 0 (`model.py:530-548`).  Keeping only the active head's weights gives the
    same numbers: `linear_2`'s rows are rescaled by 1/sqrt(num_heads) so that the
    single-head path weight 1/sqrt(16) reproduces 1/sqrt(16 x num_heads)."""
    h = head_index(cfg, head)
    H = cfg.num_heads

    def pick(v):
        if isinstance(v, (list, tuple)):
            return float(v[h] if h < len(v) else v[0])
        return float(v)

    ae = cfg.atomic_energies
    if ae is not None and H > 1:
        ae = [float(x) for x in np.asarray(ae, dtype=np.float64).reshape(H, -1)[h]]
    out_cfg = replace(cfg, heads=None, scale=pick(cfg.scale), shift=pick(cfg.shift), atomic_energies=ae)
    if H == 1:
        return out_cfg, dict(w)
    last = f"readouts.{cfg.num_interactions - 1}."
    out: Dict[str, np.ndarray] = {}
    for k, v in w.items():
        v = np.asarray(v)
        if k == "atomic_energies_fn.atomic_energies":
            v = v.reshape(H, -1)[h]
        elif k.startswith(last + "linear_1.weights."):
            v = v[:, 16 * h:16 * (h + 1)]
        elif k.startswith(last + "linear_2.weights."):
            # kept in float64: the reference applies the path weight at run time
            v = v[16 * h:16 * (h + 1), h:h + 1].astype(np.float64) / math.sqrt(H)
        elif k.startswith("readouts.") and ".linear.weights." in k:
            v = v[:, h:h + 1]
        out[k] = np.ascontiguousarray(v)
    return out_cfg, out


# ---------------------------------------------------------------------------
# Channel padding: a model of C channels as an equivalent model of C' > C channels
# ---------------------------------------------------------------------------

def pad_channels(cfg: ModelConfig, w: Dict[str, np.ndarray], target: int):
    """(cfg', w') with every irrep multiplicity C raised to ``target`` such that the padded
    model computes the same energies as the original: the extra channels carry zeros
    everywhere.  Rules, checked against the weight inventories of both configs:

    * per-channel weights -- conv-TP weights of the radial MLP's last layer (rows slot-major,
      channel-minor, `tensor_product.py:728-735`), symmetric-contraction weights
      [n_el][k][C], the node embedding's outputs, output columns of every linear -- are
      zero-padded;
    * weights summed over an input channel axis (EquivariantLinear `linear.py:46-74` and the
      skip FCTP `tensor_product.py:1080-1098`, whose path weights are 1/sqrt(fan-in) with the
      fan-in proportional to C) are zero-padded and multiplied by sqrt(target / C), so that the
      padded model's path weight 1/sqrt(n target) reproduces 1/sqrt(n C).

    A zero channel stays zero through the channel-wise conv TP, the symmetric contraction (no
    constant term) and the gate-free readouts, so no padded value reaches a real one."""
    C = cfg.num_features
    if any(b.mul != C for b in cfg.hidden):
        raise NotImplementedError(f"hidden irreps {cfg.hidden_irreps} with unequal multiplicities")
    if target < C:
        raise ValueError(f"cannot pad {C} channels down to {target}")
    if target == C:
        return cfg, dict(w)
    if cfg.nonlinear:
        raise NotImplementedError("channel padding of the non-linear interaction block")
    hid = Irreps([(target, b.ir) for b in cfg.hidden])
    cfg2 = replace(cfg, hidden_irreps=str(hid))
    s1, s2 = weight_shapes(cfg), weight_shapes(cfg2)
    assert set(s1) == set(s2)
    f = math.sqrt(target / C)
    out: Dict[str, np.ndarray] = {}
    for k, v in w.items():
        a, b = s1.get(k), s2.get(k)
        v = np.asarray(v)
        if a is None or tuple(a) == tuple(b):
            out[k] = v
            continue
        if ".conv_tp_weights." in k:
            n = a[0] // C
            assert a[0] == n * C and b[0] == n * target and a[1:] == b[1:], (k, a, b)
            p = np.zeros((n, target) + tuple(a[1:]), dtype=v.dtype)
            p[:, :C] = v.reshape((n, C) + tuple(a[1:]))
            out[k] = p.reshape(b)
            continue
        assert len(a) == len(b), (k, a, b)
        axes = [i for i in range(len(a)) if a[i] != b[i]]
        assert all(a[i] == C and b[i] == target for i in axes), (k, a, b)
        p = np.zeros(b, dtype=np.float64)      # the compensation factor applied in float64
        p[tuple(slice(0, s) for s in a)] = v
        summed = (".symmetric_contractions." not in k and not k.startswith("node_embedding.") and 0 in axes)
        out[k] = p * f if summed else p
    return cfg2, out
