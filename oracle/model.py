"""PyTorch-CPU restatement of the reference MACE energy model -- TEST INFRASTRUCTURE ONLY.

Semantics follow the reference's generic code paths:

* edge geometry                `utils.py:47-84` (stress variant `calculators.py:532-557`)
* spherical harmonics          `spherical_harmonics.py:67-155` (e3nn basis, component norm)
* Bessel x polynomial cutoff   `radial.py:18-71,108-124,265-321`
* ZBL pair repulsion           `radial.py:127-201`
* radial MLP                   `radial.py:329-341` (no bias, plain SiLU)
* EquivariantLinear            `linear.py:421-446` (`_loop_forward`)
* conv tensor product          `tensor_product.py:833-893,895-1043` (`_loop_forward`, uvu)
* FullyConnectedTensorProduct  `tensor_product.py:1046-1098` (uvw, internal weights)
* symmetric contraction        `symmetric_contraction.py:505-595` (row-compressed main
                               step over U's nonzero (i, k) pairs + dense lower chain,
                               i.e. the reference's CPU path)
* interaction / product / readout blocks `blocks.py:179-279,493-608`; the trained-model
                               variants: Agnesi distance transform `radial.py:207-262`,
                               density normalisation `blocks.py:282-490`, non-residual
                               first interaction `blocks.py:68-176`, `model.py:213-247`
* mh-1 family                  non-linear interaction block `blocks.py:611-807` (species
                               source / target embeddings, LayerNorm radial and density
                               MLPs `radial.py:344-357`, gate `gate.py:19-164` with the
                               normalize2mom constants `blocks.py:708-717`, linear_res,
                               linear_1 / (beta rho + alpha), linear_2), separate cutoff
                               (`radial.py:265-321` apply_cutoff=False), element-agnostic
                               product (`blocks.py:493-537`)
* energy assembly              `model.py:403-438`; ScaleShiftMACE `model.py:508-589`;
                               multi-head readouts: every head evaluated, the non-linear
                               readout's features masked to the active head, the active
                               column taken (`model.py:302-326,392-400`, `blocks.py:553-608`)
* forces / stress              `calculators.py:440-563` (autograd; symmetric displacement)

Constants (3j, U) come from ``mace_mlx_amd.cg``, which is pinned against golden
vectors written from the reference.  The architecture bookkeeping (instruction
lists, path weights) is restated here independently of the product's kernel
tables so that a mistake in either shows up as a parity failure.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch
from torch.utils.checkpoint import checkpoint

_PKG = Path(__file__).resolve().parents[1] / "mace-mlx_amd"
if str(_PKG) not in sys.path:
    sys.path.insert(0, str(_PKG))

from mace_mlx_amd.cg import so3_cg, u_matrix, wigner_3j  # noqa: E402
from mace_mlx_amd.irreps import Irrep, Irreps  # noqa: E402
from mace_mlx_amd.model_io import (COVALENT_RADII, SIGMOID_NORM_FACTOR,  # noqa: E402
                                   SILU_NORM_FACTOR, ModelConfig, load_config, load_weights)


def _t(x, dtype):
    return torch.as_tensor(np.asarray(x, dtype=np.float64), dtype=dtype)


# ---------------------------------------------------------------------------
# Edge front end
# ---------------------------------------------------------------------------


def spherical_harmonics(v: torch.Tensor, lmax: int) -> torch.Tensor:
    """Real SH, e3nn basis, component normalisation, recursion of
    `spherical_harmonics.py:112-155` (l=1 seed sqrt(3)*(x, y, z))."""
    sq = (v * v).sum(-1, keepdim=True)
    r = torch.sqrt(torch.clamp(sq, min=1e-24))
    u = v / r
    blocks = [torch.ones_like(u[..., :1])]
    if lmax >= 1:
        Y1 = math.sqrt(3.0) * u
        blocks.append(Y1)
        prev = Y1
        for l in range(2, lmax + 1):
            c = l - 1
            C = torch.as_tensor(so3_cg(c, 1, l) * math.sqrt((2 * l + 1) / (3 * l)), dtype=v.dtype)
            prev = torch.einsum("ei,ej,ijk->ek", prev, Y1, C)
            blocks.append(prev)
    return torch.cat(blocks, dim=-1)


def poly_envelope(u: torch.Tensor, p: int) -> torch.Tensor:
    pf = float(p)
    up = u ** p
    env = (1.0 - (pf + 1.0) * (pf + 2.0) / 2.0 * up + pf * (pf + 2.0) * up * u
           - pf * (pf + 1.0) / 2.0 * up * u * u)
    return env * (u < 1.0).to(u.dtype)


def bessel(r: torch.Tensor, w: torch.Tensor, r_max: float) -> torch.Tensor:
    x = r[:, None]
    num = torch.sin(w[None, :] * x)
    safe = torch.where(x == 0.0, torch.ones_like(x), x)
    out = math.sqrt(2.0 / r_max) * num / safe
    return torch.where(x == 0.0, math.sqrt(2.0 / r_max) * w[None, :].expand_as(out), out)


def agnesi(r, zs, zr, params, radii):
    """AgnesiTransform, `radial.py:231-262`: r / r0 with r0 the mean covalent radius of
    the pair, mapped to 1 / (1 + a x^q / (1 + x^(q - p)))."""
    r0 = 0.5 * (radii[zs] + radii[zr])
    x = torch.clamp(r / r0, min=1e-12)
    q, p, a = params["q"], params["p"], params["a"]
    return 1.0 / (1.0 + a * x ** q / (1.0 + x ** (q - p)))


# Universal screening function phi(x) = sum_k c_k exp(-d_k x) of Ziegler, Biersack and
# Littmark, at the 4-digit rounding the reference uses (`radial.py:149,184-189`), with its
# Bohr radius (Angstrom) and e^2 / (4 pi eps0) (eV Angstrom, `radial.py:179-181,191-192`).
ZBL_C = (0.1818, 0.5099, 0.2802, 0.02817)
ZBL_D = (3.2, 0.9423, 0.4028, 0.2016)
ZBL_BOHR = 0.529
ZBL_COULOMB = 14.3996


def zbl_node_energy(r, zs, zr, receiver, n_nodes, params):
    """Per-node ZBL repulsion, `radial.py:156-201`: half of each edge's pair energy
    V(r) = ke Z_u Z_v / r phi(r / a), a = a_prefactor a0 / (Z_u^a_exp + Z_v^a_exp), times the
    polynomial envelope at r / (r_cov(Z_u) + r_cov(Z_v)), summed onto the receiver."""
    dtype = r.dtype
    p = int(params.get("p", 6))
    a_exp = float(params.get("a_exp", 0.3))
    a_pref = float(params.get("a_prefactor", 0.4543))
    zu = zs.to(dtype)
    zv = zr.to(dtype)
    a = a_pref * ZBL_BOHR / (zu ** a_exp + zv ** a_exp)
    x = r / a
    phi = sum(c * torch.exp(-d * x) for c, d in zip(ZBL_C, ZBL_D))
    v = ZBL_COULOMB * zu * zv / r * phi
    cov = torch.as_tensor(COVALENT_RADII, dtype=dtype)
    rmax = cov[zs] + cov[zr]
    v = 0.5 * v * poly_envelope(r / rmax, p)
    out = torch.zeros(n_nodes, dtype=dtype)
    return out.index_add(0, receiver, v)


# ---------------------------------------------------------------------------
# Equivariant building blocks
# ---------------------------------------------------------------------------


class Linear:
    """`linear.py:28-446` loop form: per matching (i_in, i_out) pair
    out[w, m] += pw * sum_u x[u, m] W[u, w]."""

    def __init__(self, irreps_in, irreps_out, weights: List[torch.Tensor]):
        self.ii, self.io = Irreps(irreps_in), Irreps(irreps_out)
        tot = {jo: sum(bi.mul for bi in self.ii if bi.ir == bo.ir) for jo, bo in enumerate(self.io)}
        self.inst = []
        for ji, bi in enumerate(self.ii):
            for jo, bo in enumerate(self.io):
                if bi.ir == bo.ir:
                    self.inst.append((ji, jo, 1.0 / math.sqrt(tot[jo])))
        assert len(self.inst) == len(weights), (len(self.inst), len(weights))
        self.w = weights

    def __call__(self, x):
        B = x.shape[:-1]
        offs_i, offs_o = self.ii.offsets, self.io.offsets
        parts = [torch.zeros(*B, b.dim, dtype=x.dtype) for b in self.io]
        for (ji, jo, pw), W in zip(self.inst, self.w):
            bi = self.ii[ji]
            xb = x[..., offs_i[ji]:offs_i[ji] + bi.dim].reshape(*B, bi.mul, bi.ir.dim)
            yb = pw * torch.einsum("...ui,uw->...wi", xb, W)
            parts[jo] = parts[jo] + yb.reshape(*B, -1)
        return torch.cat(parts, dim=-1) if parts else x[..., :0]


def conv_tp_instructions(irreps1: Irreps, irreps2: Irreps, target: Irreps):
    """`utils.py:87-156` restated."""
    outs, inst = [], []
    for i, b1 in enumerate(irreps1):
        for j, b2 in enumerate(irreps2):
            for l in range(abs(b1.ir.l - b2.ir.l), b1.ir.l + b2.ir.l + 1):
                ir = Irrep(l, b1.ir.p * b2.ir.p)
                if ir in target:
                    inst.append([i, j, len(outs), b2.mul])
                    outs.append((b1.mul, ir))
    alpha = {}
    for _, _, k, m2 in inst:
        alpha[k] = alpha.get(k, 0) + m2
    order = sorted(range(len(outs)), key=lambda k: (outs[k][1].l, outs[k][1].p))
    inv = {k: n for n, k in enumerate(order)}
    mid = Irreps([outs[k] for k in order])
    res = sorted([(i, j, inv[k], math.sqrt(outs[k][1].dim / alpha[k])) for i, j, k, _ in inst],
                 key=lambda t: t[2])
    return mid, res


class ConvTP:
    """uvu tensor product with per-edge external weights, `_loop_forward`."""

    def __init__(self, irreps1, irreps2, target):
        self.i1, self.i2 = Irreps(irreps1), Irreps(irreps2)
        self.mid, self.inst = conv_tp_instructions(self.i1, self.i2, Irreps(target))
        self.weight_numel = sum(self.i1[i].mul * self.i2[j].mul for i, j, _, _ in self.inst)

    def __call__(self, x1, x2, w):
        E = x1.shape[0]
        o1, o2 = self.i1.offsets, self.i2.offsets
        parts = [None] * len(self.mid)
        woff = 0
        for (i, j, k, pw) in self.inst:
            b1, b2, bo = self.i1[i], self.i2[j], self.mid[k]
            cg = torch.as_tensor(wigner_3j(b1.ir.l, b2.ir.l, bo.ir.l), dtype=x1.dtype)
            xa = x1[:, o1[i]:o1[i] + b1.dim].reshape(E, b1.mul, b1.ir.dim)
            xb = x2[:, o2[j]:o2[j] + b2.dim].reshape(E, b2.mul, b2.ir.dim)
            nw = b1.mul * b2.mul
            ww = w[:, woff:woff + nw].reshape(E, b1.mul, b2.mul)
            woff += nw
            tp = torch.einsum("eui,evj,ijk->euvk", xa, xb, cg)
            out = torch.einsum("euvk,euv->euk", tp, ww) * pw
            parts[k] = out.reshape(E, -1) if parts[k] is None else parts[k] + out.reshape(E, -1)
        return torch.cat(parts, dim=-1)


class ConvTPGemm(ConvTP):
    """The same tensor product in the x2-first GEMM form of the reference's CPU path
    (`tensor_product.py:497-513,545-575`): for each input block, the edge's CG table
    M[e, i, col] = sum_j Y[e, j] C_s[i, j, k] pw_s over that block's output slots, then one batched
    product x1[e] (mul x d1) @ M[e] (d1 x K), times the slot's per-channel weight.  Used to time the
    CPU baseline; equal to the loop form (tests/test_oracle.py)."""

    def __init__(self, irreps1, irreps2, target):
        super().__init__(irreps1, irreps2, target)
        self.groups = {}
        woff = 0
        for (i, j, k, pw) in self.inst:
            b1, b2, bo = self.i1[i], self.i2[j], self.mid[k]
            cg = np.asarray(wigner_3j(b1.ir.l, b2.ir.l, bo.ir.l)) * pw
            self.groups.setdefault(i, []).append((j, k, cg, woff))
            woff += b1.mul * b2.mul

    def __call__(self, x1, x2, w):
        E = x1.shape[0]
        o1, o2 = self.i1.offsets, self.i2.offsets
        parts = [None] * len(self.mid)
        for i, slots in self.groups.items():
            b1 = self.i1[i]
            d1 = b1.ir.dim
            cols, widths = [], []
            for (j, k, cg, woff) in slots:
                b2 = self.i2[j]
                yj = x2[:, o2[j]:o2[j] + b2.dim]                                   # (E, d2)
                cols.append(torch.einsum("ej,ijk->eik", yj, torch.as_tensor(cg, dtype=x1.dtype)))
                widths.append(cg.shape[2])
            M = torch.cat(cols, dim=2)                                           # (E, d1, K)
            xa = x1[:, o1[i]:o1[i] + b1.dim].reshape(E, b1.mul, d1)
            T = torch.bmm(xa, M)                                                 # (E, mul, K)
            c0 = 0
            for (j, k, cg, woff), wd in zip(slots, widths):
                ww = w[:, woff:woff + b1.mul]                                    # uvu, mul2 = 1
                out = (T[:, :, c0:c0 + wd] * ww[:, :, None]).reshape(E, -1)
                parts[k] = out if parts[k] is None else parts[k] + out
                c0 += wd
        return torch.cat(parts, dim=-1)


class SkipFCTP:
    """FullyConnectedTensorProduct (uvw, internal weights) with the one-hot
    attributes as second input, `tensor_product.py:1046-1098` + `_compute_mode`."""

    def __init__(self, irreps1, n_el, irreps_out, weights):
        self.i1 = Irreps(irreps1)
        self.i2 = Irreps(f"{n_el}x0e")
        self.io = Irreps(irreps_out)
        inst = []
        for i, b1 in enumerate(self.i1):
            for j, b2 in enumerate(self.i2):
                for k, bo in enumerate(self.io):
                    if b1.ir.p * b2.ir.p == bo.ir.p and abs(b1.ir.l - b2.ir.l) <= bo.ir.l <= b1.ir.l + b2.ir.l:
                        inst.append((i, j, k))
        alpha = {}
        for i, j, k in inst:
            alpha[k] = alpha.get(k, 0) + self.i1[i].mul * self.i2[j].mul
        self.inst = [(i, j, k, math.sqrt(self.io[k].ir.dim / alpha[k])) for i, j, k in inst]
        assert len(self.inst) == len(weights)
        self.w = weights

    def __call__(self, x1, onehot):
        B = x1.shape[0]
        o1, o2, oo = self.i1.offsets, self.i2.offsets, self.io.offsets
        parts = [torch.zeros(B, b.dim, dtype=x1.dtype) for b in self.io]
        for (i, j, k, pw), W in zip(self.inst, self.w):
            b1, b2, bo = self.i1[i], self.i2[j], self.io[k]
            cg = torch.as_tensor(wigner_3j(b1.ir.l, b2.ir.l, bo.ir.l), dtype=x1.dtype)
            xa = x1[:, o1[i]:o1[i] + b1.dim].reshape(B, b1.mul, b1.ir.dim)
            xb = onehot[:, o2[j]:o2[j] + b2.dim].reshape(B, b2.mul, b2.ir.dim)
            tp = torch.einsum("bui,bvj,ijk->buvk", xa, xb, cg)
            out = torch.einsum("buvk,uvw->bwk", tp, W) * pw
            parts[k] = parts[k] + out.reshape(B, -1)
        return torch.cat(parts, dim=-1)


class Contraction:
    """One output irrep of the symmetric contraction (`symmetric_contraction.py:124-595`)."""

    def __init__(self, coupling: Irreps, ir_out: Irrep, corr: int, w_max, w_lower, dtype):
        self.corr = corr
        self.U = {nu: u_matrix(coupling, ir_out, nu) for nu in range(1, corr + 1)}
        Um = self.U[corr]
        self.prefix = Um.shape[:-2]
        self.I, self.K = Um.shape[-2], Um.shape[-1]
        P = int(np.prod(self.prefix))
        U3 = Um.reshape(P, self.I, self.K)
        i_r, k_r = np.nonzero(np.abs(U3).max(axis=0) > 1e-12)
        self.i_r = torch.as_tensor(i_r)
        self.k_r = torch.as_tensor(k_r)
        self.u_rows = torch.as_tensor(U3[:, i_r, k_r].T.copy(), dtype=dtype)  # (nrow, P)
        self.P = P
        self.lower = []
        for idx, nu in enumerate(range(corr - 1, 0, -1)):
            Ul = self.U[nu]
            pshape = Ul.shape[:-1]
            self.lower.append((torch.as_tensor(Ul.reshape(-1, Ul.shape[-1]).T.copy(), dtype=dtype),
                               int(np.prod(pshape)), pshape[-1]))
        # orders whose U is identically zero get zero weights
        # (symmetric_contraction.py:255-262)
        if not np.any(np.abs(self.U[corr]) > 1e-15):
            w_max = torch.zeros_like(w_max)
        w_lower = [torch.zeros_like(W) if not np.any(np.abs(self.U[nu]) > 1e-15) else W
                   for W, nu in zip(w_lower, range(corr - 1, 0, -1))]
        self.w_max = w_max            # (n_el, K, C)
        self.w_lower = w_lower        # list of (n_el, k, C)
        self.out_dim = ir_out.dim

    def __call__(self, f, species):
        b, C, I = f.shape
        Wm = self.w_max[species].transpose(1, 2)                    # (b, C, K)
        X = f[:, :, self.i_r] * Wm[:, :, self.k_r]                   # (b, C, nrow)
        out = X @ self.u_rows                                        # (b, C, P)
        for (Ut, psize, idim), W in zip(self.lower, self.w_lower):
            Wl = W[species].transpose(1, 2)                          # (b, C, k)
            c = Wl @ Ut + out                                        # (b, C, psize)
            out = (c.reshape(b, C, psize // idim, idim) @ f[..., None]).reshape(b, C, psize // idim)
        return out.reshape(b, -1)


class SymmetricContraction:
    def __init__(self, irreps_in: Irreps, irreps_out: Irreps, corr, weights_fn, dtype):
        self.ii = irreps_in
        coupling = Irreps([(1, b.ir) for b in irreps_in])
        self.C = irreps_in.count("0e")
        self.contr = []
        for ci, b in enumerate(Irreps(irreps_out)):
            wm, wl = weights_fn(ci)
            self.contr.append(Contraction(coupling, b.ir, corr, wm, wl, dtype))

    def __call__(self, x, species):
        B = x.shape[0]
        blocks = []
        for b, off in zip(self.ii, self.ii.offsets):
            blocks.append(x[:, off:off + b.dim].reshape(B, b.mul, b.ir.dim))
        f = torch.cat(blocks, dim=-1)                                # (B, C, 16)
        return torch.cat([c(f, species) for c in self.contr], dim=-1)


def _silu(x):
    return x * torch.sigmoid(x)


class RadialMLP:
    def __init__(self, mats: List[torch.Tensor]):
        self.mats = mats              # nn.Linear layout (out, in)

    def __call__(self, x):
        for n, W in enumerate(self.mats):
            x = x @ W.T
            if n < len(self.mats) - 1:
                x = _silu(x)
        return x


def layer_norm(x, w, b, eps=1e-5):
    """MLX nn.LayerNorm over the last axis: (x - mean) / sqrt(var + eps) * w + b with the
    population variance."""
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * w + b


class RadialMLPLN:
    """`make_radial_mlp_with_layernorm` (`radial.py:344-357`): Linear(bias) -> LayerNorm ->
    SiLU -> ... -> Linear(bias); ``layers.{k}`` with Linear at k = 0, 3, 6, ... and
    LayerNorm at k = 1, 4, 7, ..."""

    def __init__(self, W, prefix):
        self.lin, self.ln = [], []
        k = 0
        while f"{prefix}.layers.{3 * k}.weight" in W:
            self.lin.append((W[f"{prefix}.layers.{3 * k}.weight"], W[f"{prefix}.layers.{3 * k}.bias"]))
            if f"{prefix}.layers.{3 * k + 1}.weight" in W:
                self.ln.append((W[f"{prefix}.layers.{3 * k + 1}.weight"], W[f"{prefix}.layers.{3 * k + 1}.bias"]))
            k += 1
        assert len(self.ln) == len(self.lin) - 1

    def __call__(self, x):
        for n, (Wl, bl) in enumerate(self.lin):
            x = x @ Wl.T + bl
            if n < len(self.lin) - 1:
                x = _silu(layer_norm(x, *self.ln[n]))
        return x


class Gate:
    """`gate.py:19-164` as the non-linear block builds it (`blocks.py:700-733`): input
    [scalars | gate scalars | gated blocks]; output [c_silu silu(scalars) | c_sig
    sigmoid(gate_k) x gated block k]."""

    def __init__(self, irreps_out: Irreps):
        self.scal = Irreps([b for b in irreps_out if b.ir.l == 0])
        self.gated = Irreps([b for b in irreps_out if b.ir.l > 0])
        self.ngate = sum(b.mul for b in self.gated)

    def __call__(self, x):
        ds = self.scal.dim
        out = [SILU_NORM_FACTOR * _silu(x[:, :ds])]
        gates = SIGMOID_NORM_FACTOR * torch.sigmoid(x[:, ds:ds + self.ngate])
        off, go = ds + self.ngate, 0
        for b in self.gated:
            blk = x[:, off:off + b.dim].reshape(-1, b.mul, b.ir.dim)
            out.append((gates[:, go:go + b.mul, None] * blk).reshape(x.shape[0], -1))
            off += b.dim
            go += b.mul
        return torch.cat(out, dim=-1)


# ---------------------------------------------------------------------------
# Whole model
# ---------------------------------------------------------------------------


class OracleMACE:
    """Energy model; ``dtype`` torch.float64 for parity, float32 for timing."""

    def __init__(self, model_dir=None, cfg: Optional[ModelConfig] = None,
                 weights: Optional[Dict[str, np.ndarray]] = None,
                 dtype=torch.float64, edge_chunk: int = 8192, head: Optional[str] = None,
                 gemm_tp: bool = False, recompute: bool = True):
        if model_dir is not None:
            cfg = load_config(model_dir)
            weights = load_weights(model_dir)
        cfg.check_supported()
        # active head (`calculators.py:128-137`): named, else the first
        self.H = len(cfg.heads) if cfg.heads else 1
        self.h = 0
        if self.H > 1:
            name = cfg.heads[0] if head is None else head
            if name not in cfg.heads:
                raise ValueError(f"Head '{name}' not found in model heads: {cfg.heads}")
            self.h = cfg.heads.index(name)
        self.cfg, self.dtype, self.edge_chunk = cfg, dtype, edge_chunk
        self.gemm_tp = gemm_tp
        # recompute: edge chunks re-run in the backward (bounded memory, for parity runs);
        # off for the CPU baseline, which keeps every activation as the reference's CPU path does
        self.recompute = recompute
        W = {k: _t(v, dtype) for k, v in weights.items()}
        self.W = W
        nel = cfg.num_elements
        self.nel = nel
        self.z_table = torch.as_tensor(cfg.z_table if cfg.z_table else list(range(nel)))
        C = cfg.num_features
        sh = Irreps.spherical_harmonics(cfg.max_ell)
        inter = Irreps([(C, b.ir) for b in sh])
        hidden = Irreps(cfg.hidden_irreps)
        scal = Irreps([b for b in hidden if b.ir.l == 0])
        hid_layers = [hidden if i < cfg.num_interactions - 1 else scal
                      for i in range(cfg.num_interactions)]

        def wl(prefix):
            out, n = [], 0
            while f"{prefix}.{n}" in W:
                out.append(W[f"{prefix}.{n}"])
                n += 1
            return out

        self.embed = Linear(Irreps(f"{nel}x0e"), scal, wl("node_embedding.linear.weights"))
        self.layers = []
        irr_in = scal
        edges = cfg.edge_irreps_per_layer()
        for li in range(cfg.num_interactions):
            p = f"interactions.{li}"
            hid = hid_layers[li]
            if cfg.nonlinear:
                self.layers.append(self._nonlinear_layer(li, irr_in, hid, edges[li], inter, sh, wl))
                irr_in = hid
                continue
            L = {"resid": cfg.residual(li)}
            if L["resid"]:
                L["skip"] = SkipFCTP(irr_in, nel, hid, wl(f"{p}.skip_tp.tp.weights"))
            else:
                L["skip"] = SkipFCTP(inter, nel, inter, wl(f"{p}.skip_tp.tp.weights"))
            if cfg.use_density_normalization:
                L["dens"] = W[f"{p}.density_fn.weight"]
            L["up"] = Linear(irr_in, irr_in, wl(f"{p}.linear_up.weights"))
            L["tp"] = (ConvTPGemm if gemm_tp else ConvTP)(irr_in, sh, inter)
            mats, n = [], 0
            while f"{p}.conv_tp_weights.layers.{2 * n}.weight" in W:
                mats.append(W[f"{p}.conv_tp_weights.layers.{2 * n}.weight"])
                n += 1
            assert mats[-1].shape[0] == L["tp"].weight_numel
            L["mlp"] = RadialMLP(mats)
            L["lin"] = Linear(L["tp"].mid, inter, wl(f"{p}.linear.weights"))
            q = f"products.{li}.symmetric_contractions.contractions"

            def wfn(ci, q=q):
                return W[f"{q}.{ci}.weights_max"], wl(f"{q}.{ci}.weights")

            L["sc"] = SymmetricContraction(inter, hid, cfg.correlation[li], wfn, dtype)
            L["plin"] = Linear(hid, hid, wl(f"products.{li}.linear.weights"))
            r = f"readouts.{li}"
            ro_out = Irreps(f"{self.H}x0e")   # model.py:135-139
            if li < cfg.num_interactions - 1:
                L["ro"] = ("linear", Linear(hid, ro_out, wl(f"{r}.linear.weights")))
            else:
                mlp = Irreps(f"{16 * self.H}x0e")
                L["ro"] = ("nonlinear", Linear(hid, mlp, wl(f"{r}.linear_1.weights")),
                           Linear(mlp, ro_out, wl(f"{r}.linear_2.weights")))
            self.layers.append(L)
            irr_in = hid
        self.sh_lmax = cfg.max_ell
        # (num_heads, num_elements) for multi-head models; x @ ae.T, then the active column
        # (blocks.py:45-65, model.py:316-326)
        self.e0 = W["atomic_energies_fn.atomic_energies"].reshape(self.H, -1)[self.h]
        ss = cfg.model_type == "ScaleShiftMACE"

        def per_head(v):   # ScaleShiftMACE.scale_val / shift_val, model.py:530-548
            if isinstance(v, (list, tuple)):
                return float(v[self.h] if self.h < len(v) else v[0])
            return float(v)
        self.scale = per_head(cfg.scale) if ss else None
        self.shift = per_head(cfg.shift) if ss else 0.0
        self.bw = W["radial_embedding.bessel_fn.bessel_weights"]
        self.agnesi = cfg.agnesi()
        self.radii = _t(cfg.agnesi_radii(), dtype)

    def _product_readout(self, L, li, hid, inter, wl):
        cfg, W = self.cfg, self.W
        q = f"products.{li}.symmetric_contractions.contractions"

        def wfn(ci, q=q):
            return W[f"{q}.{ci}.weights_max"], wl(f"{q}.{ci}.weights")

        L["sc"] = SymmetricContraction(inter, hid, cfg.correlation[li], wfn, self.dtype)
        L["plin"] = Linear(hid, hid, wl(f"products.{li}.linear.weights"))
        r = f"readouts.{li}"
        ro_out = Irreps(f"{self.H}x0e")   # model.py:135-139
        if li < cfg.num_interactions - 1:
            L["ro"] = ("linear", Linear(hid, ro_out, wl(f"{r}.linear.weights")))
        else:
            mlp = Irreps(f"{16 * self.H}x0e")
            L["ro"] = ("nonlinear", Linear(hid, mlp, wl(f"{r}.linear_1.weights")),
                       Linear(mlp, ro_out, wl(f"{r}.linear_2.weights")))

    def _nonlinear_layer(self, li, irr_in, hid, edge, inter, sh, wl):
        """`blocks.py:611-733` with the element-agnostic product option (`blocks.py:493-537`)."""
        cfg, W = self.cfg, self.W
        p = f"interactions.{li}"
        attrs = Irreps(f"{self.nel}x0e")
        nsc = Irreps(f"{irr_in.count('0e')}x0e")
        nonlin = cfg.nonlin_irreps()
        L = {"nonlin": True, "resid": True}
        L["src"] = Linear(attrs, nsc, wl(f"{p}.source_embedding.weights"))
        L["tgt"] = Linear(attrs, nsc, wl(f"{p}.target_embedding.weights"))
        L["skip"] = Linear(irr_in, hid, wl(f"{p}.skip_tp.weights"))
        L["up"] = Linear(irr_in, edge, wl(f"{p}.linear_up.weights"))
        L["tp"] = (ConvTPGemm if self.gemm_tp else ConvTP)(edge, sh, inter)
        L["mlp"] = RadialMLPLN(W, f"{p}.conv_tp_weights")
        assert L["mlp"].lin[-1][0].shape[0] == L["tp"].weight_numel
        L["dens"] = RadialMLPLN(W, f"{p}.density_fn")
        L["alpha"], L["beta"] = W[f"{p}.alpha"].reshape(()), W[f"{p}.beta"].reshape(())
        L["res"] = Linear(edge, nonlin, wl(f"{p}.linear_res.weights"))
        L["lin1"] = Linear(L["tp"].mid, nonlin, wl(f"{p}.linear_1.weights"))
        L["gate"] = Gate(inter)
        L["lin2"] = Linear(inter, inter, wl(f"{p}.linear_2.weights"))
        self._product_readout(L, li, hid, inter, wl)
        return L

    def _nonlinear_message(self, L, h, onehot, Y, ef, cut, sender, receiver, N):
        """message of the non-linear block (`blocks.py:735-807`)."""
        dtype = self.dtype
        up = L["up"](h)
        res = L["res"](up)
        src, tgt = L["src"](onehot), L["tgt"](onehot)
        D = L["tp"].mid.dim
        E = Y.shape[0]
        M = torch.zeros(N, D, dtype=dtype)
        rho = torch.zeros(N, dtype=dtype)
        if E == 0:
            M = M + 0.0 * up.sum()

        def chunk_fn(up_, Y_, ef_, cut_, s_, r_, accM, accR):
            aug = torch.cat([ef_, src[s_], tgt[r_]], dim=-1)
            w = L["mlp"](aug)
            d = torch.tanh(L["dens"](aug) ** 2)
            if cut_ is not None:
                w = w * cut_
                d = d * cut_
            m = L["tp"](up_[s_], Y_, w)
            return accM.index_add(0, r_, m), accR.index_add(0, r_, d[:, 0])

        for a in range(0, E, self.edge_chunk):
            b = min(E, a + self.edge_chunk)
            args = (up, Y[a:b], ef[a:b], None if cut is None else cut[a:b], sender[a:b], receiver[a:b], M, rho)
            M, rho = checkpoint(chunk_fn, *args, use_reentrant=False) if self.recompute else chunk_fn(*args)
        msg = L["lin1"](M) / (rho * L["beta"] + L["alpha"])[:, None] + res
        return L["lin2"](L["gate"](msg))

    # -- forward from edge vectors ------------------------------------------
    def energy_from_vectors(self, vec, species, sender, receiver):
        cfg, dtype = self.cfg, self.dtype
        N = species.shape[0]
        sq = (vec * vec).sum(-1)
        r = torch.sqrt(torch.clamp(sq, min=1e-24))
        onehot = torch.nn.functional.one_hot(species, self.nel).to(dtype)
        node_e0 = self.e0[species]
        Y = spherical_harmonics(vec, self.sh_lmax)
        if self.agnesi is not None:
            z = self.z_table[species]
            rb = agnesi(r, z[sender], z[receiver], self.agnesi, self.radii)
        else:
            rb = r
        env = poly_envelope(r / cfg.r_max, cfg.num_polynomial_cutoff)[:, None]
        if cfg.apply_cutoff:
            ef, cut = bessel(rb, self.bw, cfg.r_max) * env, None
        else:  # radial.py:316-318: basis and cutoff returned separately
            ef, cut = bessel(rb, self.bw, cfg.r_max), env
        terms = [node_e0]
        if cfg.pair_repulsion:
            z = self.z_table[species]
            terms.append(zbl_node_energy(r, z[sender], z[receiver], receiver, N, cfg.pair_repulsion))
        h = self.embed(onehot).detach()
        for L in self.layers:
            if L.get("nonlin"):
                sc = L["skip"](h)
                msg = self._nonlinear_message(L, h, onehot, Y, ef, cut, sender, receiver, N)
                sp = torch.zeros_like(species) if cfg.use_agnostic_product else species
                h = L["plin"](L["sc"](msg, sp)) + sc
                terms.append(self._readout(L, h))
                continue
            sc = L["skip"](h, onehot) if L["resid"] else None
            up = L["up"](h)
            msg = self._message(L, up, Y, ef, sender, receiver, N)
            msg = L["lin"](msg)
            if "dens" in L:   # density normalisation, blocks.py:372-380
                d = torch.tanh((ef @ L["dens"].T) ** 2)[:, 0]
                rho = torch.zeros(N, dtype=dtype).index_add(0, receiver, d)
                msg = msg / (rho + 1.0)[:, None]
            else:
                msg = msg / cfg.avg_num_neighbors
            if not L["resid"]:
                msg = L["skip"](msg, onehot)
            h = L["plin"](L["sc"](msg, species))
            if sc is not None:
                h = h + sc
            terms.append(self._readout(L, h))
        if self.scale is not None:
            # ScaleShiftMACE (model.py:550-589): pair + readouts scaled, shift per atom
            inter = torch.stack(terms[1:], 0).sum(0)
            terms = [terms[0], self.scale * inter + self.shift]
        node_energy = torch.stack(terms, 0).sum(0)
        return node_energy.sum(), node_energy

    def _readout(self, L, h):
        ro = L["ro"]
        if ro[0] == "linear":
            return ro[1](h)[:, self.h]
        g = _silu(ro[1](h))
        if self.H > 1:   # keep the active head's 16 features (blocks.py:583-608)
            mask = torch.zeros(g.shape[1], dtype=g.dtype)
            mask[16 * self.h:16 * (self.h + 1)] = 1.0
            g = g * mask
        return ro[2](g)[:, self.h]

    def _message(self, L, up, Y, ef, sender, receiver, N):
        E = Y.shape[0]
        D = L["tp"].mid.dim
        out = torch.zeros(N, D, dtype=self.dtype)
        if E == 0:
            return out + 0.0 * up.sum()

        def chunk_fn(up_, Y_, ef_, s_, r_, acc):
            w = L["mlp"](ef_)
            m = L["tp"](up_[s_], Y_, w)
            return acc.index_add(0, r_, m)

        for a in range(0, E, self.edge_chunk):
            b = min(E, a + self.edge_chunk)
            args = (up, Y[a:b], ef[a:b], sender[a:b], receiver[a:b], out)
            out = checkpoint(chunk_fn, *args, use_reentrant=False) if self.recompute else chunk_fn(*args)
        return out

    # -- public entry points -------------------------------------------------
    def _inputs(self, positions, species, edge_index, shifts, cell):
        dt = self.dtype
        pos = torch.as_tensor(np.asarray(positions, np.float64), dtype=dt)
        sp = torch.as_tensor(np.asarray(species, np.int64))
        ei = torch.as_tensor(np.asarray(edge_index, np.int64))
        S = torch.as_tensor(np.asarray(shifts, np.float64), dtype=dt)
        cl = torch.as_tensor(np.asarray(cell, np.float64), dtype=dt)
        return pos, sp, ei[0], ei[1], S, cl

    def energy(self, positions, species, edge_index, shifts, cell):
        pos, sp, s, r, S, cl = self._inputs(positions, species, edge_index, shifts, cell)
        with torch.no_grad():
            vec = pos[r] - pos[s] + S @ cl
            E, ne = self.energy_from_vectors(vec, sp, s, r)
        return float(E), ne.numpy()

    def energy_forces(self, positions, species, edge_index, shifts, cell):
        pos, sp, s, r, S, cl = self._inputs(positions, species, edge_index, shifts, cell)
        pos.requires_grad_(True)
        vec = pos[r] - pos[s] + S @ cl
        E, ne = self.energy_from_vectors(vec, sp, s, r)
        if not E.requires_grad:   # no edges: the energy does not depend on positions
            return float(E), np.zeros(pos.shape), ne.detach().numpy()
        (g,) = torch.autograd.grad(E, pos)
        return float(E.detach()), (-g).numpy(), ne.detach().numpy()

    def energy_forces_stress(self, positions, species, edge_index, shifts, cell):
        """`calculators.py:482-563`: symmetric displacement, stress = dE/d(eps)/V
        in Voigt order xx, yy, zz, yz, xz, xy."""
        pos, sp, s, r, S, cl = self._inputs(positions, species, edge_index, shifts, cell)
        pos.requires_grad_(True)
        disp = torch.zeros(3, 3, dtype=self.dtype, requires_grad=True)
        sym = 0.5 * (disp + disp.T)
        ps = pos + pos @ sym
        cs = cl + cl @ sym
        vec = ps[r] - ps[s] + S @ cs
        E, ne = self.energy_from_vectors(vec, sp, s, r)
        if not E.requires_grad:
            gp, gd = torch.zeros_like(pos), torch.zeros(3, 3, dtype=self.dtype)
        else:
            gp, gd = torch.autograd.grad(E, (pos, disp), allow_unused=True)
            gd = torch.zeros(3, 3, dtype=self.dtype) if gd is None else gd
        E = E.detach()
        vol = abs(np.linalg.det(np.asarray(cell, np.float64)))
        st = gd.detach().numpy() / vol
        voigt = st[[0, 1, 2, 1, 0, 0], [0, 1, 2, 2, 2, 1]]
        return float(E), (-gp).numpy(), voigt, ne.detach().numpy(), gd.detach().numpy()
