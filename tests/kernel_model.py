"""Float64 CPU re-evaluation of the engine's *kernel-level* formulation (test helper).

Uses exactly what the HIP kernels consume -- the tensors of
``mace_mlx_amd.device_model`` (folded path weights, component-major block
layouts), the conv-TP slot layout and the symmetrised symmetric-contraction
polynomial terms emitted by ``csrc/gen_tables.py`` -- so that comparing it with
the oracle checks the host-side folding and the generated tables independently
of the GPU.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "mace-mlx_amd" / "csrc"))

import gen_tables  # noqa: E402
from mace_mlx_amd.cg import sh_coupling, wigner_3j  # noqa: E402
from mace_mlx_amd.model_io import COVALENT_RADII  # noqa: E402


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _env(u, p):
    pf = float(p)
    up = u ** p
    e = 1 - (pf + 1) * (pf + 2) / 2 * up + pf * (pf + 2) * up * u - pf * (pf + 1) / 2 * up * u * u
    return e * (u < 1.0)


def sh(vec):
    r = np.sqrt(np.maximum((vec * vec).sum(-1, keepdims=True), 1e-24))
    u = vec / r
    Y1 = math.sqrt(3.0) * u
    Y2 = np.einsum("ei,ej,ijk->ek", Y1, Y1, sh_coupling(2))
    Y3 = np.einsum("ei,ej,ijk->ek", Y2, Y1, sh_coupling(3))
    return np.concatenate([np.ones_like(u[:, :1]), Y1, Y2, Y3], axis=1)


def energy(dm, positions, species, sender, receiver, shifts, cell):
    T = {k: np.asarray(v, np.float64) for k, v in dm.tensors.items()}
    d = dm.dims
    N = len(species)
    C = d["num_channels"]
    vec = positions[receiver] - positions[sender] + shifts @ cell
    r = np.sqrt(np.maximum((vec * vec).sum(-1), 1e-24))
    Y = sh(vec)
    rmax = d["r_max"]
    bw = T["bessel_w"]
    ef = math.sqrt(2 / rmax) * np.sin(bw[None, :] * r[:, None]) / r[:, None] * _env(r / rmax, d["num_poly_cutoff"])[:, None]
    node_e = T["e0"][species].copy()
    if d["has_zbl"]:
        zu, zv = T["zbl_z"][species[sender]], T["zbl_z"][species[receiver]]
        a = d["zbl_a_prefactor"] * 0.529 / (zu ** d["zbl_a_exp"] + zv ** d["zbl_a_exp"])
        x = r / a
        phi = 0.1818 * np.exp(-3.2 * x) + 0.5099 * np.exp(-0.9423 * x) + 0.2802 * np.exp(-0.4028 * x) + 0.02817 * np.exp(-0.2016 * x)
        rc = T["zbl_cov"][species[sender]] + T["zbl_cov"][species[receiver]]
        ez = d["zbl_scale"] * 0.5 * 14.3996 * zu * zv / r * phi * _env(r / rc, d["zbl_p"])
        np.add.at(node_e, receiver, ez)
    h = [T["embed"][species][:, None, :]]            # blocks: (N, 2b+1, C)
    L = d["num_layers"]
    for l in range(L):
        p = f"L{l}."
        lin, lhid, corr = d["layer_in_blocks"][l], d["layer_hid_blocks"][l], d["correlation"][l]
        up = [h[b] @ T[f"{p}up.{b}"] for b in range(lin)]
        x = ef
        for k in range(4):
            x = x @ T[f"{p}mlp.{k}"]
            if k < 3:
                x = _silu(x)
        slots = gen_tables.tp_layout(lin)
        w = x.reshape(len(r), len(slots), C)
        M = []
        for s, (l1, l2, l3) in enumerate(slots):
            cg = wigner_3j(l1, l2, l3) * math.sqrt(2 * l3 + 1)
            Ys = Y[:, l2 * l2:(l2 + 1) ** 2]
            val = np.einsum("eiu,ej,ijk->eku", up[l1][sender], Ys, cg) * w[:, s, None, :]
            m = np.zeros((N, 2 * l3 + 1, C))
            np.add.at(m, receiver, val)
            M.append(m)
        A = []
        for lo in range(4):
            X = np.concatenate([M[s] for s, sl in enumerate(slots) if sl[2] == lo], axis=2)
            A.append(X @ T[f"{p}lin.{lo}"])
        f = np.concatenate(A, axis=1).transpose(0, 2, 1)  # (N, C, 16)
        hn = []
        for b in range(lhid):
            terms, ks = gen_tables.sc_poly(b, corr)
            Wsc = T[f"{p}sc.{b}"][species]                # (N, KT, C)
            out = np.zeros((N, 2 * b + 1, C))
            for (pp, mono, k), coef in terms:
                t = coef * Wsc[:, k, :]
                for i in mono:
                    t = t * f[:, :, i]
                out[:, pp, :] += t
            hb = out @ T[f"{p}plin.{b}"]
            if b < lin:
                Ws = T[f"{p}skip.{b}"][species]           # (N, C, C)
                hb = hb + np.einsum("nmu,nuw->nmw", h[b], Ws)
            hn.append(hb)
        h = hn
        if l < L - 1:
            node_e += h[0][:, 0, :] @ T[f"{p}ro"]
        else:
            y = h[0][:, 0, :] @ T[f"{p}ro1"]
            node_e += _silu(y) @ T[f"{p}ro2"]
    return node_e.sum(), node_e
