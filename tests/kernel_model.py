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


def _ln(x, sc, sh):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * sc + sh


def _tp(up, Y, w, slots, sender, receiver, N, C):
    M = []
    for s, (l1, l2, l3) in enumerate(slots):
        cg = wigner_3j(l1, l2, l3) * math.sqrt(2 * l3 + 1)
        Ys = Y[:, l2 * l2:(l2 + 1) ** 2]
        val = np.einsum("eiu,ej,ijk->eku", up[l1][sender], Ys, cg) * w[:, s, None, :]
        m = np.zeros((N, 2 * l3 + 1, C))
        np.add.at(m, receiver, val)
        M.append(m)
    return M


def _nonlinear_message(T, d, p, l, h, species, sender, receiver, ef, cut, Y, N, C):
    """The mh-1 block from the engine's tensors: LayerNorm MLPs with per-species first-layer
    tables, w = (h3 W3 + b3) cut, rho, Q = linear_1(M) / (beta rho + alpha), R = linear_res(up),
    gate, linear_2."""
    lin, ledge = d["layer_in_blocks"][l], d["layer_edge_blocks"][l]
    up = [h[b] @ T[f"{p}up.{b}"] if b < lin else np.zeros((N, 2 * b + 1, C)) for b in range(ledge)]
    zs, zr = species[sender], species[receiver]
    z = ef @ T[f"{p}rmlp.w0"] + T[f"{p}rmlp.ts"][zs] + T[f"{p}rmlp.tt"][zr]
    for k in range(3):
        a = _silu(_ln(z, *T[f"{p}rmlp.ln"][k]))
        if k < 2:
            z = a @ T[f"{p}rmlp.w{k + 1}"] + T[f"{p}rmlp.bias"][k]
    w = (a @ T[f"{p}mlp.3"] + T[f"{p}rmlp.b3"]) * cut[:, None]
    zd = ef @ T[f"{p}dmlp.w0"] + T[f"{p}dmlp.ts"][zs] + T[f"{p}dmlp.tt"][zr]
    x = _silu(_ln(zd, *T[f"{p}dmlp.ln"])) @ T[f"{p}dmlp.w1"][:64] + T[f"{p}dmlp.w1"][64]
    rho = np.zeros(N)
    np.add.at(rho, receiver, np.tanh(x * x) * cut)
    alpha, beta = T[f"{p}ab"]
    rinv = 1.0 / (beta * rho + alpha)
    slots = gen_tables.tp_layout(ledge)
    M = _tp(up, Y, w.reshape(len(ef), len(slots), C), slots, sender, receiver, N, C)
    pre = []
    for lo in range(4):
        X = np.concatenate([M[s] for s, sl in enumerate(slots) if sl[2] == lo], axis=2)
        q = X @ T[f"{p}lin.{lo}"] * rinv[:, None, None]
        if lo < ledge:
            q = q + up[lo] @ T[f"{p}res.{lo}"]
        pre.append(q)
    s0 = pre[0][:, 0, :]
    out = [1.6791768074035645 * _silu(s0[:, :C])[:, None, :]]
    for lo in (1, 2, 3):
        g = 1.8467055569904827 / (1.0 + np.exp(-s0[:, lo * C:(lo + 1) * C]))
        out.append(g[:, None, :] * pre[lo])
    return [out[lo] @ T[f"{p}lin2.{lo}"] for lo in range(4)]


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
    env = _env(r / rmax, d["num_poly_cutoff"])
    sep = bool(d.get("separate_cutoff"))
    ef = math.sqrt(2 / rmax) * np.sin(bw[None, :] * r[:, None]) / r[:, None] * (1.0 if sep else env[:, None])
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
        sp_sc = np.zeros_like(species) if d.get("agnostic_product") else species
        if d.get("nonlinear"):
            A = _nonlinear_message(T, d, p, l, h, species, sender, receiver, ef, env if sep else np.ones_like(r),
                                   Y, N, C)
            f = np.concatenate(A, axis=1).transpose(0, 2, 1)
            hn = []
            for b in range(lhid):
                terms, ks = gen_tables.sc_poly(b, corr)
                Wsc = T[f"{p}sc.{b}"][sp_sc]
                out = np.zeros((N, 2 * b + 1, C))
                for (pp, mono, k), coef in terms:
                    t = coef * Wsc[:, k, :]
                    for i in mono:
                        t = t * f[:, :, i]
                    out[:, pp, :] += t
                hb = out @ T[f"{p}plin.{b}"]
                if b < min(lin, lhid):
                    hb = hb + h[b] @ T[f"{p}skip.{b}"]
                hn.append(hb)
            h = hn
            if l < L - 1:
                node_e += h[0][:, 0, :] @ T[f"{p}ro"]
            else:
                node_e += _silu(h[0][:, 0, :] @ T[f"{p}ro1"]) @ T[f"{p}ro2"]
            continue
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
            Wsc = T[f"{p}sc.{b}"][sp_sc]                  # (N, KT, C)
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
