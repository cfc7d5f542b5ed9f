"""Float64 brute-force periodic neighbour list -- TEST INFRASTRUCTURE ONLY.

Restates what the reference obtains from matscipy / ASE ``neighbour_list("ijS")``
(`calculators.py:44-55`): all (i, j, S) with S an integer lattice translation and
``|x_j - x_i + S @ cell| < cutoff``, excluding the self pair (i == j, S == 0).
Positions may be unwrapped (outside the cell); S then absorbs the wrap.
"""

from __future__ import annotations

import numpy as np


def plane_spacings(cell: np.ndarray) -> np.ndarray:
    vol = abs(np.linalg.det(cell))
    return np.array([vol / np.linalg.norm(np.cross(cell[(k + 1) % 3], cell[(k + 2) % 3]))
                     for k in range(3)])


def neighbor_list(positions, cell, pbc, cutoff, chunk: int = 512):
    """Return (i, j, S) sorted lexicographically by (j, i, S)."""
    pos = np.asarray(positions, dtype=np.float64)
    cell = np.asarray(cell, dtype=np.float64)
    pbc = np.asarray(pbc, dtype=bool)
    n = len(pos)
    if pbc.any():
        d = plane_spacings(cell)
        frac = pos @ np.linalg.inv(cell)
        span = np.ptp(frac, axis=0) if n else np.zeros(3)
        nmax = [int(np.ceil(cutoff / d[k] + span[k])) + 1 if pbc[k] else 0 for k in range(3)]
    else:
        nmax = [0, 0, 0]
    rng = [np.arange(-m, m + 1) for m in nmax]
    shifts = np.array(np.meshgrid(*rng, indexing="ij")).reshape(3, -1).T  # (T, 3)
    sh_cart = shifts @ cell if pbc.any() else np.zeros((len(shifts), 3))
    I, J, S = [], [], []
    c2 = cutoff * cutoff
    for a0 in range(0, n, chunk):
        pi = pos[a0:a0 + chunk]                       # (c, 3)
        # D[c, j, t] = x_j - x_i + shift_t
        base = pos[None, :, :] - pi[:, None, :]       # (c, n, 3)
        for t in range(len(shifts)):
            D = base + sh_cart[t]
            r2 = np.einsum("cjk,cjk->cj", D, D)
            ii, jj = np.nonzero(r2 < c2)
            ii = ii + a0
            if not shifts[t].any():
                keep = ii != jj
                ii, jj = ii[keep], jj[keep]
            I.append(ii)
            J.append(jj)
            S.append(np.repeat(shifts[t][None, :], len(ii), axis=0))
    I = np.concatenate(I) if I else np.zeros(0, np.int64)
    J = np.concatenate(J) if J else np.zeros(0, np.int64)
    S = np.concatenate(S) if S else np.zeros((0, 3), np.int64)
    order = np.lexsort((S[:, 2], S[:, 1], S[:, 0], I, J))
    return I[order].astype(np.int64), J[order].astype(np.int64), S[order].astype(np.int64)
