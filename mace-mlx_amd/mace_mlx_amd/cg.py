"""Real Wigner-3j symbols, SH recursion couplings and symmetric-contraction U tensors.

All host-side, float64, computed once when a model is built; the HIP library only
receives the resulting tables.

Basis.  The real spherical-harmonic basis is the one the reference fixes through
its rotation generators (`clebsch_gordan.py:26-83`): the z-rotation
``Rz(a)[i,i] = cos((l-i)a)``, ``Rz(a)[i,2l-i] = sin((l-i)a)`` and the y-generator
``J = Re(U Jc U^H)`` with the complex-to-real unitary ``U`` and ladder generator
``Jc`` of `clebsch_gordan.py:26-65`.

Wigner-3j.  The reference finds the invariant tensor as the null vector of
``sum_R (D1 x D2 x D3 - I)^T (D1 x D2 x D3 - I)`` over five fixed random rotations
(`clebsch_gordan.py:191-235`).  Here the same tensor is obtained from the
infinitesimal condition instead: it is the common null vector of
``G x 1 x 1 + 1 x G x 1 + 1 x 1 x G`` for the two generators ``G = Gz, J``.  The
null space is one-dimensional, so both constructions give the same unit tensor up
to sign; the sign and the derivation of unsorted triples from sorted ones then
follow the reference's convention exactly (`clebsch_gordan.py:220-272`), because
that convention is part of the model definition.

U tensors.  ``U_matrix_real`` restates the coupling recursion of
`clebsch_gordan.py:296-445` (path order matters: it fixes which weight index
multiplies which coupling path).
"""

from __future__ import annotations

import functools
import math
from typing import Dict, List, Sequence, Tuple

import numpy as np

from .irreps import Irrep, Irreps

# ---------------------------------------------------------------------------
# Real-basis rotation generators
# ---------------------------------------------------------------------------


@functools.lru_cache(maxsize=None)
def _complex_to_real(l: int) -> np.ndarray:
    """Unitary map complex -> real SH of degree l (Condon-Shortley phase),
    the basis definition of `clebsch_gordan.py:27-45`."""
    d = 2 * l + 1
    U = np.zeros((d, d), dtype=np.complex128)
    s = 1.0 / math.sqrt(2.0)
    for m in range(-l, l + 1):
        r = l + m
        if m > 0:
            U[r, l + m] = (-1) ** m * s
            U[r, l - m] = s
        elif m == 0:
            U[r, l] = 1.0
        else:
            U[r, l - m] = -1j * (-1) ** (-m) * s
            U[r, l + m] = 1j * s
    return U


@functools.lru_cache(maxsize=None)
def generator_y(l: int) -> np.ndarray:
    """Real antisymmetric generator of y-rotations (``exp(b*J)`` rotates by b)."""
    d = 2 * l + 1
    Jc = np.zeros((d, d))
    for m in range(-l, l + 1):
        if m + 1 <= l:
            Jc[m + l + 1, m + l] = 0.5 * math.sqrt(l * (l + 1) - m * (m + 1))
        if m - 1 >= -l:
            Jc[m + l - 1, m + l] = -0.5 * math.sqrt(l * (l + 1) - m * (m - 1))
    U = _complex_to_real(l)
    J = U @ Jc @ U.conj().T
    assert np.abs(J.imag).max() < 1e-12
    return np.ascontiguousarray(J.real)


@functools.lru_cache(maxsize=None)
def generator_z(l: int) -> np.ndarray:
    """Derivative at 0 of the real z-rotation of degree l."""
    d = 2 * l + 1
    G = np.zeros((d, d))
    for i in range(d):
        if i != d - 1 - i:
            G[i, d - 1 - i] = float(l - i)
    return G


def rot_z(l: int, a: float) -> np.ndarray:
    d = 2 * l + 1
    M = np.zeros((d, d))
    for i in range(d):
        f = float(l - i)
        M[i, d - 1 - i] = math.sin(f * a)
    for i in range(d):
        M[i, i] = math.cos(float(l - i) * a)
    return M


def wigner_D(l: int, alpha: float, beta: float, gamma: float) -> np.ndarray:
    """Real Wigner D in the reference basis: Rz(alpha) exp(beta J) Rz(gamma)."""
    J = generator_y(l)
    # exp of a real antisymmetric matrix through its eigen-decomposition of iJ
    w, V = np.linalg.eigh(1j * J)
    E = (V * np.exp(-1j * beta * w)) @ V.conj().T
    return rot_z(l, alpha) @ E.real @ rot_z(l, gamma)


# ---------------------------------------------------------------------------
# Wigner 3j
# ---------------------------------------------------------------------------


def _triangle(l1: int, l2: int, l3: int) -> bool:
    return abs(l1 - l2) <= l3 <= l1 + l2


@functools.lru_cache(maxsize=None)
def _w3j_sorted(l1: int, l2: int, l3: int) -> np.ndarray:
    d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
    n = d1 * d2 * d3
    I1, I2, I3 = np.eye(d1), np.eye(d2), np.eye(d3)
    rows = []
    for gen in (generator_z, generator_y):
        A = (np.kron(np.kron(gen(l1), I2), I3)
             + np.kron(np.kron(I1, gen(l2)), I3)
             + np.kron(np.kron(I1, I2), gen(l3)))
        rows.append(A)
    A = np.concatenate(rows, axis=0)
    w, V = np.linalg.eigh(A.T @ A)
    if not (w[0] < 1e-9 and (n == 1 or w[1] > 1e-6)):
        raise RuntimeError(f"3j null space for ({l1},{l2},{l3}) is not one-dimensional: {w[:3]}")
    q = V[:, 0].reshape(d1, d2, d3)
    q = q / np.linalg.norm(q)
    q[np.abs(q) < 1e-14] = 0.0
    # sign convention of clebsch_gordan.py:223-233
    c = q[l1, l2, l3]
    if c != 0.0:
        if c < 0:
            q = -q
    else:
        first = q.ravel()[np.flatnonzero(q.ravel())[0]]
        if first < 0:
            q = -q
    return q


@functools.lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    """Unit-norm real 3j tensor of shape (2l1+1, 2l2+1, 2l3+1) (e3nn convention);
    unsorted triples come from the sorted one by the transposition rules of
    `clebsch_gordan.py:238-272`."""
    if not _triangle(l1, l2, l3):
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    s = (-1) ** (l1 + l2 + l3)
    if l1 <= l2 <= l3:
        return _w3j_sorted(l1, l2, l3).copy()
    if l1 <= l3 <= l2:
        return np.ascontiguousarray(_w3j_sorted(l1, l3, l2).transpose(0, 2, 1) * s)
    if l2 <= l1 <= l3:
        return np.ascontiguousarray(_w3j_sorted(l2, l1, l3).transpose(1, 0, 2) * s)
    if l3 <= l2 <= l1:
        return np.ascontiguousarray(_w3j_sorted(l3, l2, l1).transpose(2, 1, 0) * s)
    if l2 <= l3 <= l1:
        return np.ascontiguousarray(_w3j_sorted(l2, l3, l1).transpose(2, 0, 1))
    # l3 <= l1 <= l2
    return np.ascontiguousarray(_w3j_sorted(l3, l1, l2).transpose(1, 2, 0))


def so3_cg(l1: int, l2: int, l3: int) -> np.ndarray:
    """Component-normalised real CG: 3j * sqrt(2 l3 + 1)."""
    return wigner_3j(l1, l2, l3) * math.sqrt(2 * l3 + 1)


@functools.lru_cache(maxsize=None)
def sh_coupling(l: int) -> np.ndarray:
    """Recursion tensor ``Y_l[k] = sum_ij Y_{l-1}[i] Y_1[j] C[i,j,k]``
    (`spherical_harmonics.py:31-40`): so3 CG(l-1, 1, l) * sqrt((2l+1)/(3l))."""
    return so3_cg(l - 1, 1, l) * math.sqrt((2 * l + 1) / (3 * l))


# ---------------------------------------------------------------------------
# U tensors for the symmetric contraction
# ---------------------------------------------------------------------------


def _coupling_paths(irrepss: Sequence[Irreps], keep_last: Sequence[Irrep] | None
                    ) -> List[Tuple[Irrep, np.ndarray]]:
    """Recursive n-fold coupling (`clebsch_gordan.py:296-362`, component
    normalisation).  Returns [(ir_out, C)] with C of shape
    (ir_out.dim, *[irreps.dim for irreps in irrepss]), stably sorted by (l, p)
    at every level.  ``keep_last`` drops unwanted outputs at the outermost level
    only (this changes nothing in the kept entries or their order)."""
    if len(irrepss) == 1:
        (irreps,) = irrepss
        eye = np.eye(irreps.dim)
        out = []
        off = 0
        for mul, ir in irreps:
            for _ in range(mul):
                out.append((ir, eye[off:off + ir.dim]))
                off += ir.dim
        # the single-factor level is returned in input order (no sort), as in
        # clebsch_gordan.py:310-320
        if keep_last is not None:
            out = [t for t in out if t[0] in keep_last]
        return out
    *left_list, right = irrepss
    left_dims = tuple(x.dim for x in left_list)
    out = []
    for ir_left, C_left in _coupling_paths(left_list, None):
        off = 0
        for mul, ir in right:
            for ir_out in ir_left.couple(ir):
                if keep_last is not None and ir_out not in keep_last:
                    continue
                w = wigner_3j(ir_out.l, ir_left.l, ir.l) * math.sqrt(ir_out.dim)
                C = np.einsum("jk,ijl->ikl", C_left.reshape(ir_left.dim, -1), w)
                C = C.reshape(ir_out.dim, *left_dims, ir.dim)
                for u in range(mul):
                    E = np.zeros((ir_out.dim, *left_dims, right.dim))
                    E[..., off + u * ir.dim: off + (u + 1) * ir.dim] = C
                    out.append((ir_out, E))
            off += mul * ir.dim
    return sorted(out, key=lambda t: t[0].sort_key())


@functools.lru_cache(maxsize=None)
def _u_matrix_cached(irreps_in: str, ir_out: str, correlation: int) -> np.ndarray:
    irreps = Irreps(irreps_in)
    target = Irrep.parse(ir_out)
    paths = _coupling_paths([irreps] * correlation, [target])
    if not paths:
        shape = ((target.dim,) if target.dim != 1 else ()) + (irreps.dim,) * correlation + (1,)
        return np.zeros(shape)
    pieces = [np.squeeze(C)[..., None] for _, C in paths]
    return np.concatenate(pieces, axis=-1)


def u_matrix(irreps_in: Irreps | str, ir_out: Irrep | str, correlation: int) -> np.ndarray:
    """U tensor of `clebsch_gordan.py:365-445` for a single output irrep.

    Shape (*[irreps_in.dim]*correlation, n_paths) for a scalar output, else
    (ir_out.dim, *[irreps_in.dim]*correlation, n_paths).  Read-only copy."""
    U = _u_matrix_cached(str(Irreps(irreps_in)), str(Irrep.parse(ir_out)), int(correlation))
    U = U.copy()
    U.setflags(write=False)
    return U
