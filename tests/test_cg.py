"""Coupling constants: golden vectors from the reference + mathematical invariants.

Golden vectors: tests/golden/cg_fixtures.npz, written by tests/golden/make_cg_fixtures.py
from the reference's `clebsch_gordan.py` (wigner_3j 238-272, _wigner_D_real 80-83,
U_matrix_real 365-445).  Invariants restate `tests/test_cg.py:65-191` of the reference.
"""

import itertools
import math
from pathlib import Path

import numpy as np
import pytest

from mace_mlx_amd import cg

FIX = np.load(Path(__file__).parent / "golden" / "cg_fixtures.npz")


def _triples(lmax=3):
    for l1 in range(lmax + 1):
        for l2 in range(lmax + 1):
            for l3 in range(abs(l1 - l2), min(l1 + l2, lmax) + 1):
                yield l1, l2, l3


@pytest.mark.parametrize("l1,l2,l3", list(_triples()))
def test_w3j_matches_reference(l1, l2, l3):
    np.testing.assert_allclose(cg.wigner_3j(l1, l2, l3), FIX[f"w3j_{l1}{l2}{l3}"], atol=1e-12)


@pytest.mark.parametrize("l", range(4))
@pytest.mark.parametrize("k", range(3))
def test_wigner_D_matches_reference(l, k):
    a, b, c = FIX["angles"][k]
    np.testing.assert_allclose(cg.wigner_D(l, a, b, c), FIX[f"D_{l}_{k}"], atol=1e-12)


U_CASES = [("0e+1o+2e+3o", "0e"), ("0e+1o+2e+3o", "1o"), ("0e+1o+2e+3o", "2e"),
           ("0e+1o+2e", "0e"), ("0e+1o", "0e"), ("0e+1o", "1o")]


@pytest.mark.parametrize("irreps,out", U_CASES)
@pytest.mark.parametrize("nu", [1, 2, 3])
def test_u_matrix_matches_reference(irreps, out, nu):
    key = f"U_{irreps.replace('+', '_')}_{out}_{nu}"
    ref = np.zeros(tuple(FIX[key + "_shape"]))
    ref[tuple(FIX[key + "_idx"].astype(np.int64).T)] = FIX[key + "_val"]
    U = cg.u_matrix(irreps, out, nu)
    assert U.shape == ref.shape
    np.testing.assert_allclose(U, ref, atol=1e-12)


@pytest.mark.parametrize("l1,l2,l3", list(_triples(4)))
def test_w3j_unit_norm_and_sign_rule(l1, l2, l3):
    w = cg.wigner_3j(l1, l2, l3)
    assert abs((w ** 2).sum() - 1.0) < 1e-12
    if l1 <= l2 <= l3:  # sign convention applies to the sorted base case
        c = w[l1, l2, l3]
        first = w.ravel()[np.flatnonzero(np.abs(w.ravel()) > 1e-14)[0]]
        assert (c > 0) if abs(c) > 1e-14 else (first > 0)


@pytest.mark.parametrize("l1,l2,l3", list(_triples()))
def test_w3j_equivariance(l1, l2, l3):
    rng = np.random.default_rng(7)
    a, b, c = rng.uniform(0, 2 * np.pi, 3)
    D1, D2, D3 = (cg.wigner_D(l, a, b, c) for l in (l1, l2, l3))
    w = cg.wigner_3j(l1, l2, l3)
    rot = np.einsum("il,jm,kn,lmn->ijk", D1, D2, D3, w)
    np.testing.assert_allclose(rot, w, atol=1e-10)


@pytest.mark.parametrize("l1,l2", list(itertools.product(range(4), range(4))))
def test_cg_completeness(l1, l2):
    """sum_{l3, m3} C[m1,m2,m3] C[m1',m2',m3] = delta delta (test_cg.py:90-111)."""
    d1, d2 = 2 * l1 + 1, 2 * l2 + 1
    acc = np.zeros((d1, d2, d1, d2))
    for l3 in range(abs(l1 - l2), l1 + l2 + 1):
        w = cg.wigner_3j(l1, l2, l3) * math.sqrt(2 * l3 + 1)
        acc += np.einsum("abk,cdk->abcd", w, w)
    np.testing.assert_allclose(acc.reshape(d1 * d2, -1), np.eye(d1 * d2), atol=1e-10)


def test_wigner_D_is_representation():
    rng = np.random.default_rng(3)
    for l in range(4):
        D = cg.wigner_D(l, *rng.uniform(0, 6, 3))
        np.testing.assert_allclose(D @ D.T, np.eye(2 * l + 1), atol=1e-12)
    # l = 1 acts on SH l=1 = sqrt(3)(x, y, z) like a rotation matrix in some basis order
    D1 = cg.wigner_D(1, 0.3, 1.1, -0.7)
    assert abs(np.linalg.det(D1) - 1.0) < 1e-12


def test_u_matrix_symmetric_in_feature_indices():
    """U for correlation 2 contracts a symmetric pair of identical features."""
    U = cg.u_matrix("0e+1o+2e+3o", "0e", 2)
    # symmetrising over (i1, i2) must not annihilate any path
    sym = U + U.transpose(1, 0, 2)
    assert np.all(np.abs(sym).reshape(-1, U.shape[-1]).max(axis=0) > 1e-8)
