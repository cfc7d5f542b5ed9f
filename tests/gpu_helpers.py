"""Shared helpers for the GPU tests: run the engine and the oracle on the same inputs."""

from __future__ import annotations

import numpy as np
import torch

from mace_mlx_amd._ffi import Engine
from mace_mlx_amd.device_model import build_device_model, round_weights
from mace_mlx_amd.model_io import random_init
from oracle.model import OracleMACE
from oracle.neighbors import neighbor_list

torch.set_num_threads(16)


def species_of(dm, numbers):
    zmap = {int(z): k for k, z in enumerate(dm.z_table)}
    return np.array([zmap[int(z)] for z in numbers], np.int32)


class Case:
    """Engine + oracle for one (model config, seed, feature dtype).  For "float16" and
    "bfloat16" the oracle evaluates the same half-precision model (weights rounded to fp16 /
    bf16 except the pinned ones) in float64, i.e. without the feature-path roundings."""

    def __init__(self, cfg, seed=0, dtype="float32", head=None):
        self.cfg, self.head = cfg, head
        self.w = random_init(cfg, seed)
        self.w_model = round_weights(self.w, dtype)
        self.dm = build_device_model(cfg, self.w, dtype=dtype, head=head)
        self.eng = Engine(0, channels=self.dm.dims["num_channels"])
        self.eng.load_model(self.dm)
        self._oracle = None

    @property
    def oracle(self):
        if self._oracle is None:
            self._oracle = OracleMACE(cfg=self.cfg, weights=self.w_model, dtype=torch.float64,
                                      head=self.head)
        return self._oracle

    def run(self, s, stress=False, skin=0.5, force_nl=False):
        sp = species_of(self.dm, s.numbers)
        self.eng.set_system(sp, s.cell, s.pbc, skin)
        E, ne, F, vir = self.eng.step(s.positions, stress=stress, force_nl=force_nl)
        return dict(E=E, ne=ne, F=F, vir=vir, sp=sp)

    def edges(self):
        return self.eng.get_edges()

    def reference(self, s, sp, edges, stress=False):
        snd, rcv, sh = edges
        ei = np.stack([snd, rcv]).astype(np.int64)
        if stress:
            E, F, st, ne, vir = self.oracle.energy_forces_stress(s.positions, sp, ei, sh, s.cell)
            return dict(E=E, F=F, ne=ne, vir=vir)
        E, F, ne = self.oracle.energy_forces(s.positions, sp, ei, sh, s.cell)
        return dict(E=E, F=F, ne=ne)


def edge_set(s, r, S):
    return set(zip(np.asarray(s).tolist(), np.asarray(r).tolist(), map(tuple, np.asarray(S).tolist())))


def bruteforce_edges(s, cutoff=6.5):
    i, j, S = neighbor_list(s.positions, s.cell, s.pbc, cutoff)
    return edge_set(i, j, S)


def assert_parity(got, ref, n_atoms, stress=False, vol=None, energy="relative"):
    """north_star tolerances: energy |dE|/|E| <= 1e-6 (energy="relative", the default),
    or, named by the cases whose per-atom energies cancel, |dE|/N <= 1e-6 eV/atom
    (energy="per_atom": the random-init large architecture sums to |E| = 7.4 eV over
    216 atoms, where a float32 restatement of the reference itself differs from float64
    by 1.1e-5 eV, i.e. 1.5e-6 relative); forces max-abs 1e-4 eV/A; node energies 1e-5
    relative to the largest; virial 1e-5 relative.  Both energy measures are printed."""
    dE = abs(got["E"] - ref["E"])
    rel = dE / abs(ref["E"]) if ref["E"] != 0 else dE
    per_atom = dE / max(n_atoms, 1)
    print(f"parity: |dE|={dE:.3e} eV  |dE|/|E|={rel:.3e}  |dE|/N={per_atom:.3e} eV/atom", flush=True)
    if energy == "relative":
        assert dE <= 1e-6 * abs(ref["E"]), (got["E"], ref["E"], dE, rel)
    elif energy == "per_atom":
        assert per_atom <= 1e-6, (got["E"], ref["E"], dE, per_atom)
    else:
        raise ValueError(energy)
    dF = float(np.abs(got["F"] - ref["F"]).max()) if n_atoms else 0.0
    print(f"parity: max|dF|={dF:.3e} eV/A (max|F| {float(np.abs(ref['F']).max()) if n_atoms else 0.0:.3g})", flush=True)
    assert dF <= 1e-4, dF
    dne = float(np.abs(got["ne"] - ref["ne"]).max()) if n_atoms else 0.0
    assert dne <= 1e-5 * max(1.0, float(np.abs(ref["ne"]).max())), dne
    if stress:
        dv = np.abs(got["vir"] - ref["vir"]).max()
        assert dv <= 1e-5 * max(1.0, np.abs(ref["vir"]).max()), (got["vir"], ref["vir"])
    return dE, dF
