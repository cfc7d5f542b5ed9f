"""Callable model objects: the reference's ``load_model`` / ``MACE`` / ``ScaleShiftMACE``
(`mace_mlx/model.py:86-720`) evaluated by the HIP engine.

``load_model(model_dir, dtype)`` reads a reference-format model directory (``config.json`` +
``weights.npz``) and returns a ``MACE`` or ``ScaleShiftMACE`` object (``model_type``, default
ScaleShiftMACE as `model.py:680`).  Calling it follows `MACE.__call__` (`model.py:440-484`):

    model(positions, node_attrs, edge_index, shifts, cell=None, batch=None, num_graphs=1)
        -> {"energy": (num_graphs,), "node_energy": (N,)}   (+ "interaction_energy" for
                                                            ScaleShiftMACE, `model.py:550-589`)

with ``edge_index = [senders; receivers]``, ``shifts`` integer lattice shifts applied as
``shifts @ cell`` when a cell is given and Cartesian shift vectors otherwise
(`utils.py:47-84`), and per-graph energies summed over ``batch`` (`utils.py:35-44`).
``energy_forces`` returns the energy with its forces (and the virial dE/d(eps) on request),
the quantities the reference's calculator obtains by differentiating that call
(`calculators.py:424-563`).  Results are float64 numpy arrays; the arithmetic is the engine's
(float32 policy, or the float16 / bfloat16 feature policies of `model.py:592-661`).

Differences: there is no MLX graph to differentiate, so ``__call__`` takes no autograd
transformations; Cartesian shifts without a cell must be zero (an explicit cell carries periodic
images here).
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np

from ._ffi import Engine
from .device_model import FEATURE_POLICY, build_device_model, round_weights
from .model_io import ModelConfig, load_config, load_weights, select_head


class MACE:
    """A loaded model bound to one GPU (`model.py:86-484`)."""

    def __init__(self, config: ModelConfig, weights: Dict[str, np.ndarray], dtype: str = "float32",
                 head: Optional[str] = None, device: int = 0):
        if dtype not in FEATURE_POLICY:
            raise ValueError(f"dtype={dtype!r}: expected one of {sorted(FEATURE_POLICY)}")
        self.config = config
        self.dtype = dtype
        self.z_table = list(config.z_table) if config.z_table else list(range(config.num_elements))
        self._dm = build_device_model(config, weights, dtype=dtype, head=head)
        sel_cfg, sel_w = select_head(config, round_weights(weights, dtype), head)
        self._e0 = np.asarray(sel_w["atomic_energies_fn.atomic_energies"], dtype=np.float64).reshape(-1)
        self._engine = Engine(device, channels=self._dm.dims["num_channels"])
        self._engine.load_model(self._dm)
        self._sys_key = None
        self._edge_key = None

    # -- inputs ----------------------------------------------------------------
    def _species(self, node_attrs) -> np.ndarray:
        a = np.asarray(node_attrs)
        if a.ndim != 2 or a.shape[1] != self.config.num_elements:
            raise ValueError(f"node_attrs must be (num_atoms, {self.config.num_elements}) one-hot; got {a.shape}")
        return np.argmax(a, axis=1).astype(np.int32)

    def _prepare(self, positions, node_attrs, edge_index, shifts, cell):
        pos = np.ascontiguousarray(np.asarray(positions, dtype=np.float64).reshape(-1, 3))
        species = self._species(node_attrs)
        if len(species) != len(pos):
            raise ValueError(f"positions has {len(pos)} atoms, node_attrs {len(species)}")
        ei = np.asarray(edge_index).reshape(2, -1)
        sh = np.asarray(shifts, dtype=np.float64).reshape(-1, 3)
        if sh.shape[0] != ei.shape[1]:
            raise ValueError(f"shifts has {sh.shape[0]} rows, edge_index {ei.shape[1]} edges")
        if cell is not None:
            c = np.asarray(cell, dtype=np.float64).reshape(3, 3)
            S = np.rint(sh)
            if sh.size and np.abs(sh - S).max() > 1e-6:
                raise ValueError("with a cell, shifts must be integer lattice shifts (utils.py:74-78)")
            pbc = np.ones(3, dtype=bool)
        else:
            if sh.size and np.abs(sh).max() > 0:
                raise NotImplementedError("Cartesian shift vectors without a cell: pass the cell and "
                                          "integer lattice shifts")
            c = np.eye(3)
            S = np.zeros_like(sh)
            pbc = np.zeros(3, dtype=bool)
        key = (species.tobytes(), c.tobytes(), pbc.tobytes())
        if key != self._sys_key:
            self._engine.set_system(species, c, pbc, 0.0)
            self._sys_key = key
            self._edge_key = None
        snd = np.ascontiguousarray(ei[0], dtype=np.int32)
        rcv = np.ascontiguousarray(ei[1], dtype=np.int32)
        S = np.ascontiguousarray(S, dtype=np.int32)
        ekey = (snd.tobytes(), rcv.tobytes(), S.tobytes())
        if ekey != self._edge_key:
            self._engine.set_edges(snd, rcv, S)
            self._edge_key = ekey
        return pos, species

    # -- evaluation ------------------------------------------------------------
    def energy_forces(self, positions, node_attrs, edge_index, shifts, cell=None, stress: bool = False):
        """(energy, node_energy (N,), forces (N, 3), virial dE/d(eps_sym) (3, 3) or None) of one
        structure: `calculators.py:440-476` (forces) and 526-563 (virial, which needs the cell)."""
        pos, _ = self._prepare(positions, node_attrs, edge_index, shifts, cell)
        if stress and cell is None:
            raise ValueError("stress needs a cell")
        e, ne, f, vir = self._engine.step(pos, stress=stress)
        return e, ne, f, vir

    def __call__(self, positions, node_attrs, edge_index, shifts, cell=None, batch=None,
                 num_graphs: int = 1) -> dict:
        pos, species = self._prepare(positions, node_attrs, edge_index, shifts, cell)
        e, ne, _, _ = self._engine.step(pos)
        out = {"node_energy": ne}
        if num_graphs == 1 and batch is None:
            out["energy"] = np.array([e])
        else:
            b = np.zeros(len(ne), dtype=np.int64) if batch is None else np.asarray(batch, dtype=np.int64)
            out["energy"] = np.bincount(b, weights=ne, minlength=num_graphs)[:num_graphs]
        self._extra(out, species, batch, num_graphs)
        return out

    def _extra(self, out, species, batch, num_graphs):
        pass

    def close(self):
        self._engine.close()


class ScaleShiftMACE(MACE):
    """`model.py:508-589`: also reports the per-graph interaction energy (everything but E0,
    scaled and shifted)."""

    def _extra(self, out, species, batch, num_graphs):
        inter = out["node_energy"] - self._e0[species]
        b = np.zeros(len(inter), dtype=np.int64) if batch is None else np.asarray(batch, dtype=np.int64)
        out["interaction_energy"] = np.bincount(b, weights=inter, minlength=num_graphs)[:num_graphs]


def load_model(model_dir: str, dtype: str = "float32", head: Optional[str] = None, device: int = 0) -> MACE:
    """Drop-in for `mace_mlx.model.load_model` (`model.py:664-720`): a MACE or ScaleShiftMACE
    (``model_type`` in config.json, default ScaleShiftMACE) with its weights, rounded as a model
    of ``dtype`` ("float32", "float16", "bfloat16") holds them, on GPU ``device``."""
    if dtype not in FEATURE_POLICY:
        raise ValueError(f"dtype={dtype!r}: expected one of {sorted(FEATURE_POLICY)}")
    cfg = load_config(model_dir)
    w = load_weights(model_dir)
    cls = ScaleShiftMACE if cfg.model_type == "ScaleShiftMACE" else MACE
    return cls(cfg, w, dtype=dtype, head=head, device=device)
