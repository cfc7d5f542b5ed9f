"""ASE calculator API of the reference (`mace_mlx/calculators.py`), driving the HIP engine.

Drop-in names: ``MACECalculator`` (= ``MACEHIPCalculator``), ``mace_mp``,
``mace_off``, plus ``mace_anicc`` / ``mace_omol`` which raise like the reference.

Behaviour kept from the reference:

* constructor arguments ``model_path | model_paths, device, default_dtype, head,
  skin=0.5, use_compile=True`` (`calculators.py:87-96`); committee models raise
  NotImplementedError (100-106); float64 warns and falls back to float32 (112-118);
* ``implemented_properties`` and the results keys ``energy, free_energy, forces,
  node_energy, energies, stress`` (82, 413-418);
* neighbour list at ``r_max + skin`` rebuilt only when N, pbc or the cell change
  (atol 1e-10) or an atom moved more than ``skin / 2`` (266-283) -- evaluated
  inside the engine, on the device;
* unknown atomic numbers raise ValueError with the supported list (345-354);
* multi-head models evaluate the ``head`` named at construction, else the first;
  an unknown name raises ValueError (128-137);
* stress = dE/d(eps_sym) / |det cell| in Voigt order xx, yy, zz, yz, xz, xy
  (515-523), computed in the same backward pass; once requested for a 3-D
  periodic cell it stays on for later steps (385-388).

Differences: ``device="cpu"`` is refused (this engine has no CPU path), and
named foundation models are read from the reference's conversion cache
(``$MACE_MLX_CACHE_DIR`` or ``~/.cache/mace_mlx/<name>/v2``); converting a
checkpoint needs torch + mace-torch + network, as in the reference (194-260).
"""

from __future__ import annotations

import os
import warnings
from pathlib import Path
from typing import Optional

import numpy as np

from ._ffi import Engine
from .device_model import build_device_model
from .model_io import head_index, load_config, load_weights

try:  # ASE is optional: the engine works with any object exposing the Atoms API
    from ase.calculators.calculator import Calculator as _AseCalculator, all_changes  # type: ignore
    _HAVE_ASE = True
except ImportError:  # pragma: no cover - exercised in the ASE-free test image
    _HAVE_ASE = False
    all_changes = ["positions", "numbers", "cell", "pbc", "initial_charges", "initial_magmoms"]

    class _AseCalculator:  # minimal stand-in for ase.calculators.calculator.Calculator
        implemented_properties: list = []

        def __init__(self, **kwargs):
            self.results = {}
            self.atoms = None
            self.parameters = dict(kwargs)

        def calculate(self, atoms=None, properties=None, system_changes=all_changes):
            if atoms is not None:
                self.atoms = atoms.copy()

        def get_property(self, name, atoms=None, allow_calculation=True):
            if atoms is None:
                atoms = self.atoms
            if name not in self.results or self._changed(atoms):
                self.results = {}
                self.calculate(atoms, [name], all_changes)
            return self.results[name]

        def _changed(self, atoms):
            a = self.atoms
            if a is None or atoms is None:
                return True
            return not (len(a) == len(atoms)
                        and np.array_equal(a.get_positions(), atoms.get_positions())
                        and np.array_equal(a.get_atomic_numbers(), atoms.get_atomic_numbers())
                        and np.array_equal(np.asarray(a.get_cell()), np.asarray(atoms.get_cell()))
                        and np.array_equal(np.asarray(a.pbc), np.asarray(atoms.pbc)))

        def get_potential_energy(self, atoms=None, force_consistent=False):
            return self.get_property("free_energy" if force_consistent else "energy", atoms)

        def get_forces(self, atoms=None):
            return self.get_property("forces", atoms).copy()

        def get_stress(self, atoms=None):
            return self.get_property("stress", atoms).copy()

_DEVICE_MAP = {"cuda": "gpu", "mps": "gpu", "gpu": "gpu", "rocm": "gpu", "hip": "gpu", "cpu": "cpu", "": "gpu"}
_CONVERTER_CACHE_VERSION = 2
_NAMED = ("small", "medium", "large", "medium-mpa-0")


def _cache_root() -> Path:
    env = os.environ.get("MACE_MLX_CACHE_DIR")
    return Path(env).expanduser() if env else Path.home() / ".cache" / "mace_mlx"


def _cell_rank(atoms) -> int:
    cell = atoms.cell if hasattr(atoms, "cell") else atoms.get_cell()
    if hasattr(cell, "rank"):
        return int(cell.rank)
    c = np.asarray(cell, dtype=np.float64)
    return int(np.sum(np.linalg.norm(c, axis=1) > 0))


def _pbc(atoms) -> np.ndarray:
    return np.asarray(atoms.pbc, dtype=bool).reshape(3)


class MACEHIPCalculator(_AseCalculator):
    """ASE calculator running the MACE energy / forces / stress step on an AMD GPU."""

    implemented_properties = ["energy", "energies", "free_energy", "node_energy", "forces", "stress"]

    def __init__(self, model_path: Optional[str] = None, device: str = "gpu", default_dtype: str = "float32",
                 head: Optional[str] = None, skin: float = 0.5, use_compile: bool = True, **kwargs):
        if model_path is None:
            model_path = kwargs.pop("model_paths", None)
            if isinstance(model_path, (list, tuple)):
                if len(model_path) > 1:
                    raise NotImplementedError(
                        f"committee models are not supported; got {len(model_path)} model paths")
                model_path = model_path[0] if model_path else None
        if model_path is None:
            model_path = "medium-mpa-0"
        if default_dtype == "float64":
            warnings.warn("the HIP engine computes in float32; falling back from float64 "
                          "(results differ from float64 at the float32 precision level)")
            default_dtype = "float32"
        if default_dtype not in ("float32", "float16", "bfloat16"):
            raise NotImplementedError(
                f"default_dtype={default_dtype!r} (float32, float16 and bfloat16 are implemented)")
        dev = _DEVICE_MAP.get(str(device).split(":")[0], device)
        if dev != "gpu":
            raise NotImplementedError(f"device={device!r}: this engine runs on AMD GPUs only")
        dev_index = int(str(device).split(":")[1]) if ":" in str(device) else 0
        super().__init__(**kwargs)
        model_dir = self._resolve_model(str(model_path))
        self.config = load_config(model_dir)
        # multi-head: the named head, else the first; ValueError for an unknown name
        # (calculators.py:128-137); the engine holds that head's readouts only
        self._head = None
        if self.config.num_heads > 1:
            self._head = self.config.heads[head_index(self.config, head)]
        weights = load_weights(model_dir)
        self._dm = build_device_model(self.config, weights, dtype=default_dtype, head=self._head)
        self.default_dtype = default_dtype
        self.r_max = float(self.config.r_max)
        self.z_table = list(self._dm.z_table)
        self._z_to_idx = {int(z): i for i, z in enumerate(self.z_table)}
        self._skin = float(skin)
        self._use_compile = use_compile
        self._engine = Engine(dev_index, channels=self._dm.dims["num_channels"])
        self._engine.load_model(self._dm)
        self._sys_key = None
        self._stress_always = False

    @staticmethod
    def _resolve_model(model_path: str) -> str:
        p = Path(model_path).expanduser()
        if (p / "config.json").exists() and (p / "weights.npz").exists():
            return str(p)
        named = model_path.startswith("off-") or model_path in _NAMED
        if not named:
            raise FileNotFoundError(f"model directory {model_path!r} has no config.json + weights.npz")
        target = _cache_root() / model_path / f"v{_CONVERTER_CACHE_VERSION}"
        if (target / "config.json").exists() and (target / "weights.npz").exists():
            return str(target)
        raise ImportError(
            f"Converting the named model '{model_path}' requires torch and mace-torch (one-time "
            f"download + weight conversion into {target}); place a converted config.json + "
            "weights.npz there or pass a model directory")

    # -- ASE -----------------------------------------------------------------
    def _species(self, atoms) -> np.ndarray:
        """Element indices of the atoms, cached while the atomic numbers stay the same (the
        reference's one-hot cache, `calculators.py:330-364`); ValueError names the first
        unsupported atomic number (345-354)."""
        numbers = np.asarray(atoms.get_atomic_numbers())
        key = numbers.tobytes()
        cache = getattr(self, "_species_cache", None)
        if cache is not None and cache[0] == key:
            return cache[1]
        lut = getattr(self, "_z_lut", None)
        if lut is None:
            lut = np.full(max(self._z_to_idx, default=0) + 1, -1, dtype=np.int64)
            for z, i in self._z_to_idx.items():
                lut[z] = i
            self._z_lut = lut
        z = numbers.astype(np.int64).reshape(-1)
        idx = np.where((z >= 0) & (z < len(lut)), lut[np.clip(z, 0, len(lut) - 1)], -1)
        if (idx < 0).any():
            bad = int(z[np.argmax(idx < 0)])
            raise ValueError(f"Atomic number {bad} is not supported by this model. "
                             f"Supported: {sorted(self._z_to_idx)}")
        out = idx.astype(np.int32)
        self._species_cache = (key, out)
        return out

    def calculate(self, atoms=None, properties=None, system_changes=all_changes):
        super().calculate(atoms, properties, system_changes)
        atoms = self.atoms if atoms is None else atoms
        species = self._species(atoms)
        cell = np.asarray(atoms.get_cell(), dtype=np.float64).reshape(3, 3)
        pbc = _pbc(atoms)
        key = (species.tobytes(), cell.tobytes(), pbc.tobytes())
        if key != self._sys_key:
            self._engine.set_system(species, cell, pbc, self._skin)
            self._sys_key = key
        rank3 = _cell_rank(atoms) == 3
        if properties is not None and "stress" in properties and rank3:
            self._stress_always = True
        want = "stress" in (properties or self.implemented_properties)
        compute_stress = (want or self._stress_always) and rank3
        e, ne, f, vir = self._engine.step(np.asarray(atoms.get_positions(), dtype=np.float64),
                                          stress=compute_stress)
        self.results["energy"] = float(e)
        self.results["free_energy"] = self.results["energy"]
        self.results["forces"] = f
        self.results["node_energy"] = ne
        self.results["energies"] = ne
        if compute_stress:
            vol = abs(np.linalg.det(cell))
            st = vir / vol
            self.results["stress"] = st[[0, 1, 2, 1, 0, 0], [0, 1, 2, 2, 2, 1]]

    def calculate_batch(self, atoms_list, properties=("energy", "forces")):
        """Several structures in one engine step: the reference model's batched call
        (`model.py:440-484` with `batch` / `num_graphs`; energies per structure by
        `graph_sum`, `utils.py:35-44`), each structure in its own cell.  Returns one dict per
        structure with the keys `calculate` fills (stress only for 3-D periodic cells when
        requested); the calculator's own `results` are left alone."""
        atoms_list = list(atoms_list)
        if not atoms_list:
            return []
        species = [self._species(a) for a in atoms_list]
        cells = np.stack([np.asarray(a.get_cell(), dtype=np.float64).reshape(3, 3) for a in atoms_list])
        pbcs = np.stack([_pbc(a) for a in atoms_list])
        self._engine.set_batch(species, cells, pbcs, self._skin)
        self._sys_key = None   # the engine now holds the batch; calculate() re-uploads its system
        stress = "stress" in properties
        pos = np.concatenate([np.asarray(a.get_positions(), dtype=np.float64).reshape(-1, 3) for a in atoms_list])
        eg, ne, f, vir = self._engine.step_batch(pos, stress=stress)
        out, i0 = [], 0
        for g, a in enumerate(atoms_list):
            n = len(species[g])
            r = {"energy": float(eg[g]), "free_energy": float(eg[g]), "forces": f[i0:i0 + n],
                 "node_energy": ne[i0:i0 + n], "energies": ne[i0:i0 + n]}
            if stress and _cell_rank(a) == 3:
                st = vir[g] / abs(np.linalg.det(cells[g]))
                r["stress"] = st[[0, 1, 2, 1, 0, 0], [0, 1, 2, 2, 2, 1]]
            out.append(r)
            i0 += n
        return out

    # timing of the last step on the device (ms): total, neighbour list, forward, backward
    def last_timings(self) -> np.ndarray:
        return self._engine.timings()


def mace_mp(model: Optional[str] = None, device: str = "gpu", default_dtype: str = "float32",
            head: Optional[str] = None, dispersion: bool = False, return_raw_model: bool = False,
            **kwargs) -> MACEHIPCalculator:
    """Drop-in for ``mace_mlx.mace_mp`` (`calculators.py:566-598`)."""
    if return_raw_model:
        raise NotImplementedError("return_raw_model is not supported")
    if dispersion:
        warnings.warn("D3 dispersion corrections are not supported. Ignoring dispersion=True.")
    for key in ("damping", "dispersion_xc", "dispersion_cutoff"):
        kwargs.pop(key, None)
    return MACEHIPCalculator(model_path=model, device=device, default_dtype=default_dtype, head=head, **kwargs)


def mace_off(model: str = "small", device: str = "gpu", default_dtype: str = "float32",
             **kwargs) -> MACEHIPCalculator:
    """Drop-in for ``mace_mlx.mace_off`` (`calculators.py:601-617`)."""
    return MACEHIPCalculator(model_path=f"off-{model}", device=device, default_dtype=default_dtype, **kwargs)


def mace_anicc(**kwargs):
    raise NotImplementedError("mace_anicc is not supported. Use mace-torch for ANI models.")


def mace_omol(**kwargs):
    raise NotImplementedError("mace_omol is not supported. Use mace-torch for OMOL models.")


MACECalculator = MACEHIPCalculator
