"""Synthetic structures and models for the five benchmark configurations.

ASE is not required.  Lattices are built in the order ASE uses
(``bulk(..., cubic=True)`` followed by ``atoms.repeat((n1, n2, n3))``: copies of
the conventional cell ordered with the first repeat index outermost), and rattled
the way the reference's benchmarks do it
(``pos += np.random.default_rng(seed).normal(scale=sigma, size=(N, 3))``,
`docs/prototypes/xbench.py:85-86`).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import List, Optional

import numpy as np

from .model_io import NONLINEAR_BLOCK, ModelConfig, random_init, save_model

# conventional cells in fractional coordinates
_DIAMOND = np.array([
    (0, 0, 0), (0.25, 0.25, 0.25), (0, 0.5, 0.5), (0.25, 0.75, 0.75),
    (0.5, 0, 0.5), (0.75, 0.25, 0.75), (0.5, 0.5, 0), (0.75, 0.75, 0.25)])
_FCC = np.array([(0, 0, 0), (0, 0.5, 0.5), (0.5, 0, 0.5), (0.5, 0.5, 0)])

HEA_SPECIES = [26, 28, 27, 24, 25]  # Fe, Ni, Co, Cr, Mn


@dataclass
class System:
    """Plain structure record (positions in Angstrom, Cartesian)."""

    positions: np.ndarray      # (N, 3) float64
    numbers: np.ndarray        # (N,) int64 atomic numbers
    cell: np.ndarray           # (3, 3) float64, rows are lattice vectors
    pbc: np.ndarray            # (3,) bool
    name: str = ""

    def __len__(self) -> int:
        return len(self.numbers)

    # duck-typed subset of ase.Atoms used by the calculator
    def get_positions(self):
        return self.positions.copy()

    def get_atomic_numbers(self):
        return self.numbers.copy()

    def get_cell(self):
        return self.cell.copy()

    def copy(self) -> "System":
        return System(self.positions.copy(), self.numbers.copy(), self.cell.copy(),
                      self.pbc.copy(), self.name)


def lattice(basis: np.ndarray, a: float, reps, z) -> System:
    reps = tuple(int(r) for r in reps)
    cell0 = np.eye(3) * a
    frac = []
    for m0 in range(reps[0]):
        for m1 in range(reps[1]):
            for m2 in range(reps[2]):
                frac.append(basis + np.array([m0, m1, m2], dtype=np.float64))
    frac = np.concatenate(frac, axis=0)
    pos = frac @ cell0
    cell = cell0 * np.array(reps, dtype=np.float64)[:, None]
    n = len(pos)
    numbers = np.full(n, z, dtype=np.int64) if np.isscalar(z) else np.asarray(z, np.int64)
    return System(pos, numbers, cell, np.array([True, True, True]))


def diamond_si(reps, a: float = 5.43) -> System:
    return lattice(_DIAMOND, a, reps, 14)


def rattle(s: System, sigma: float, seed: int, rng: Optional[np.random.Generator] = None) -> System:
    rng = np.random.default_rng(seed) if rng is None else rng
    out = s.copy()
    out.positions = out.positions + rng.normal(scale=sigma, size=out.positions.shape)
    return out


def arch_config(arch: str, num_elements: int = 1, z_table=None, zbl: bool = False,
                atomic_energies=None, avg_num_neighbors: float = 1.0,
                trained_topology: bool = False) -> ModelConfig:
    """Benchmark architectures.  trained_topology selects the layout of the reference's
    default foundation models (medium-mpa-0 family, `model.py:153-247`): Agnesi distance
    transform, density-normalised interactions, non-residual first interaction, 10 Bessel
    functions."""
    hidden = {"small": "128x0e", "medium": "128x0e+128x1o",
              "large": "128x0e+128x1o+128x2e"}[arch]
    return ModelConfig(
        r_max=6.0, num_bessel=10 if trained_topology else 8, num_polynomial_cutoff=5, max_ell=3,
        num_interactions=2, hidden_irreps=hidden, correlation=[3, 3],
        num_elements=num_elements, atomic_energies=atomic_energies,
        avg_num_neighbors=avg_num_neighbors, radial_MLP=[64, 64, 64],
        model_type="MACE", z_table=list(z_table) if z_table is not None else [14],
        pair_repulsion={"p": 6, "a_exp": 0.3, "a_prefactor": 0.4543} if zbl else None,
        distance_transform={"q": 0.9183, "p": 4.5791, "a": 1.0805} if trained_topology else None,
        use_density_normalization=trained_topology,
        first_interaction_nonresidual=trained_topology,
    )


# MACE-OFF23 elements (H, C, N, O, F, P, S, Cl, Br, I) and widths by model size
OFF_ELEMENTS = [1, 6, 7, 8, 9, 15, 16, 17, 35, 53]
OFF_HIDDEN = {"small": "96x0e", "medium": "128x0e+128x1o", "large": "192x0e+192x1o+192x2e"}


def off_config(size: str = "small") -> ModelConfig:
    """The layout of the MACE-OFF23 organic force fields that ``mace_off`` loads (`README.md:75`,
    `calculators.py:601-617`): ScaleShiftMACE over ten elements, r_max 5 A, non-residual first
    interaction, 96 / 128 / 192 channels.  E0, scale / shift and avg_num_neighbors are chosen so
    that a random model's interaction energy is not hidden under E0 and its forces are O(1) eV/A."""
    rng = np.random.default_rng(40)
    return ModelConfig(
        r_max=5.0, num_bessel=8, num_polynomial_cutoff=5, max_ell=3, num_interactions=2,
        hidden_irreps=OFF_HIDDEN[size], correlation=[3, 3], num_elements=len(OFF_ELEMENTS),
        atomic_energies=[float(x) for x in -rng.uniform(0.5, 2.0, len(OFF_ELEMENTS))],
        avg_num_neighbors=3.0, radial_MLP=[64, 64, 64], model_type="ScaleShiftMACE", scale=8.0,
        shift=0.05, z_table=list(OFF_ELEMENTS), first_interaction_nonresidual=True)


def organic_cluster(n: int = 48, seed: int = 41) -> System:
    """A non-periodic cluster of H / C / N / O atoms on a rattled 1.5 A grid (a stand-in for
    the organic molecules MACE-OFF is used on)."""
    rng = np.random.default_rng(seed)
    k = int(np.ceil(n ** (1 / 3)))
    g = np.stack(np.meshgrid(*[np.arange(k)] * 3, indexing="ij"), -1).reshape(-1, 3)[:n]
    pos = 10.0 + 1.5 * g + rng.normal(scale=0.1, size=(n, 3))
    z = np.array([1, 6, 7, 8])[rng.integers(0, 4, n)]
    return System(pos, z.astype(np.int64), np.eye(3) * 40.0, np.array([False, False, False]))


@dataclass
class BenchConfig:
    index: int
    name: str
    system: System
    model: ModelConfig
    properties: List[str]
    dtype: str = "float32"


def make_config(index: int) -> BenchConfig:
    """Configurations 1..5 of the benchmark definition (0-based index 0..4); index 5, outside
    that definition, is the Si1000 system under an mh-1 model (non-linear interaction blocks,
    `blocks.py:611-807`, with the mh-1 foundation models' element-agnostic product, separate
    cutoff, 1o edge irreps and 89 elements); indices 6 and 7, also outside it, are MACE-OFF-shaped
    models (96 and 192 channels, run zero-padded on the 128- and 256-channel engines) on a periodic
    1000-atom organic liquid stand-in."""
    if index == 0:
        s = rattle(diamond_si((2, 2, 2)), 0.01, 0)
        m = arch_config("small")
        return BenchConfig(0, "Si64-small", s, m, ["energy", "forces"])
    if index == 1:
        s = rattle(diamond_si((5, 5, 5)), 0.03, 1)
        m = arch_config("medium", zbl=True)
        return BenchConfig(1, "Si1000-medium", s, m, ["energy", "forces"])
    if index == 2:
        s = diamond_si((5, 5, 10))
        s.positions *= 1.02
        s.cell *= 1.02
        s = rattle(s, 0.03, 2)
        m = arch_config("medium")
        return BenchConfig(2, "Si2000-medium-strained", s, m, ["energy", "forces", "stress"])
    if index == 3:
        s = rattle(diamond_si((8, 8, 8)), 0.05, 3)
        m = arch_config("large")
        return BenchConfig(3, "Si4096-large", s, m, ["energy", "forces", "stress"])
    if index == 4:
        rng = np.random.default_rng(4)
        base = lattice(_FCC, 3.6, (20, 20, 20), 26)
        kinds = rng.integers(0, 5, len(base))
        base.numbers = np.array(HEA_SPECIES, dtype=np.int64)[kinds]
        s = rattle(base, 0.05, 4, rng=rng)
        e0rng = np.random.default_rng(1004)
        e0 = (-5.0 + e0rng.normal(scale=2.0, size=89)).tolist()
        m = arch_config("medium", num_elements=89, z_table=range(1, 90),
                        atomic_energies=e0)
        return BenchConfig(4, "HEA32000-medium-fp16", s, m, ["energy", "forces"],
                           dtype="float16")
    if index == 5:
        s = rattle(diamond_si((5, 5, 5)), 0.03, 1)
        m = arch_config("medium", num_elements=89, z_table=range(1, 90))
        m.interaction_cls = NONLINEAR_BLOCK
        m.edge_irreps = "128x0e+128x1o"
        m.apply_cutoff = False
        m.use_agnostic_product = True
        return BenchConfig(5, "Si1000-mh1", s, m, ["energy", "forces"])
    if index in (6, 7):
        size = "small" if index == 6 else "large"
        return BenchConfig(index, f"Organic1000-off-{size}", organic_liquid(), off_config(size),
                           ["energy", "forces"])
    raise ValueError(index)


def organic_liquid(n_side: int = 10, density: float = 0.1, seed: int = 49) -> System:
    """A periodic H / C / N / O liquid stand-in at a molecular liquid's atom density (0.1 per
    cubic Angstrom, ~50 neighbours within 5.5 A): n_side^3 atoms on a cubic grid jittered by
    0.25 A, elements drawn 5 : 3 : 1 : 1."""
    rng = np.random.default_rng(seed)
    a = density ** (-1.0 / 3.0)
    g = np.stack(np.meshgrid(*[np.arange(n_side)] * 3, indexing="ij"), -1).reshape(-1, 3)
    pos = a * g + rng.normal(scale=0.25, size=g.shape)
    z = rng.choice(np.array([1, 6, 7, 8]), size=len(g), p=[0.5, 0.3, 0.1, 0.1])
    return System(pos, z.astype(np.int64), np.eye(3) * a * n_side, np.array([True, True, True]))


def write_model_dir(cfg: ModelConfig, path, seed: int = 0) -> Path:
    return save_model(path, cfg, random_init(cfg, seed))
