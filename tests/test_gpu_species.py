"""GPU tests of the per-species products.

With one-hot node attributes the reference's skip connections are FullyConnectedTensorProducts
whose weights depend on the element: the residual skip (`blocks.py:262,467`) and, in a
non-residual first block, the message skip (`blocks.py:174,382`).  The engine sorts the atoms by
species once per system and runs each such product as one matrix-core problem per species
present, over that species' atoms (a row map into the sorted order).  These tests take ragged
species counts (a species with one atom, absent species, interleaved order), both product paths
(split fp16 and fp32 matrix cores), and a change of species at the same atom count, which
re-sorts the atoms and re-captures the step graphs.
"""

import numpy as np
import pytest

from gpu_helpers import Case, assert_parity
from mace_mlx_amd.systems import arch_config, diamond_si, rattle

pytestmark = pytest.mark.gpu

Z10 = [1, 6, 7, 8, 9, 14, 15, 16, 17, 35]


def _ragged_numbers(n, seed):
    """Seven of the ten elements, counts 1, 2, 5 and the rest spread at random over the order."""
    rng = np.random.default_rng(seed)
    present = [Z10[k] for k in (0, 1, 3, 5, 6, 8, 9)]
    nums = [present[0]] + [present[1]] * 2 + [present[2]] * 5
    nums += list(rng.choice(present[3:], size=n - len(nums)))
    return np.array(rng.permutation(nums))


@pytest.mark.parametrize("trained", [True, False])
def test_species_grouped_products(trained):
    """E, F and stress against the float64 oracle for a ten-element model on a 216-atom cell
    with seven species present: trained topology (non-residual first block: message skip, then a
    residual block: skip connection) and the plain layout (skip connections in both blocks).
    Without E0 the random-init interaction energies of either sign sum to |E| of about 2 eV over
    216 atoms, so the energy bar is the per-atom one; node energies (1e-5 of the largest) and
    forces check every atom's species-dependent terms."""
    cfg = arch_config("medium", num_elements=10, z_table=Z10, zbl=True, trained_topology=trained)
    case = Case(cfg, seed=61)
    s = rattle(diamond_si((3, 3, 3)), 0.05, 62)
    s.numbers = _ragged_numbers(len(s), 63)
    print(f"ten elements, trained={trained}: split products", flush=True)
    got = case.run(s, stress=True)
    edges = case.edges()
    ref = case.reference(s, got["sp"], edges, stress=True)
    assert_parity(got, ref, len(s), stress=True, energy="per_atom")
    print(f"ten elements, trained={trained}: fp32 matrix cores", flush=True)
    case.eng.set_split_products(False)
    got = case.run(s, stress=True)
    assert_parity(got, ref, len(s), stress=True, energy="per_atom")
    case.eng.set_split_products(True)


def test_species_change_at_same_size():
    """A new species assignment with the same atom count re-sorts the rows: each assignment
    matches the oracle, and returning to the first reproduces its result bit for bit."""
    cfg = arch_config("medium", num_elements=10, z_table=Z10, zbl=True, trained_topology=True)
    case = Case(cfg, seed=64)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 65)
    first = _ragged_numbers(len(s), 66)
    results = []
    for k, nums in enumerate([first, first[::-1].copy(), np.full(len(s), Z10[4]), first]):
        s.numbers = nums
        print(f"species assignment {k}", flush=True)
        got = case.run(s)
        if k < 3:
            assert_parity(got, case.reference(s, got["sp"], case.edges()), len(s), energy="per_atom")
        results.append(got)
    assert results[3]["E"] == results[0]["E"]
    assert np.array_equal(results[3]["F"], results[0]["F"])


def test_model_reload_keeps_or_drops_the_system():
    """Loading another model keeps the system when its species are elements of the new model
    (the species order is rebuilt for the new element count: the step equals a fresh engine's)
    and drops it otherwise (the step raises until mace_set_system is called again)."""
    cfg10 = arch_config("medium", num_elements=10, z_table=Z10, zbl=True, trained_topology=True)
    a, b = Case(cfg10, seed=67), Case(cfg10, seed=68)
    s = rattle(diamond_si((2, 2, 2)), 0.05, 69)
    s.numbers = _ragged_numbers(len(s), 70)
    a.run(s)
    a.eng.load_model(b.dm)                       # same elements: the system stays
    E, ne, F, _ = a.eng.step(s.positions)
    want = b.run(s)
    assert abs(E - want["E"]) <= 1e-7 * max(abs(want["E"]), len(s))
    assert np.abs(F - want["F"]).max() <= 1e-5
    cfg2 = arch_config("medium", num_elements=2, z_table=[6, 14], zbl=True)
    c = Case(cfg2, seed=71)
    a.eng.load_model(c.dm)                       # species 2..9 are not elements of this model
    with pytest.raises(RuntimeError):
        a.eng.step(s.positions)
    s2 = s.copy()
    s2.numbers = np.where(np.arange(len(s)) % 3 == 0, 6, 14)
    sp = np.where(np.arange(len(s)) % 3 == 0, 0, 1).astype(np.int32)
    a.eng.set_system(sp, s2.cell, s2.pbc, 0.5)
    E2, _, F2, _ = a.eng.step(s2.positions)
    want2 = c.run(s2)
    assert abs(E2 - want2["E"]) <= 1e-7 * max(abs(want2["E"]), len(s))
    assert np.abs(F2 - want2["F"]).max() <= 1e-5
