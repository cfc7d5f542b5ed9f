"""mace_step_device_noalloc (the entry point that allocates nothing) against
mace_step_device, through the C ABI, on two calls in a row, the second with a smaller
system.  Both run the same kernels in the same order, so the results must be identical
bit for bit (energy, virial and forces); the no-allocation variant differs only in where
the per-block energy / virial partials live (a fixed device array inside the library)
and in launching eagerly instead of replaying a captured graph."""

import numpy as np
import pytest
import torch

from gpu_helpers import Case
from mace_mlx_amd.systems import arch_config, diamond_si, rattle

pytestmark = pytest.mark.gpu


def _both(case, s, stress):
    eng = case.eng
    sp = np.zeros(len(s), np.int32)
    eng.set_system(sp, s.cell, s.pbc, 0.5)
    eng.step(s.positions, stress=stress)            # builds the neighbour list
    N = len(s)
    pos_d = torch.from_numpy(np.ascontiguousarray(s.positions, dtype=np.float64)).cuda()
    ref_d = torch.full((10 + 3 * N,), -1.0, dtype=torch.float64, device="cuda")
    got_d = torch.full((10 + 3 * N,), -2.0, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    eng.step_device(pos_d.data_ptr(), ref_d.data_ptr(), stress=stress)
    eng.sync()
    eng.step_device_noalloc(pos_d.data_ptr(), got_d.data_ptr(), stress=stress)
    eng.sync()
    return ref_d.cpu().numpy(), got_d.cpu().numpy()


def test_noalloc_matches_step_device_twice():
    case = Case(arch_config("medium", zbl=True))
    big = rattle(diamond_si((3, 3, 3)), 0.05, 21)
    small = rattle(diamond_si((2, 2, 2)), 0.04, 22)
    for s, stress in ((big, True), (small, True), (small, False)):
        print(f"noalloc vs step_device: N={len(s)} stress={stress}", flush=True)
        ref, got = _both(case, s, stress)
        assert np.isfinite(ref).all() and ref[0] != -1.0
        np.testing.assert_array_equal(got, ref)
    # what the entry point refuses, without launching anything
    eng = case.eng
    N = len(small)
    pos_d = torch.from_numpy(np.ascontiguousarray(small.positions, dtype=np.float64)).cuda()
    out_d = torch.zeros(10 + 3 * N, dtype=torch.float64, device="cuda")
    flags_force_nl = 1 | 4
    rc = eng._lib.mace_step_device_noalloc(eng._h, pos_d.data_ptr(), flags_force_nl, out_d.data_ptr())
    assert rc == -1 and b"neighbour list" in eng._lib.mace_last_error(eng._h)
    moved = rattle(diamond_si((2, 2, 3)), 0.04, 23)         # new topology: no neighbour list yet
    eng.set_system(np.zeros(len(moved), np.int32), moved.cell, moved.pbc, 0.5)
    pos_m = torch.from_numpy(np.ascontiguousarray(moved.positions, dtype=np.float64)).cuda()
    out_m = torch.zeros(10 + 3 * len(moved), dtype=torch.float64, device="cuda")
    with pytest.raises(RuntimeError):
        eng.step_device_noalloc(pos_m.data_ptr(), out_m.data_ptr())
