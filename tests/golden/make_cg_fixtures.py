"""Write golden vectors for the host-side coupling constants.

Run in the build container only (it reads the reference checkout, which never
travels to the GPU box):

    python tests/golden/make_cg_fixtures.py [/root/reference]

It loads exactly two MLX-free modules of the reference by file path --
`mace_mlx/irreps.py` and `mace_mlx/clebsch_gordan.py` -- under a stub parent
package (the real `mace_mlx/__init__.py` imports MLX and is not executed), and
records their outputs:

* ``w3j_{l1}{l2}{l3}``   -- `wigner_3j` (clebsch_gordan.py:238-272), all l <= 3
* ``D_{l}_{k}``          -- `_wigner_D_real` (clebsch_gordan.py:80-83) at fixed angles
* ``U_{irreps}_{out}_{nu}_{idx|val|shape}`` -- `U_matrix_real`
  (clebsch_gordan.py:365-445), stored sparsely (the tensors are >99% zeros)

The path order inside the U tensors decides which weight multiplies which
coupling path; no invariant pins it, hence these vectors.
"""

from __future__ import annotations

import importlib.util
import sys
import types
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "cg_fixtures.npz"

ANGLES = [(0.3, 1.1, -0.7), (2.5, 0.4, 1.9), (-1.2, 2.8, 0.05)]
U_CASES = [
    ("0e+1o+2e+3o", "0e"), ("0e+1o+2e+3o", "1o"), ("0e+1o+2e+3o", "2e"),
    ("0e+1o+2e", "0e"), ("0e+1o", "0e"), ("0e+1o", "1o"),
]


def _load(ref: Path):
    pkg = types.ModuleType("mace_mlx")
    pkg.__path__ = [str(ref / "mace_mlx")]
    sys.modules["mace_mlx"] = pkg
    mods = {}
    for name in ("irreps", "clebsch_gordan"):
        spec = importlib.util.spec_from_file_location(
            f"mace_mlx.{name}", ref / "mace_mlx" / f"{name}.py")
        mod = importlib.util.module_from_spec(spec)
        sys.modules[f"mace_mlx.{name}"] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods["clebsch_gordan"]


def main(ref: str = "/root/reference") -> None:
    cg = _load(Path(ref))
    out = {}
    for l1 in range(4):
        for l2 in range(4):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 3) + 1):
                out[f"w3j_{l1}{l2}{l3}"] = cg.wigner_3j(l1, l2, l3)
    for l in range(4):
        for k, (a, b, c) in enumerate(ANGLES):
            out[f"D_{l}_{k}"] = cg._wigner_D_real(l, a, b, c)
    for irreps, ir_out in U_CASES:
        for nu in (1, 2, 3):
            U = cg.U_matrix_real(irreps_in=irreps, irreps_out=f"1x{ir_out}", correlation=nu)[-1]
            key = f"U_{irreps.replace('+', '_')}_{ir_out}_{nu}"
            idx = np.argwhere(np.abs(U) > 0.0)
            out[key + "_shape"] = np.array(U.shape, dtype=np.int64)
            out[key + "_idx"] = idx.astype(np.int16)
            out[key + "_val"] = U[tuple(idx.T)]
    out["angles"] = np.array(ANGLES)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({len(out)} arrays)")


if __name__ == "__main__":
    main(*sys.argv[1:])
