"""Build the HIP engine in-tree: generate the constant tables, then hipcc (gfx950).

``python -m mace_mlx_amd.build`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parents[1] / "csrc"


def build(jobs: int = 8, verbose: bool = False) -> Path:
    env = dict(os.environ)
    env.setdefault("PYTHON", sys.executable)
    subprocess.run([sys.executable, str(CSRC / "gen_tables.py"), str(CSRC / "gen")], check=True,
                   stdout=None if verbose else subprocess.DEVNULL)
    # -B: compile every source each time (the build is also the "does it build" check)
    proc = subprocess.run(["make", "-B", "-C", str(CSRC), f"-j{jobs}"], env=env, capture_output=not verbose, text=True)
    if proc.returncode != 0:
        sys.stderr.write((proc.stdout or "") + (proc.stderr or ""))
        raise RuntimeError("HIP engine build failed")
    from ._ffi import LIB_PATH, LIB_PATHS
    # every kernel the host registers must exist in the gfx950 code objects of each library (the
    # HIP runtime aborts at the first launch of one that does not)
    for path in LIB_PATHS.values():
        chk = subprocess.run([sys.executable, str(CSRC / "check_kernel_symbols.py"), str(path)],
                             capture_output=True, text=True)
        if chk.returncode != 0:
            sys.stderr.write(chk.stdout + chk.stderr)
            raise RuntimeError(f"HIP engine build ({path.name}): host / device kernel names differ")
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
