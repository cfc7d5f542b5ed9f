"""ctypes binding of the HIP engine's C ABI (include/mace_hip.h).

The library is loaded from ``mace_mlx_amd/_lib/libmace_hip.so``.  There is no
fallback: if the library is missing or no HIP device is present, construction
raises.  Status codes map to the exception types the reference raises for the
same conditions (`calculators.py:100-136,345-354`).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmace_hip.so"
# the same engine compiled for each channel count (csrc/common.h MACE_NC); a model with C
# channels runs on the smallest width >= C (device_model pads the rest with zeros)
ENGINE_WIDTHS = (128, 192, 256)
LIB_PATHS = {128: LIB_PATH, 192: LIB_PATH.with_name("libmace_hip_c192.so"),
             256: LIB_PATH.with_name("libmace_hip_c256.so")}

MACE_OK = 0
MACE_ERR_INVALID = -1
MACE_ERR_HIP = -2
MACE_ERR_UNSUPPORTED = -3
MACE_ERR_STATE = -4
MACE_ERR_SPECIES = -5

STEP_FORCES = 1
STEP_STRESS = 2
STEP_FORCE_NL = 4
STEP_SKIN_CHECK = 8

EXPORTED_SYMBOLS = (
    "mace_create", "mace_destroy", "mace_last_error", "mace_model_begin", "mace_model_set_tensor",
    "mace_model_end", "mace_set_system", "mace_step", "mace_set_edges", "mace_get_edges",
    "mace_get_timings", "mace_step_device", "mace_sync", "mace_set_profiling", "mace_get_kernel_times",
    "mace_set_graphs",
    "mace_set_split_products",
    "mace_set_fused_tp",
    "mace_set_rebuild_w",
    "mace_set_batch", "mace_step_batch",
    "mace_get_launch_order",
    "mace_step_device_noalloc",
)


class HipError(RuntimeError):
    pass


class ModelDims(ctypes.Structure):
    _fields_ = [
        ("num_elements", ctypes.c_int32), ("num_channels", ctypes.c_int32),
        ("max_ell", ctypes.c_int32), ("num_bessel", ctypes.c_int32),
        ("num_poly_cutoff", ctypes.c_int32), ("num_layers", ctypes.c_int32),
        ("radial_hidden", ctypes.c_int32), ("radial_depth", ctypes.c_int32),
        ("layer_in_blocks", ctypes.c_int32 * 4), ("layer_hid_blocks", ctypes.c_int32 * 4),
        ("correlation", ctypes.c_int32 * 4), ("has_zbl", ctypes.c_int32), ("zbl_p", ctypes.c_int32),
        ("r_max", ctypes.c_double), ("zbl_a_exp", ctypes.c_double),
        ("zbl_a_prefactor", ctypes.c_double), ("zbl_scale", ctypes.c_double),
        ("feature_half", ctypes.c_int32), ("density_norm", ctypes.c_int32),
        ("first_nonresidual", ctypes.c_int32), ("agnesi", ctypes.c_int32),
        ("agnesi_q", ctypes.c_double), ("agnesi_p", ctypes.c_double), ("agnesi_a", ctypes.c_double),
        ("nonlinear", ctypes.c_int32), ("separate_cutoff", ctypes.c_int32),
        ("agnostic_product", ctypes.c_int32), ("layer_edge_blocks", ctypes.c_int32 * 4),
    ]


_libs: dict = {}


def load_library(path: Optional[str] = None, channels: int = 128) -> ctypes.CDLL:
    """Load (once per channel width) and type the engine library; raises if it is not built.
    ``MACE_HIP_LIB`` overrides the 128-channel library's path."""
    if path is None and channels in _libs:
        return _libs[channels]
    if channels not in LIB_PATHS:
        raise ValueError(f"no engine compiled for {channels} channels (widths {ENGINE_WIDTHS})")
    default = os.environ.get("MACE_HIP_LIB", LIB_PATHS[128]) if channels == 128 else LIB_PATHS[channels]
    p = Path(path) if path else Path(default)
    if not p.exists():
        raise ImportError(f"HIP engine library not found at {p}; build it with "
                          "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(p))
    P, I32, I64, D, U32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_double, ctypes.c_uint32
    sig = {
        "mace_create": (ctypes.c_int, [I32, ctypes.POINTER(P)]),
        "mace_destroy": (None, [P]),
        "mace_last_error": (ctypes.c_char_p, [P]),
        "mace_model_begin": (ctypes.c_int, [P, ctypes.POINTER(ModelDims)]),
        "mace_model_set_tensor": (ctypes.c_int, [P, ctypes.c_char_p, P, I64]),
        "mace_model_end": (ctypes.c_int, [P]),
        "mace_set_system": (ctypes.c_int, [P, I32, P, P, P, D]),
        "mace_step": (ctypes.c_int, [P, P, U32, ctypes.POINTER(D), P, P, P]),
        "mace_set_edges": (ctypes.c_int, [P, I64, P, P, P]),
        "mace_get_edges": (ctypes.c_int, [P, I64, P, P, P, ctypes.POINTER(I64)]),
        "mace_get_timings": (ctypes.c_int, [P, P, I32]),
        "mace_step_device": (ctypes.c_int, [P, P, U32, P]),
        "mace_step_device_noalloc": (ctypes.c_int, [P, P, U32, P]),
        "mace_sync": (ctypes.c_int, [P]),
        "mace_set_profiling": (ctypes.c_int, [P, I32]),
        "mace_set_graphs": (ctypes.c_int, [P, I32]),
        "mace_set_split_products": (ctypes.c_int, [P, I32]),
        "mace_set_fused_tp": (ctypes.c_int, [P, I32]),
        "mace_set_rebuild_w": (ctypes.c_int, [P, I32]),
        "mace_set_batch": (ctypes.c_int, [P, I32, P, P, P, P, D]),
        "mace_step_batch": (ctypes.c_int, [P, P, U32, P, P, P, P]),
        "mace_get_kernel_times": (ctypes.c_int, [P, ctypes.c_char_p, I64, P, P, I32, ctypes.POINTER(I32)]),
        "mace_get_launch_order": (ctypes.c_int, [P, ctypes.c_char_p, I64, ctypes.POINTER(I32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _libs[channels] = lib
    return lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Engine:
    """One engine context on one HIP device (not thread-safe, like the reference's
    calculator which is driven from one Python thread)."""

    def __init__(self, device: int = 0, channels: int = 128):
        """``channels``: the width of the models this context will load (a device model's
        ``dims["num_channels"]``), which selects the library compiled for it."""
        self._lib = load_library(channels=channels)
        self.channels = channels
        h = ctypes.c_void_p()
        rc = self._lib.mace_create(int(device), ctypes.byref(h))
        if rc != MACE_OK:
            msg = self._lib.mace_last_error(None)
            self._raise(rc, msg.decode() if msg else "mace_create failed")
        self._h = h
        self.n_atoms = 0

    def _raise(self, rc: int, msg: str):
        if rc in (MACE_ERR_INVALID, MACE_ERR_SPECIES):
            raise ValueError(msg)
        if rc == MACE_ERR_UNSUPPORTED:
            raise NotImplementedError(msg)
        if rc == MACE_ERR_HIP:
            raise HipError(msg)
        raise RuntimeError(msg)

    def _check(self, rc: int):
        if rc != MACE_OK:
            msg = self._lib.mace_last_error(self._h)
            self._raise(rc, msg.decode() if msg else f"error {rc}")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.mace_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- model --------------------------------------------------------------
    def load_model(self, dm) -> None:
        if int(dm.dims["num_channels"]) != self.channels:
            raise ValueError(f"a {dm.dims['num_channels']}-channel device model needs "
                             f"Engine(device, channels={dm.dims['num_channels']}); this context runs "
                             f"the {self.channels}-channel engine")
        d = ModelDims()
        for k, v in dm.dims.items():
            if isinstance(v, list):
                arr = getattr(d, k)
                for i, x in enumerate(v):
                    arr[i] = int(x)
            else:
                setattr(d, k, v)
        self._check(self._lib.mace_model_begin(self._h, ctypes.byref(d)))
        for name, t in dm.tensors.items():
            t = np.ascontiguousarray(t, dtype=np.float32)
            self._check(self._lib.mace_model_set_tensor(self._h, name.encode(), _ptr(t), t.size))
        self._check(self._lib.mace_model_end(self._h))

    # -- system -------------------------------------------------------------
    def set_system(self, species: np.ndarray, cell: np.ndarray, pbc, skin: float) -> None:
        sp = np.ascontiguousarray(species, dtype=np.int32)
        cl = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(9))
        pb = np.ascontiguousarray(np.asarray(pbc, dtype=bool).reshape(3).astype(np.uint8))
        self._check(self._lib.mace_set_system(self._h, len(sp), _ptr(sp), _ptr(cl), _ptr(pb), float(skin)))
        self.n_atoms = len(sp)
        self.batch_sizes = np.array([len(sp)], dtype=np.int32)

    def step(self, positions: np.ndarray, stress: bool = False, force_nl: bool = False,
             node_energy: bool = True) -> Tuple[float, Optional[np.ndarray], np.ndarray, Optional[np.ndarray]]:
        pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
        if len(pos) != self.n_atoms:
            raise ValueError(f"positions has {len(pos)} atoms, system has {self.n_atoms}")
        e = ctypes.c_double()
        ne = np.empty(self.n_atoms, dtype=np.float64) if node_energy else None
        f = np.empty((self.n_atoms, 3), dtype=np.float64)
        v = np.empty((3, 3), dtype=np.float64) if stress else None
        flags = STEP_FORCES | (STEP_STRESS if stress else 0) | (STEP_FORCE_NL if force_nl else 0)
        self._check(self._lib.mace_step(self._h, _ptr(pos), flags, ctypes.byref(e), _ptr(ne), _ptr(f), _ptr(v)))
        return e.value, ne, f, v

    # -- batches of structures (model.py:440-484 with `batch`, utils.py:35-44) ---
    def set_batch(self, species_list, cells, pbcs, skin: float) -> None:
        """Structures g = 0..G-1 (species arrays, 3x3 cells, pbc triples) evaluated together."""
        sizes = np.array([len(sp) for sp in species_list], dtype=np.int32)
        if len(sizes) == 0:
            raise ValueError("empty batch")
        sp = np.ascontiguousarray(np.concatenate([np.asarray(x, dtype=np.int32).reshape(-1) for x in species_list]),
                                  dtype=np.int32)
        cl = np.ascontiguousarray(np.asarray(cells, dtype=np.float64).reshape(len(sizes), 9))
        pb = np.ascontiguousarray(np.asarray(pbcs, dtype=bool).reshape(len(sizes), 3).astype(np.uint8))
        self._check(self._lib.mace_set_batch(self._h, len(sizes), _ptr(sizes), _ptr(sp), _ptr(cl), _ptr(pb),
                                             float(skin)))
        self.n_atoms = int(sizes.sum())
        self.batch_sizes = sizes

    def step_batch(self, positions, stress: bool = False, force_nl: bool = False):
        """(energies [G], node_energy [N], forces [N, 3], virials [G, 3, 3] or None) of the batch;
        ``positions`` are the structures' positions concatenated in batch order."""
        pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
        if len(pos) != self.n_atoms:
            raise ValueError(f"positions has {len(pos)} atoms, batch has {self.n_atoms}")
        G = len(self.batch_sizes)
        eg = np.empty(G, dtype=np.float64)
        ne = np.empty(self.n_atoms, dtype=np.float64)
        f = np.empty((self.n_atoms, 3), dtype=np.float64)
        v = np.empty((G, 3, 3), dtype=np.float64) if stress else None
        flags = STEP_FORCES | (STEP_STRESS if stress else 0) | (STEP_FORCE_NL if force_nl else 0)
        self._check(self._lib.mace_step_batch(self._h, _ptr(pos), flags, _ptr(eg), _ptr(ne), _ptr(f), _ptr(v)))
        return eg, ne, f, v

    # -- test hooks -----------------------------------------------------------
    def set_edges(self, sender, receiver, shifts) -> None:
        s = np.ascontiguousarray(sender, dtype=np.int32)
        r = np.ascontiguousarray(receiver, dtype=np.int32)
        S = np.ascontiguousarray(np.asarray(shifts).reshape(-1, 3), dtype=np.int32)
        if not (len(s) == len(r) == len(S)):
            raise ValueError("sender / receiver / shifts lengths differ")
        self._check(self._lib.mace_set_edges(self._h, len(s), _ptr(s), _ptr(r), _ptr(S)))

    def num_edges(self) -> int:
        """Edge count of the current list (mace_get_edges without arrays)."""
        n = ctypes.c_int64()
        self._check(self._lib.mace_get_edges(self._h, 0, None, None, None, ctypes.byref(n)))
        return n.value

    def get_edges(self):
        n = ctypes.c_int64()
        self._check(self._lib.mace_get_edges(self._h, 0, None, None, None, ctypes.byref(n)))
        E = n.value
        s = np.empty(E, np.int32)
        r = np.empty(E, np.int32)
        S = np.empty((E, 3), np.int32)
        self._check(self._lib.mace_get_edges(self._h, E, _ptr(s), _ptr(r), _ptr(S), ctypes.byref(n)))
        return s, r, S

    def step_device(self, d_positions: int, d_out: int, stress: bool = False, force_nl: bool = False,
                    skin_check: bool = False) -> None:
        """Queue one step on device buffers (raw device addresses); see mace_step_device.
        ``skin_check``: the engine applies the skin criterion itself (one synchronisation)."""
        flags = (STEP_FORCES | (STEP_STRESS if stress else 0) | (STEP_FORCE_NL if force_nl else 0)
                 | (STEP_SKIN_CHECK if skin_check else 0))
        self._check(self._lib.mace_step_device(self._h, ctypes.c_void_p(d_positions), flags,
                                               ctypes.c_void_p(d_out)))

    def step_device_noalloc(self, d_positions: int, d_out: int, stress: bool = False) -> None:
        """mace_step_device without any device allocation (see mace_step_device_noalloc):
        needs a neighbour list built by a previous step; launches eagerly."""
        flags = STEP_FORCES | (STEP_STRESS if stress else 0)
        self._check(self._lib.mace_step_device_noalloc(self._h, ctypes.c_void_p(d_positions), flags,
                                                       ctypes.c_void_p(d_out)))

    def sync(self) -> None:
        self._check(self._lib.mace_sync(self._h))

    def set_profiling(self, enable: bool) -> None:
        self._check(self._lib.mace_set_profiling(self._h, int(bool(enable))))

    def set_graphs(self, enable: bool) -> None:
        """Replay steps through captured HIP graphs (default) or launch them eagerly."""
        self._check(self._lib.mace_set_graphs(self._h, int(bool(enable))))

    def set_split_products(self, enable: bool) -> None:
        """Float32 policy: matrix products (radial-MLP output layer, node linears) on fp16 matrix
        cores with split operands (default) or on fp32 matrix cores."""
        self._check(self._lib.mace_set_split_products(self._h, int(bool(enable))))

    def set_fused_tp(self, enable: bool) -> None:
        """With split products: radial-MLP output layer built inside the tensor-product kernels
        (default) or in a separate pass."""
        self._check(self._lib.mace_set_fused_tp(self._h, int(bool(enable))))

    def set_rebuild_w(self, enable: bool) -> None:
        """Half-precision feature policies: the tensor-product VJP rebuilds the per-edge weights
        from the radial MLP's hidden layer (default) instead of reading them back."""
        self._check(self._lib.mace_set_rebuild_w(self._h, int(bool(enable))))

    def kernel_times(self) -> dict:
        """{site: (total_ms, launches)} accumulated since the last call."""
        n = ctypes.c_int32()
        self._check(self._lib.mace_get_kernel_times(self._h, None, 0, None, None, 0, ctypes.byref(n)))
        cap = n.value
        buf = ctypes.create_string_buffer(64 * max(cap, 1) + 1)
        tot = np.zeros(max(cap, 1), np.float64)
        cnt = np.zeros(max(cap, 1), np.int64)
        self._check(self._lib.mace_get_kernel_times(self._h, buf, len(buf), _ptr(tot), _ptr(cnt), cap,
                                                    ctypes.byref(n)))
        names = buf.value.decode().split("\n")[:cap]
        return {nm: (float(tot[i]), int(cnt[i])) for i, nm in enumerate(names)}

    def launch_order(self) -> list:
        """Launch site of every kernel dispatch of the last profiled step, in order."""
        n = ctypes.c_int32()
        self._check(self._lib.mace_get_launch_order(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(64 * max(n.value, 1) + 1)
        self._check(self._lib.mace_get_launch_order(self._h, buf, len(buf), ctypes.byref(n)))
        return buf.value.decode().split("\n")[:n.value]

    def timings(self) -> np.ndarray:
        out = np.zeros(4, dtype=np.float64)
        self._lib.mace_get_timings(self._h, _ptr(out), 4)
        return out
