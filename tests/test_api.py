"""Calculator API surface and argument errors (no GPU needed: these raise before
an engine context is created), mirroring `calculators.py:87-136,566-637`."""

import inspect
import warnings

import pytest

import mace_mlx_amd
from mace_mlx_amd import calculators as calc


def test_public_names():
    for name in ("MACECalculator", "mace_mp", "mace_off", "load_model"):
        assert hasattr(mace_mlx_amd, name)
    assert mace_mlx_amd.MACECalculator is calc.MACEHIPCalculator
    assert calc.MACEHIPCalculator.implemented_properties == [
        "energy", "energies", "free_energy", "node_energy", "forces", "stress"]


def test_signatures_match_reference():
    sig = inspect.signature(calc.MACEHIPCalculator.__init__)
    assert list(sig.parameters)[1:7] == ["model_path", "device", "default_dtype", "head", "skin", "use_compile"]
    assert sig.parameters["skin"].default == 0.5
    sig = inspect.signature(calc.mace_mp)
    assert list(sig.parameters)[:6] == ["model", "device", "default_dtype", "head", "dispersion", "return_raw_model"]


def test_argument_errors():
    with pytest.raises(NotImplementedError):
        calc.MACEHIPCalculator(model_paths=["a", "b"])
    with pytest.raises(NotImplementedError):
        calc.mace_mp(return_raw_model=True)
    with pytest.raises(NotImplementedError):
        calc.MACEHIPCalculator(model_path="x", device="cpu")
    with pytest.raises(NotImplementedError):
        calc.MACEHIPCalculator(model_path="x", default_dtype="float8")
    with pytest.raises(NotImplementedError):
        calc.mace_anicc()
    with pytest.raises(NotImplementedError):
        calc.mace_omol()


def test_model_resolution(tmp_path, monkeypatch):
    monkeypatch.setenv("MACE_MLX_CACHE_DIR", str(tmp_path))
    with pytest.raises(FileNotFoundError):
        calc.MACEHIPCalculator._resolve_model(str(tmp_path / "missing"))
    with pytest.raises(ImportError):
        calc.MACEHIPCalculator._resolve_model("small")
    d = tmp_path / "small" / "v2"
    d.mkdir(parents=True)
    (d / "config.json").write_text("{}")
    (d / "weights.npz").write_bytes(b"")
    assert calc.MACEHIPCalculator._resolve_model("small") == str(d)


def test_float64_warns_then_requires_model():
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        with pytest.raises(FileNotFoundError):
            calc.MACEHIPCalculator(model_path="/nonexistent/dir", default_dtype="float64")
    assert any("float32" in str(r.message) for r in rec)


def test_load_model_surface(tmp_path):
    """`model.py:664-720`: load_model(model_dir, dtype) returns a MACE or ScaleShiftMACE object
    (ScaleShiftMACE when config.json names no model_type); a bad dtype raises before any GPU
    work, and the call signature follows `MACE.__call__` (`model.py:440-449`)."""
    from mace_mlx_amd import model as mm
    assert mace_mlx_amd.load_model is mm.load_model
    assert issubclass(mm.ScaleShiftMACE, mm.MACE)
    sig = inspect.signature(mm.MACE.__call__)
    assert list(sig.parameters)[1:] == ["positions", "node_attrs", "edge_index", "shifts", "cell", "batch",
                                         "num_graphs"]
    assert sig.parameters["num_graphs"].default == 1
    with pytest.raises(ValueError):
        mace_mlx_amd.load_model(str(tmp_path), dtype="float8")
