"""MI355X-native MACE energy / forces / stress engine with the mace-mlx ASE API.

Public names mirror `mace_mlx/__init__.py`: ``MACECalculator``, ``mace_mp``,
``mace_off``, ``load_model`` (here: returns the parsed config and weights).
"""

from .calculators import MACECalculator, MACEHIPCalculator, mace_anicc, mace_mp, mace_off, mace_omol
from .model_io import ModelConfig, load_config, load_weights


def load_model(model_dir: str, dtype: str = "float32"):
    """Read a reference-format model directory: (ModelConfig, weights dict), the weights rounded
    as a model of ``dtype`` ("float32", "float16", "bfloat16") holds them (`model.py:664-720`)."""
    from .device_model import FEATURE_POLICY, round_weights
    if dtype not in FEATURE_POLICY:
        raise ValueError(f"dtype={dtype!r}: expected one of {sorted(FEATURE_POLICY)}")
    return load_config(model_dir), round_weights(load_weights(model_dir), dtype)


__all__ = ["MACECalculator", "MACEHIPCalculator", "mace_mp", "mace_off", "mace_anicc", "mace_omol",
           "load_model", "ModelConfig"]
