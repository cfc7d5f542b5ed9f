"""MI355X-native MACE energy / forces / stress engine with the mace-mlx ASE API.

Public names mirror `mace_mlx/__init__.py`: ``MACECalculator``, ``mace_mp``,
``mace_off``, ``load_model`` (here: returns the parsed config and weights).
"""

from .calculators import MACECalculator, MACEHIPCalculator, mace_anicc, mace_mp, mace_off, mace_omol
from .model_io import ModelConfig, load_config, load_weights


def load_model(model_dir: str):
    """Read a reference-format model directory: (ModelConfig, weights dict)."""
    return load_config(model_dir), load_weights(model_dir)


__all__ = ["MACECalculator", "MACEHIPCalculator", "mace_mp", "mace_off", "mace_anicc", "mace_omol",
           "load_model", "ModelConfig"]
