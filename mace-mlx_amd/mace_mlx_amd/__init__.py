"""MI355X-native MACE energy / forces / stress engine with the mace-mlx ASE API.

Public names mirror `mace_mlx/__init__.py`: ``MACECalculator``, ``mace_mp``,
``mace_off``, ``load_model`` (a callable ``MACE`` / ``ScaleShiftMACE`` on the GPU).
"""

from .calculators import MACECalculator, MACEHIPCalculator, mace_anicc, mace_mp, mace_off, mace_omol
from .model import MACE, ScaleShiftMACE, load_model
from .model_io import ModelConfig, load_config, load_weights

__all__ = ["MACECalculator", "MACEHIPCalculator", "mace_mp", "mace_off", "mace_anicc", "mace_omol",
           "load_model", "MACE", "ScaleShiftMACE", "ModelConfig"]
