"""schedforge_amd -- MI355X (gfx950) execution backend for SchedForge's compiled
decoder layer.  The compute path is libsfg_hip.so (include/sfg_hip.h); this
package binds it and mirrors the reference's DecoderCompiler /
execute_decoder_layer boundary for Python callers."""
from ._abi import load, SfgError, SfgInvalidArgument  # noqa: F401
from .configs import CONFIGS, CONFIG_SEEDS, DecoderConfig, algorithmic_work  # noqa: F401

__all__ = ["load", "SfgError", "SfgInvalidArgument", "CONFIGS", "CONFIG_SEEDS", "DecoderConfig",
           "algorithmic_work", "layer"]


def __getattr__(name):
    # torch-dependent parts load lazily so the ABI binding imports without torch
    if name == "layer":
        from . import layer
        return layer
    raise AttributeError(name)
