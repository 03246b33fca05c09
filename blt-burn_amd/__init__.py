"""blt_burn_amd — MI355X (gfx950) entropy-patching path of blt-burn.

Host mirror of the reference's fused_ops / patcher / model API over the C ABI
of libblt_hip.so (include/blt_hip.h).  Import-time work is limited to Python;
the library is loaded on first use and a missing build raises BltError.
"""
from ._lib import BltError, LIB_PATH, lib, last_error  # noqa: F401
from . import mpk_io, safetensors_io, synth, tokenizer  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    # torch-dependent submodules load lazily so synth/_lib work without torch
    import importlib
    if name in ("fused_ops", "patcher", "model", "ingest", "pipeline"):
        return importlib.import_module("." + name, __name__)
    raise AttributeError(name)
