"""MI355X (gfx950) backend for the raviadi12/directcompute_torch ``nn_engine`` API.

``directcompute_torch_amd.nn_engine`` is the drop-in module (it initialises the
HIP device on import).  This package ``__init__`` touches no device so that
building and symbol checks work on machines without a GPU.
"""
import os as _os

PKG_DIR = _os.path.dirname(_os.path.abspath(__file__))
LIB_PATH = _os.path.join(PKG_DIR, "libdcengine.so")
__all__ = ["PKG_DIR", "LIB_PATH"]
