"""The torch binding of libmhc_hip (``_mhc_torch.so``, built from csrc/torch_ext.cpp).

It holds MHCLayer's forward and backward as a C++ autograd Function over the
same C ABI that ops.py calls through ctypes, so the small-batch path makes
the fewest host steps and the backward runs without Python.  Loaded once,
from this package directory, after libmhc_hip.so (whose symbols it uses).
Like the library, it must be present where a GPU is: a missing build raises
RuntimeError naming the build command.
"""

from __future__ import annotations

import importlib.util
import threading
from pathlib import Path

from . import _lib

EXT_PATH = Path(__file__).resolve().parent / "_mhc_torch.so"

_mod = None
_lock = threading.Lock()


def load():
    """The binding's module (loaded once); raises RuntimeError if it is not built."""
    global _mod
    if _mod is not None:
        return _mod
    with _lock:
        if _mod is None:
            _lib.load()
            if not EXT_PATH.exists():
                raise RuntimeError(
                    f"{EXT_PATH.name} not found at {EXT_PATH}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'`"
                )
            spec = importlib.util.spec_from_file_location("mhc_mlx_amd._mhc_torch", EXT_PATH)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _mod = mod
    return _mod
