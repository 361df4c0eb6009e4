"""ctypes binding of libmhc_hip.so (declared in include/mhc_hip.h).

The library is loaded once, from this package directory.  There is no
fallback: if the library is missing or fails to load, every accelerated op
raises RuntimeError naming the path and the build command.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmhc_hip.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

H_NONE = 0
H_ACTIVATED = 1
H_RAW = 2

MAX_N = 64

_VP = ctypes.c_void_p
_I32 = ctypes.c_int
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t
_PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> (argtypes, restype); must list exactly the functions of mhc_hip.h
SIGNATURES = {
    "mhc_abi_version": ([], _I32),
    "mhc_last_error": ([], ctypes.c_char_p),
    "mhc_knob_count": ([], _I32),
    "mhc_knob_name": ([_I32], ctypes.c_char_p),
    "mhc_set_knob": ([ctypes.c_char_p, _I32], _I32),
    "mhc_unset_knob": ([ctypes.c_char_p], _I32),
    "mhc_get_knob": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)], _I32),
    "mhc_sinkhorn_fwd": ([_VP, _VP, _I64, _I32, _I32, _F32, _VP], _I32),
    "mhc_sinkhorn_bwd_workspace_bytes": ([_I64, _I32, _I32], _SZ),
    "mhc_sinkhorn_bwd": ([_VP, _VP, _VP, _I64, _I32, _I32, _F32, _VP, _SZ, _VP], _I32),
    "mhc_sinkhorn_state_bytes": ([_I64, _I32, _I32], _SZ),
    "mhc_sinkhorn_fwd_record": ([_VP, _VP, _VP, _SZ, _I64, _I32, _I32, _F32, _VP], _I32),
    "mhc_sinkhorn_bwd_recorded": ([_VP, _VP, _VP, _VP, _SZ, _I64, _I32, _I32, _F32, _VP], _I32),
    "mhc_fused_fwd": ([_VP, _I32, _VP, _I64, _VP, _VP, _I64, _I32, _VP, _VP, _I32, _VP, _I64, _I32,
                       _I32, _F32, _VP], _I32),
    "mhc_fused_bwd_workspace_bytes": ([_I64, _I32, _I32, _I32], _SZ),
    "mhc_fused_bwd_partials": ([_VP, _I32, _VP, _I32, _VP, _I64, _VP, _VP, _I64, _I32, _VP, _VP, _I32,
                                _VP, _VP, _VP, _VP, _SZ, _I64, _I32, _I32, _F32, _PI64, _VP], _I32),
    "mhc_reduce_param_grads": ([_VP, _SZ, _I64, _I32, _I32, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP,
                                _VP], _I32),
    "mhc_fused_bwd": ([_VP, _I32, _VP, _I32, _VP, _I64, _VP, _VP, _I64, _I32, _VP, _VP, _I32, _VP, _VP,
                       _VP, _VP, _VP, _SZ, _I64, _I32, _I32, _F32, _VP], _I32),
    "mhc_layer_fwd": ([_VP, _I32, _VP, _VP, _VP, _VP, _VP, _I32, _VP, _I64, _I32, _I32, _I32, _I32, _F32, _VP],
                      _I32),
    "mhc_layer_bwd_workspace_bytes": ([_I64, _I32, _I32, _I32, _I32], _SZ),
    "mhc_layer_bwd": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _I64,
                       _I32, _I32, _I32, _I32, _F32, _VP], _I32),
    "mhc_layer_bwd_noalloc": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I32,
                               _I32, _I32, _I32, _F32, _VP], _I32),
    "mhc_layer_bwd_reduce": ([_VP, _SZ, _I64, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I32, _I32, _I32, _I32,
                              _F32, _VP], _I32),
    "mhc_stream_mix_add_fwd": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP, _I32, _VP, _I32, _I64, _I32, _I32,
                                _VP], _I32),
    "mhc_stream_mix_add_bwd_workspace_bytes": ([_I64, _I32, _I32], _SZ),
    "mhc_stream_mix_add_bwd": ([_VP, _I32, _VP, _I32, _VP, _I32, _VP, _VP, _VP, _I32, _VP, _I32, _VP,
                                _I32, _VP, _VP, _VP, _VP, _SZ, _I64, _I32, _I32, _VP], _I32),
    "mhc_stream_scale_fwd": ([_VP, _I32, _VP, _I32, _VP, _I32, _I64, _I32, _I32, _VP], _I32),
    "mhc_stream_scale_bwd_workspace_bytes": ([_I64, _I32, _I32], _SZ),
    "mhc_stream_scale_bwd": ([_VP, _I32, _VP, _I32, _VP, _I32, _VP, _VP, _I32, _VP, _VP, _SZ, _I64,
                              _I32, _I32, _VP], _I32),
    "mhc_residual_add_agg_fwd": ([_VP, _VP, _I32, _VP, _I32, _VP, _I32, _VP, _I64, _I32, _I32, _VP], _I32),
    "mhc_residual_add_agg_bwd_workspace_bytes": ([_I64, _I32, _I32], _SZ),
    "mhc_residual_add_agg_bwd": ([_VP, _VP, _I32, _VP, _I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _SZ, _I64,
                                  _I32, _I32, _VP], _I32),
}

_lock = threading.Lock()
_lib = None
# knob settings made before the library is loaded: name -> value (None: unset)
_pending_knobs: dict[str, int | None] = {}


class MHCError(RuntimeError):
    """A HIP runtime failure reported by libmhc_hip (positive hipError_t)."""


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load libmhc_hip.so (once) and bind every signature; raise RuntimeError if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"libmhc_hip.so not found at {p}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)"
            )
        # RTLD_GLOBAL: the torch binding (_mhc_torch.so) resolves its C-ABI calls against this library
        lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.mhc_abi_version() != 1:
            raise RuntimeError(f"{p}: unexpected ABI version {lib.mhc_abi_version()}")
        if path is None:
            for name, value in _pending_knobs.items():
                rc = lib.mhc_unset_knob(name.encode()) if value is None else lib.mhc_set_knob(name.encode(), value)
                if rc != 0:
                    raise ValueError(f"knob {name}: {lib.mhc_last_error().decode()}")
            _pending_knobs.clear()
            _lib = lib
        return lib


def knob_names() -> list[str]:
    """Names of the library's launch-shape knobs (mhc_knob_name)."""
    lib = load()
    return [lib.mhc_knob_name(i).decode() for i in range(lib.mhc_knob_count())]


def set_knob(name: str, value: int | None) -> None:
    """Set a launch-shape knob (None: back to the library's own choice).

    Applied at once when the library is loaded, else when it loads.
    """
    if value is not None and (isinstance(value, bool) or not isinstance(value, int)):
        raise ValueError(f"knob {name} must be an integer, got {value!r}")
    with _lock:
        if _lib is None:
            _pending_knobs[name] = value
            return
    if value is None:
        check(_lib.mhc_unset_knob(name.encode()), f"mhc_unset_knob({name})")
    else:
        check(_lib.mhc_set_knob(name.encode(), int(value)), f"mhc_set_knob({name})")


def get_knob(name: str) -> int | None:
    """A knob's value, or None while it is unset (the library's own choice)."""
    with _lock:
        if _lib is None and name in _pending_knobs:
            return _pending_knobs[name]
    lib = load()
    v = ctypes.c_int(0)
    rc = lib.mhc_get_knob(name.encode(), ctypes.byref(v))
    check(min(rc, 0), f"mhc_get_knob({name})")
    return v.value if rc == 1 else None


def last_error() -> str:
    msg = load().mhc_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Translate a library status into ValueError (bad argument) / MHCError (HIP)."""
    if rc == 0:
        return
    msg = last_error()
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise MHCError(f"{what}: HIP error {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
