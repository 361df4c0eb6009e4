"""Tuning file: launch-shape choices measured on the GPU in use.

The reference keeps a JSON file of per-kernel threadgroup sizes, read at
import from ``mhc_tuning.json`` (working directory) and
``~/.cache/mhc-mlx/tuning.json`` and queried with ``_get_tuned_tpg``
(mhc_mlx/metal.py:21-36); ``scripts/tune.py`` writes it (tune.py:50-103).

Here the same files are read the same way.  libmhc_hip chooses its
launch shapes itself and exposes its tunable choices as named integer
knobs (``MHC_RES_GRID`` and so on; the tuned ones are listed in ``KNOBS``),
held in a process-wide table inside the library (``mhc_set_knob``).  Each
knob starts from the environment variable of the same name, read once when
the library loads.  A tuning entry of this library maps an op name to the
values of its knobs::

    {"residual_add_agg": {"MHC_RES_GRID": -1}, "sinkhorn_16": {"MHC_SK16_CPL": 4}}

Keys starting with ``_`` hold metadata (device, timings).
``load()`` (run at import) sets such values in the library's table, except
for knobs whose environment variable is set, so an explicit setting always
wins; the environment itself is never written.  Integer entries written for
the reference (Metal threadgroup sizes) are kept for ``_get_tuned_tpg`` and
otherwise ignored.  ``python -m mhc_mlx_amd.tune`` measures the candidates
and writes the file.
"""

from __future__ import annotations

import json
import os

from . import _lib

__all__ = ["KNOBS", "CONFIG_PATHS", "load", "apply", "tuning_config", "_get_tuned_tpg"]

CONFIG_PATHS = [
    "mhc_tuning.json",
    os.path.join(os.path.expanduser("~"), ".cache", "mhc-mlx", "tuning.json"),
]

# op name -> (knob name, candidate values).  The first candidate is the
# library's built-in choice.
KNOBS: dict[str, tuple[str, list[int]]] = {
    # workgroups per CU of the residual add + aggregate grid (-1: one item per thread)
    "residual_add_agg": ("MHC_RES_GRID", [-1, 4, 8, 16]),
    # workgroups per CU of the stream mix + add (post-combine) kernels
    "stream_mix_add": ("MHC_MIX_FWD_GRID", [8, 16, 32, -1]),
    "stream_mix_add_bwd": ("MHC_MIX_BWD_GRID", [8, 4, 16]),
    # workgroups per CU of the MHCRewire pre-scale kernels
    "stream_scale": ("MHC_SCALE_FWD_GRID", [8, 16, 32, -1]),
    "stream_scale_bwd": ("MHC_SCALE_BWD_GRID", [8, 4, 16]),
    # 128-channel slabs per wave of the n = 16 MFMA kernels
    "mhc_fused_n16": ("MHC_FWD_SPW", [2, 1]),
    "mhc_fused_bwd_n16": ("MHC_BWD_SPW", [2, 1]),
    # batched n = 16 Sinkhorn layout: 0 the 4 x 4-block layout (16 lanes per matrix), 4 / 2 columns per lane
    "sinkhorn_16": ("MHC_SK16_CPL", [0, 4, 2]),
    # 8-channel chunks per thread of the layer-wide n <= 8 forward (1 unless C needs 2)
    "mhc_fused": ("MHC_FWD_CH", [1, 2]),
    # persistent workgroups of the layer-wide backward (0: the library's choice)
    "mhc_fused_bwd": ("MHC_BWD_GRID", [0, 512, 1024]),
}

_ENV_NAMES = {env for env, _ in KNOBS.values()}
_TUNING_CONFIG: dict = {}


def tuning_config() -> dict:
    """The merged contents of the tuning files read so far."""
    return dict(_TUNING_CONFIG)


def apply(config: dict, override: bool = False) -> dict:
    """Set the knob values of `config` ({op: {KNOB: value}}) in the library; returns what was set.

    A knob whose environment variable is set is left alone unless `override`
    is true.  Unknown names and non-integer values raise ValueError before
    anything is set, so a corrupt file cannot pass silently or apply in part.
    """
    values = {}
    for op, entry in config.items():
        if op.startswith("_") or not isinstance(entry, dict):
            continue  # metadata, or a reference-format threadgroup size
        for env, value in entry.items():
            if env not in _ENV_NAMES:
                raise ValueError(f"tuning entry {op!r}: unknown knob {env!r}")
            if isinstance(value, bool) or not isinstance(value, int):
                raise ValueError(f"tuning entry {op!r}: {env} must be an integer, got {value!r}")
            values[env] = value
    # all entries are valid: set them
    done = {}
    for env, value in values.items():
        if override or env not in os.environ:
            _lib.set_knob(env, value)
            done[env] = value
    return done


def load(paths: list[str] | None = None) -> dict:
    """Read the tuning files (later files update earlier ones, as metal.py:28-33) and apply them.

    Unreadable files are skipped, as the reference does; invalid knob entries
    are reported with a warning and not applied.
    """
    merged = {}
    for path in paths if paths is not None else CONFIG_PATHS:
        if not os.path.exists(path):
            continue
        try:
            with open(path) as f:
                data = json.load(f)
        except (OSError, ValueError):
            continue
        if isinstance(data, dict):
            merged.update(data)
    _TUNING_CONFIG.update(merged)
    try:
        apply(merged)
    except ValueError as e:
        import warnings

        warnings.warn(f"mhc_mlx_amd: tuning file not applied: {e}")
    return merged


def _get_tuned_tpg(kernel_name: str, default: int) -> int:
    """metal.py:35-36: the tuned threadgroup size of a kernel, or `default`."""
    v = _TUNING_CONFIG.get(kernel_name, default)
    return v if isinstance(v, int) and not isinstance(v, bool) else default
