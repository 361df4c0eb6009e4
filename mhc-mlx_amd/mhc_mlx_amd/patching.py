"""AutoPatcher: wrap the square Linear layers of a torch model in MHCRewire
(mhc_mlx/patching.py:5-126, for MLX models there).

Rules (patching.py:84-126): a module is rewired when it is a Linear (or a
quantized Linear) whose input and output widths are equal and divisible by
``n_streams``.  Every candidate is found from one snapshot of
``model.named_modules()`` taken before any replacement (patching.py:27), the
root module itself is never replaced, and each replacement is installed on
its parent under the same attribute name — which for ``nn.Sequential`` /
``nn.ModuleList`` is the index and for ``nn.ModuleDict`` the key.

Differences from the MLX version, each forced by torch or chosen for safety:

* torch registers only ``nn.Module`` containers, so plain Python lists and
  dicts of layers (which MLX traverses) are not visited; ``nn.ModuleList`` /
  ``nn.ModuleDict`` are their torch form and are handled.
* the MHCRewire parameters are created on the wrapped layer's device (MLX has
  one unified memory; torch does not).
* a module that is already the ``inner`` of an MHCRewire is skipped, so
  patching twice does not wrap a layer twice.
* extra keyword arguments are passed to each MHCRewire (hence MHCLayer):
  ``sinkhorn_iters``, ``eps``, ``use_metal`` and so on.
* a layer with half-precision weights gets ``return_dtype`` equal to that
  type unless the caller sets it: MLX promotes the fp32 MHCRewire output
  through the rest of the model, while a torch half-precision Linear
  rejects an fp32 input.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .layer import MHCRewire

__all__ = ["AutoPatcher"]


def _quantized_linear_types() -> tuple:
    types = []
    try:
        import torch.ao.nn.quantized as nnq
        import torch.ao.nn.quantized.dynamic as nnqd

        types += [nnq.Linear, nnqd.Linear]
    except Exception:  # pragma: no cover - torch builds without the quantized modules
        pass
    return tuple(types)


_QUANTIZED = _quantized_linear_types()


def _module_device_dtype(module: nn.Module):
    for t in list(module.parameters(recurse=False)) + list(module.buffers(recurse=False)):
        return t.device, t.dtype
    return None, None


class AutoPatcher:
    """Automatic patching utility that injects mHC into existing torch models.

    It traverses the model and wraps suitable Linear / quantized Linear layers
    with MHCRewire (patching.py:5-11).
    """

    @staticmethod
    def patch(model: nn.Module, n_streams: int = 32, verbose: bool = True, **mhc_kwargs) -> int:
        """Rewire the model in place (patching.py:13-82); returns the number of layers patched."""
        count = 0
        modules = list(model.named_modules())
        inner_ids = {id(m.inner) for _, m in modules if isinstance(m, MHCRewire)}
        for name, module in modules:
            if name == "":
                continue
            if id(module) in inner_ids or isinstance(module, MHCRewire):
                continue
            if not AutoPatcher._is_patchable(module, n_streams):
                continue
            parent_path, _, child_name = name.rpartition(".")
            parent = model.get_submodule(parent_path) if parent_path else model
            dims = AutoPatcher._get_dims(module)
            if verbose:
                print(f"[AutoPatcher] Rewiring {name} (dims={dims}, streams={n_streams})")
            kwargs = dict(mhc_kwargs)
            dev, dt = _module_device_dtype(module)
            if dev is not None and "device" not in kwargs:
                kwargs["device"] = dev
            if dt in (torch.float16, torch.bfloat16) and "return_dtype" not in kwargs:
                kwargs["return_dtype"] = dt
            wrapped = MHCRewire(module, dims=dims, n=n_streams, **kwargs)
            setattr(parent, child_name, wrapped)
            count += 1
        if verbose:
            print(f"[AutoPatcher] Patched {count} layers.")
        return count

    @staticmethod
    def _get_dims(module: nn.Module) -> int:
        """Input width of a Linear ([out, in] weight) or quantized Linear (patching.py:84-95)."""
        if isinstance(module, nn.Linear):
            return int(module.weight.shape[1])
        if _QUANTIZED and isinstance(module, _QUANTIZED):
            return int(module.in_features)
        return 0

    @staticmethod
    def _is_patchable(module: nn.Module, n: int) -> bool:
        """patching.py:97-126: Linear / quantized Linear, in == out, in % n == 0."""
        is_linear = isinstance(module, nn.Linear)
        is_quant = bool(_QUANTIZED) and isinstance(module, _QUANTIZED)
        if not (is_linear or is_quant):
            return False
        if is_linear:
            if isinstance(module.weight, nn.parameter.UninitializedParameter):
                return False
            in_dims, out_dims = int(module.weight.shape[1]), int(module.weight.shape[0])
        else:
            in_dims, out_dims = int(module.in_features), int(module.out_features)
        if in_dims == 0 or out_dims == 0:
            return False
        # mHC relies on the residual form x + f(x): the width must be preserved
        if in_dims != out_dims:
            return False
        return in_dims % n == 0
