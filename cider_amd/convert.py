"""cider_amd.convert - in-place conversion of a model's Linear layers to
``CiderLinear`` (drop-in for ``cider/convert.py``).

``convert_model`` walks the module tree and replaces every ``torch.nn.Linear``
and every affine-quantized linear (``cider_amd.ingest.QuantizedLinear``, or
any module with ``weight``, ``scales``, ``group_size`` and ``bits``, the
tensors of MLX's ``nn.QuantizedLinear``) by ``CiderLinear.from_float``
(``cider/convert.py:25,28-47,50-99``).  Like the
reference it converts every Linear it finds; ``exclude`` (an addition) names
child modules to keep in floating point, e.g. ``exclude=("lm_head",)``.
It raises ``RuntimeError`` when the HIP extension or an MI355X is missing
(``cider/convert.py:71-74``).
"""

from __future__ import annotations

import gc
import time
from typing import Iterable, Optional

import torch

from . import ops
from .ingest import QuantizedLinear, is_affine_quantized
from .nn import CiderLinear

_TARGET_TYPES = (torch.nn.Linear, QuantizedLinear)


def _is_target(child) -> bool:
    return isinstance(child, _TARGET_TYPES) or (
        isinstance(child, torch.nn.Module) and not isinstance(child, CiderLinear)
        and is_affine_quantized(child))


def _convert_children(module: torch.nn.Module, counter, exclude, group_size, prefix=""):
    for name, child in list(module.named_children()):
        full = f"{prefix}{name}"
        if name in exclude or full in exclude:
            continue
        if _is_target(child):
            setattr(module, name, CiderLinear.from_float(child, target_group_size=group_size))
            counter[0] += 1
            if counter[0] % 28 == 0:
                gc.collect()
        else:
            _convert_children(child, counter, exclude, group_size, prefix=f"{full}.")


def convert_model(model: torch.nn.Module, *, verbose: bool = True,
                  exclude: Optional[Iterable[str]] = None,
                  group_size: Optional[int] = None) -> dict:
    """Replace all ``torch.nn.Linear`` and affine-quantized linear layers by
    ``CiderLinear`` in place.

    Returns ``{"n_converted": n, "elapsed_s": t}`` (``cider/convert.py:86-99``).
    ``group_size`` (an addition) is passed to ``CiderLinear.from_float`` as
    ``target_group_size``.  None, the default, is the reference's conversion
    (``cider/convert.py:32``): ``torch.nn.Linear`` layers become per-channel,
    and 8-bit affine layers with group size 64/128/256 keep that group size
    (``cider/nn.py:134-139``).  0 forces per-channel, 64/128/256 per-group.
    """
    if not ops.is_available():
        raise RuntimeError(
            "W8A8 INT8 kernels not available: cider_amd needs its HIP extension and an "
            "MI355X (gfx950) GPU.")
    t0 = time.perf_counter()
    counter = [0]
    _convert_children(model, counter, set(exclude or ()), group_size)
    elapsed = time.perf_counter() - t0
    stats = {"n_converted": counter[0], "elapsed_s": elapsed}
    if verbose:
        print(f"[cider] Converted {counter[0]} layers to CiderLinear in {elapsed:.1f}s")
    return stats
