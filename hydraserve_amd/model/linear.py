"""The runtime's linear-layer dispatch and projection fusion helpers.

Mirrors the static methods of QwenTextRuntime that sit directly on the
quantized path:

* ``linear``                     -> QwenTextRuntime._linear (hydraserve/model/runtime.py:1263-1270)
* ``concatenate_linear_weights`` -> _concatenate_linear_weights (runtime.py:1404-1475)
* ``split_linear_weight``        -> _split_linear_weight (runtime.py:1477-1506)

Fusion works on a per-format storage table: every quantized format is a set
of tensors whose dim 0 indexes output rows at some granularity (one packed
INT4 row per weight row, one zero-point word per 8 rows, one FP8 scale row
per 128-row block, ...).  Concatenating along N is then a field-wise
``torch.cat``, legal when every part's row count is a multiple of the
format's coarsest granularity; splitting is a field-wise ``narrow`` (a view,
which the kernels read through their row strides).  Nothing is requantized.
"""

from __future__ import annotations

import dataclasses
import math

from ..kernels.awq import awq_linear
from ..kernels.fp8 import fp8_linear
from .weights import BlockScaledFP8Weight, PackedInt4Weight


def linear(hidden, weight):
    """isinstance dispatch of runtime.py:1263-1270: INT4 -> awq_linear, FP8 ->
    fp8_linear, dense -> ``hidden @ weight.T`` on the weight's device."""
    if isinstance(weight, PackedInt4Weight):
        return awq_linear(hidden, weight)
    if isinstance(weight, BlockScaledFP8Weight):
        return fp8_linear(hidden, weight)
    if hidden.device != weight.device:
        hidden = hidden.to(weight.device)
    return hidden @ weight.transpose(0, 1)


def _storage(weight) -> dict[str, int]:
    """Tensor fields of a quantized weight -> weight rows covered by one row of
    that tensor.  The key set also fixes which fields fusion concatenates."""
    if isinstance(weight, PackedInt4Weight):
        return {"packed": 1, "scale": 1, "zero_point": 8}
    if isinstance(weight, BlockScaledFP8Weight):
        return {"data": 1, "scale_inv": weight.block_size[0]}
    raise TypeError(f"unsupported fused linear weight: {type(weight)!r}")


def _plain(weight):
    """The reference dataclass of a weight (a load-time tiled copy is dropped:
    its rows would no longer match after fusing or splitting)."""
    if getattr(weight, "tiles", None) is None:
        return weight
    if isinstance(weight, PackedInt4Weight):
        return PackedInt4Weight(weight.packed, weight.scale, weight.zero_point, weight.original_shape, weight.group_size)
    return BlockScaledFP8Weight(weight.data, weight.scale_inv, weight.original_shape, weight.block_size)


def _static(weight) -> tuple:
    """Everything besides the row count that fused parts must share."""
    if isinstance(weight, PackedInt4Weight):
        return (weight.original_shape[1], weight.group_size)
    return (weight.original_shape[1], weight.block_size)


def _tensor_key(t) -> tuple:
    return (t.device, t.dtype)


def concatenate_linear_weights(parts):
    """Fuse projections along N; ``None`` when the parts cannot be fused.

    Dense parts need equal width, device and dtype.  Quantized parts need the
    same format and K/group (or block) and matching device/dtype per field,
    and each part's N must be a multiple of every field's row granularity, so
    that no packed zero-point word or scale block straddles two parts.
    """
    import torch

    if not parts:
        return None
    parts = [_plain(p) if isinstance(p, (PackedInt4Weight, BlockScaledFP8Weight)) else p for p in parts]
    kinds = {type(p) for p in parts}
    if len(kinds) != 1:
        return None
    first = parts[0]
    if isinstance(first, torch.Tensor):
        key = (first.shape[1:] if first.ndim == 2 else None, first.device, first.dtype)
        if any(p.ndim != 2 or (p.shape[1:], p.device, p.dtype) != key for p in parts):
            return None
        return torch.cat(list(parts), dim=0).contiguous()
    if not isinstance(first, (PackedInt4Weight, BlockScaledFP8Weight)):
        return None
    fields = _storage(first)
    granule = math.lcm(*fields.values())
    if any(_static(p) != _static(first) or p.original_shape[0] % granule for p in parts):
        return None
    for name in fields:
        key = _tensor_key(getattr(first, name))
        if any(_tensor_key(getattr(p, name)) != key for p in parts):
            return None
    fused = {name: torch.cat([getattr(p, name) for p in parts], dim=0).contiguous() for name in fields}
    rows = sum(p.original_shape[0] for p in parts)
    return dataclasses.replace(first, **fused, original_shape=(rows, first.original_shape[1]))


def split_linear_weight(fused, sizes: tuple[int, ...]):
    """Row views of a fused weight, one per output size (inverse of
    ``concatenate_linear_weights``).  Quantized views share the fused storage."""
    import torch

    if isinstance(fused, torch.Tensor):
        return fused.split(sizes, dim=0)
    fused = _plain(fused)
    fields = _storage(fused)
    views = []
    row = 0
    for size in sizes:
        picked = {}
        for name, per in fields.items():
            if row % per or (size % per and row + size != fused.original_shape[0]):
                raise ValueError(f"split at rows [{row}, {row + size}) is not aligned to {name}'s {per}-row entries")
            picked[name] = getattr(fused, name).narrow(0, row // per, -(-size // per))
        views.append(dataclasses.replace(fused, **picked, original_shape=(size, fused.original_shape[1])))
        row += size
    return tuple(views)
