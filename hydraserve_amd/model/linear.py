"""The runtime's linear-layer dispatch and projection fusion helpers.

Mirrors the static methods of QwenTextRuntime that sit directly on the
quantized path:

* ``linear``                     -> QwenTextRuntime._linear (hydraserve/model/runtime.py:1263-1270)
* ``concatenate_linear_weights`` -> _concatenate_linear_weights (runtime.py:1404-1475)
* ``split_linear_weight``        -> _split_linear_weight (runtime.py:1477-1506)

Fusion concatenates packed INT4 / E4M3 storage along N without requantizing;
splits are ``narrow`` views of the fused tensors, which the kernels read
through their row strides.
"""

from __future__ import annotations

from ..kernels.awq import awq_linear
from ..kernels.fp8 import fp8_linear
from .weights import BlockScaledFP8Weight, PackedInt4Weight


def linear(hidden, weight):
    if isinstance(weight, PackedInt4Weight):
        return awq_linear(hidden, weight)
    if isinstance(weight, BlockScaledFP8Weight):
        return fp8_linear(hidden, weight)
    if hidden.device != weight.device:
        hidden = hidden.to(weight.device)
    return hidden @ weight.transpose(0, 1)


def concatenate_linear_weights(parts):
    """Fuse projections along N; ``None`` when the parts cannot be fused."""
    import torch

    if not parts:
        return None
    if all(isinstance(part, torch.Tensor) for part in parts):
        first = parts[0]
        if not all(
            part.ndim == 2
            and part.shape[1] == first.shape[1]
            and part.device == first.device
            and part.dtype == first.dtype
            for part in parts
        ):
            return None
        return torch.cat(parts, dim=0).contiguous()
    if all(isinstance(part, BlockScaledFP8Weight) for part in parts):
        first = parts[0]
        block_n, _ = first.block_size
        # Every part must start on a scale-block boundary (N % 128 == 0).
        if not all(
            part.original_shape[1] == first.original_shape[1]
            and part.block_size == first.block_size
            and part.original_shape[0] % block_n == 0
            and part.data.device == first.data.device
            and part.scale_inv.device == first.scale_inv.device
            and part.data.dtype == first.data.dtype
            and part.scale_inv.dtype == first.scale_inv.dtype
            for part in parts
        ):
            return None
        return BlockScaledFP8Weight(
            torch.cat([part.data for part in parts], dim=0).contiguous(),
            torch.cat([part.scale_inv for part in parts], dim=0).contiguous(),
            (sum(part.original_shape[0] for part in parts), first.original_shape[1]),
            first.block_size,
        )
    if all(isinstance(part, PackedInt4Weight) for part in parts):
        first = parts[0]
        # Zero points pack 8 rows per word, so every part needs N % 8 == 0.
        if not all(
            part.original_shape[1] == first.original_shape[1]
            and part.group_size == first.group_size
            and part.original_shape[0] % 8 == 0
            and part.packed.device == first.packed.device
            and part.scale.device == first.scale.device
            and part.zero_point.device == first.zero_point.device
            and part.packed.dtype == first.packed.dtype
            and part.scale.dtype == first.scale.dtype
            and part.zero_point.dtype == first.zero_point.dtype
            for part in parts
        ):
            return None
        return PackedInt4Weight(
            torch.cat([part.packed for part in parts], dim=0).contiguous(),
            torch.cat([part.scale for part in parts], dim=0).contiguous(),
            torch.cat([part.zero_point for part in parts], dim=0).contiguous(),
            (sum(part.original_shape[0] for part in parts), first.original_shape[1]),
            first.group_size,
        )
    return None


def split_linear_weight(fused, sizes: tuple[int, ...]):
    """Views of a fused weight, one per output size (inverse of concatenation)."""
    import torch

    if isinstance(fused, torch.Tensor):
        return fused.split(sizes, dim=0)
    if isinstance(fused, BlockScaledFP8Weight):
        block_n, _ = fused.block_size
        out = []
        start = 0
        for size in sizes:
            out.append(
                BlockScaledFP8Weight(
                    fused.data.narrow(0, start, size),
                    fused.scale_inv.narrow(0, start // block_n, size // block_n),
                    (size, fused.original_shape[1]),
                    fused.block_size,
                )
            )
            start += size
        return tuple(out)
    if isinstance(fused, PackedInt4Weight):
        out = []
        start = 0
        for size in sizes:
            out.append(
                PackedInt4Weight(
                    fused.packed.narrow(0, start, size),
                    fused.scale.narrow(0, start, size),
                    fused.zero_point.narrow(0, start // 8, size // 8),
                    (size, fused.original_shape[1]),
                    fused.group_size,
                )
            )
            start += size
        return tuple(out)
    raise TypeError(f"unsupported fused linear weight: {type(fused)!r}")
