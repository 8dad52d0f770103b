"""Quantized linear-weight containers.

Same fields, defaults and semantics as the reference's boundary types in
hydraserve/model/weights.py:12-38, so checkpoint loaders and callers built for
the reference construct them unchanged.  The tensors are caller-owned and
never modified.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True, slots=True)
class PackedInt4Weight:
    """Compressed-tensors asymmetric grouped INT4 linear weight.

    packed:      int32 [N, ceil(K/8)], nibble i of word j is W[n, 8j+i]
    scale:       [N, ceil(K/group)] (bf16 in checkpoints)
    zero_point:  int32 [ceil(N/8), ceil(K/group)], nibble j of word [r, g] is
                 the zero point of row 8r+j in group g
    original_shape: (N, K)
    """

    packed: Any
    scale: Any
    zero_point: Any
    original_shape: tuple[int, int]
    group_size: int = 128

    @property
    def shape(self) -> tuple[int, int]:
        return self.original_shape


@dataclass(frozen=True, slots=True)
class BlockScaledFP8Weight:
    """E4M3FN weight [N, K] with one inverse scale per 128x128 block."""

    data: Any
    scale_inv: Any
    original_shape: tuple[int, int]
    block_size: tuple[int, int] = (128, 128)

    @property
    def shape(self) -> tuple[int, int]:
        return self.original_shape
