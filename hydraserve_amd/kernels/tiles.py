"""Load-time tiled copies of quantized weights (a kernel-native layout).

The checkpoint layouts keep each weight row contiguous (packed INT4 [N, K/8]
int32, E4M3 [N, K] bytes).  The block-major decode kernel reads a 16-row
block one 128-wide K chunk at a time: 16 rows x 64 bytes (INT4) per load
instruction, i.e. sixteen 64-byte pieces 2.5-8.5 KB apart.  The tiled copy
stores those 16 row pieces contiguously (tile (t, c) = rows 16t..16t+15 of
chunk c, 1 KiB INT4 / 2 KiB FP8), so the same load instruction reads one
contiguous KiB; on MI355X a streaming probe of the gate_up weight went from
~3.6 to ~5.3 TB/s with this layout.  The copy is made once, at load time, and
the row-major tensors stay in the weight (every other kernel reads them); the
values are not changed (tests check the round trip and the GEMM results).

TiledInt4Weight / TiledFP8Weight are the reference's dataclasses with one
more field, so every caller that reads the reference's fields keeps working.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from ..model.weights import BlockScaledFP8Weight, PackedInt4Weight


@dataclass(frozen=True, slots=True)
class TiledInt4Weight(PackedInt4Weight):
    tiles: Any = None  # int32 [N/16, K/128, 16, 16]


@dataclass(frozen=True, slots=True)
class TiledFP8Weight(BlockScaledFP8Weight):
    tiles: Any = None  # uint8 [N/16, K/128, 16, 128]


def tile_int4_weight(weight: PackedInt4Weight) -> TiledInt4Weight:
    n, k = weight.original_shape
    if n % 16 or k % 128 or weight.group_size != 128:
        raise ValueError("INT4 tiles need N % 16 == 0, K % 128 == 0 and group_size 128")
    p = weight.packed[:n, : k // 8]
    tiles = p.reshape(n // 16, 16, k // 128, 16).permute(0, 2, 1, 3).contiguous()
    return TiledInt4Weight(weight.packed, weight.scale, weight.zero_point, weight.original_shape, weight.group_size, tiles)


def untile_int4(tiles, n: int, k: int):
    """Row-major packed words [N, K/8] from the tiles (inverse of the layout)."""
    return tiles.permute(0, 2, 1, 3).reshape(n, k // 8)


def tile_fp8_weight(weight: BlockScaledFP8Weight) -> TiledFP8Weight:
    import torch

    n, k = weight.original_shape
    if n % 16 or k % 128:
        raise ValueError("FP8 tiles need N % 16 == 0 and K % 128 == 0")
    d = weight.data.view(torch.uint8)[:n, :k]
    tiles = d.reshape(n // 16, 16, k // 128, 128).permute(0, 2, 1, 3).contiguous()
    return TiledFP8Weight(weight.data, weight.scale_inv, weight.original_shape, weight.block_size, tiles)
