"""Load-time tiled copies of quantized weights (a kernel-native layout).

The checkpoint layouts keep each weight row contiguous (packed INT4 [N, K/8]
int32, E4M3 [N, K] bytes).  The tiled decode kernel reads 16-row blocks one
128-wide K chunk at a time: from the row-major layout that would be 16 rows x
64 bytes (INT4) per load instruction, i.e. sixteen 64-byte pieces 2.5-8.5 KB
apart.  The tiled copy
stores those 16 row pieces contiguously (tile (t, c) = rows 16t..16t+15 of
chunk c, 1 KiB INT4 / 2 KiB FP8), so the same load instruction reads one
contiguous KiB (INT4 words also pair their nibbles: nibble i < 4 holds K
offset 2i, nibble i + 4 holds 2i + 1, the order the tiled kernel's operand
unpack wants); on MI355X a streaming probe of the gate_up weight went from
~3.6 to ~5.3 TB/s with this layout.  Tiles are stored chunk-major (all N/16
tiles of chunk 0, then chunk 1, ...): the kernel's workgroups walk K in step,
so the grid reads one window of the weight at a time (FP8 gate_up M=1:
35.9 -> 33.0 us against the tile-major order, INT4 1-3 % faster).  Inside
an FP8 tile the bytes are ordered so that each of a lane's two 16-byte loads
is one contiguous KiB across the wave (two halves of 64 K each; the 16 bytes
of row r at K quarter p of a half at (16p + r) * 16).  The copy is made once, at load time, and
the row-major tensors stay in the weight (every other kernel reads them, and
the tiled decode kernel only takes activations of at most 64 rows, the
256x256 prefill kernel reads the tiles above that); the values are
not changed (tests check the round trip and the GEMM results).

TiledInt4Weight / TiledFP8Weight are the reference's dataclasses with one
more field, so every caller that reads the reference's fields keeps working.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from ..model.weights import BlockScaledFP8Weight, PackedInt4Weight


@dataclass(frozen=True, slots=True)
class TiledInt4Weight(PackedInt4Weight):
    tiles: Any = None  # int32 [K/128, N/16, 16, 16]


@dataclass(frozen=True, slots=True)
class TiledFP8Weight(BlockScaledFP8Weight):
    tiles: Any = None  # uint8 [K/128, N/16, 2, 4, 16, 16]: [chunk, tile, K half, K quarter, row, byte]


def _pair_nibbles(words, inverse: bool = False):
    """Reorder the nibbles of int32 words: nibble 2i (K offset 2i) goes to
    position i and nibble 2i+1 to position i+4, so that one mask of
    0x000F000F picks two consecutive-K weights (``inverse``: back)."""
    import torch

    u = words.to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros_like(u)
    for i in range(8):
        dst = i // 2 + 4 * (i % 2)
        src, to = (dst, i) if inverse else (i, dst)
        out |= ((u >> (4 * src)) & 0xF) << (4 * to)
    out = torch.where(out >= 2**31, out - 2**32, out)
    return out.to(torch.int32)


def tile_int4_weight(weight: PackedInt4Weight) -> TiledInt4Weight:
    n, k = weight.original_shape
    if n % 16 or k % 128 or weight.group_size != 128:
        raise ValueError("INT4 tiles need N % 16 == 0, K % 128 == 0 and group_size 128")
    p = weight.packed[:n, : k // 8]
    tiles = _pair_nibbles(p.reshape(n // 16, 16, k // 128, 16).permute(2, 0, 1, 3)).contiguous()
    return TiledInt4Weight(weight.packed, weight.scale, weight.zero_point, weight.original_shape, weight.group_size, tiles)


def untile_int4(tiles, n: int, k: int):
    """Row-major packed words [N, K/8] from the tiles (inverse of the layout)."""
    return _pair_nibbles(tiles, inverse=True).permute(1, 2, 0, 3).reshape(n, k // 8)


def tile_fp8_weight(weight: BlockScaledFP8Weight) -> TiledFP8Weight:
    import torch

    n, k = weight.original_shape
    if n % 16 or k % 128:
        raise ValueError("FP8 tiles need N % 16 == 0 and K % 128 == 0")
    d = weight.data.view(torch.uint8)[:n, :k]
    # tile bytes [h][p][r][16]: row r's bytes 64h + 16p .. +16 (the tiled
    # kernel's lane 16p + r reads them with its load h, one contiguous KiB
    # per load instruction)
    tiles = d.reshape(n // 16, 16, k // 128, 2, 4, 16).permute(2, 0, 3, 4, 1, 5).contiguous()
    return TiledFP8Weight(weight.data, weight.scale_inv, weight.original_shape, weight.block_size, tiles)
