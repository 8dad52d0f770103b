"""Quantized linear ops with the reference's signatures (hydraserve/kernels)."""

from .awq import awq_linear, dequantize_int4_weight
from .fp8 import dequantize_fp8_weight, fp8_linear
from .fp8_stream import pin_fp8_weight
from .tiles import TiledFP8Weight, TiledInt4Weight, tile_fp8_weight, tile_int4_weight
from .mlp import awq_gate_up_silu_mul, deinterleave_gate_up, interleave_gate_up, silu_and_mul

__all__ = [
    "awq_linear",
    "dequantize_int4_weight",
    "fp8_linear",
    "dequantize_fp8_weight",
    "pin_fp8_weight",
    "TiledInt4Weight",
    "TiledFP8Weight",
    "tile_int4_weight",
    "tile_fp8_weight",
    "interleave_gate_up",
    "deinterleave_gate_up",
    "silu_and_mul",
    "awq_gate_up_silu_mul",
]
