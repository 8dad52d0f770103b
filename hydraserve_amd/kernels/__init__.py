"""Quantized linear ops with the reference's signatures (hydraserve/kernels)."""

from .awq import awq_linear, dequantize_int4_weight
from .fp8 import dequantize_fp8_weight, fp8_linear

__all__ = ["awq_linear", "dequantize_int4_weight", "fp8_linear", "dequantize_fp8_weight"]
