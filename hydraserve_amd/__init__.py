"""hydraserve_amd: HydraServe's quantized linear-layer path, native to MI355X (gfx950).

Public surface mirrors the reference's:
  kernels.awq_linear / kernels.dequantize_int4_weight   (hydraserve/kernels/awq.py)
  kernels.fp8_linear / kernels.dequantize_fp8_weight    (hydraserve/kernels/fp8.py)
  model.weights.PackedInt4Weight / BlockScaledFP8Weight (hydraserve/model/weights.py)
  model.linear.linear / concatenate_linear_weights / split_linear_weight
                                                        (hydraserve/model/runtime.py)
All compute runs in libhydraserve_amd.so (hand-written HIP for gfx950).
"""

from . import ops  # noqa: F401  (registers the torch.library custom ops)
from .kernels import awq_linear, dequantize_fp8_weight, dequantize_int4_weight, fp8_linear
from .model.checkpoint import CheckpointReader, load_linear_weights, read_linear
from .model.linear import concatenate_linear_weights, linear, split_linear_weight
from .model.weights import BlockScaledFP8Weight, PackedInt4Weight

__all__ = [
    "awq_linear",
    "fp8_linear",
    "dequantize_int4_weight",
    "dequantize_fp8_weight",
    "PackedInt4Weight",
    "BlockScaledFP8Weight",
    "linear",
    "concatenate_linear_weights",
    "split_linear_weight",
    "CheckpointReader",
    "load_linear_weights",
    "read_linear",
]
