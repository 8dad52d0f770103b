"""Grouped asymmetric INT4 weight-only GEMM on MI355X.

Drop-in for hydraserve/kernels/awq.py: same function names, arguments,
validation order, messages and exception types (awq.py:25-43).  Execution is
the HIP kernels of libhydraserve_amd.so on the current stream; unlike the
reference there is no CPU execution branch (awq.py:36-38): CPU activations are
rejected after validation.
"""

from __future__ import annotations

from .. import _native
from ._device import device_guard, require_gpu


def _check_int4_storage(weight) -> None:
    import torch

    n, k = weight.original_shape
    kw = (k + 7) // 8
    groups = (k + weight.group_size - 1) // weight.group_size
    if weight.packed.dtype != torch.int32 or weight.zero_point.dtype != torch.int32:
        raise TypeError("packed INT4 weight and zero points must be int32 tensors")
    if weight.scale.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("INT4 scales must be bfloat16, float16 or float32")
    if (
        weight.packed.dim() != 2
        or weight.packed.shape[0] < n
        or weight.packed.shape[1] < kw
        or weight.scale.dim() != 2
        or weight.scale.shape[0] < n
        or weight.scale.shape[1] < groups
        or weight.zero_point.dim() != 2
        or weight.zero_point.shape[0] < (n + 7) // 8
        or weight.zero_point.shape[1] < groups
    ):
        raise ValueError("packed INT4 tensors do not cover the weight's original_shape")


def dequantize_int4_weight(weight):
    """Dense [N, K] weight in ``weight.scale.dtype``: (q - z) * s, rounded once.

    Same result as hydraserve/kernels/awq.py:6-22, computed on the GPU by
    hs_int4_dequant (bit-exact).
    """
    require_gpu(weight.packed, "dequantize_int4_weight")
    if not all(t.is_cuda for t in (weight.packed, weight.scale, weight.zero_point)):
        raise ValueError("packed INT4 tensors must be on the same GPU")
    _check_int4_storage(weight)
    n, k = weight.original_shape
    with device_guard(weight.packed.device):
        return _native.int4_dequant(
            weight.packed, weight.scale, weight.zero_point, n, k, weight.group_size, weight.scale.dtype
        )


def awq_linear(hidden, weight):
    """Y = hidden @ dequant(weight)^T, shape hidden.shape[:-1] + (N,), dtype hidden.dtype."""
    if hidden.shape[-1] != weight.original_shape[1]:
        raise ValueError("activation width does not match packed INT4 weight")
    if weight.group_size != 128:
        raise ValueError("HydraServe AWQ kernel currently requires group_size=128")
    if hidden.device != weight.packed.device:
        raise ValueError("activation and packed weight must be on the same device")
    shape = hidden.shape[:-1] + (weight.original_shape[0],)
    flattened = hidden.reshape(-1, hidden.shape[-1]).contiguous()
    require_gpu(hidden, "awq_linear")
    if not all(
        tensor.is_cuda and tensor.is_contiguous()
        for tensor in (weight.packed, weight.scale, weight.zero_point)
    ):
        raise ValueError("packed INT4 tensors must be contiguous CUDA tensors")
    _check_int4_storage(weight)
    import torch

    if flattened.dtype != torch.bfloat16:
        raise TypeError("hydraserve_amd quantized GEMMs take bfloat16 activations")
    n, k = weight.original_shape
    if k == 0:
        return torch.zeros(shape, device=hidden.device, dtype=hidden.dtype)
    if torch.compiler.is_compiling():
        # Dynamo/Inductor: the opaque custom op (hydraserve_amd/ops.py)
        out = torch.ops.hydraserve_amd.int4_gemm(
            flattened, weight.packed, weight.scale, weight.zero_point, n, k, weight.group_size
        )
        return out.reshape(shape)
    tiles = getattr(weight, "tiles", None)  # load-time tiled copy (kernels/tiles.py)
    if tiles is not None and not (tiles.is_cuda and tiles.device == hidden.device and tiles.is_contiguous()):
        raise ValueError("INT4 weight tiles must be a contiguous tensor on the activation's GPU")
    with device_guard(hidden.device):
        out = _native.int4_gemm(flattened, weight.packed, weight.scale, weight.zero_point, n, k, weight.group_size, tiles)
    return out.reshape(shape)
