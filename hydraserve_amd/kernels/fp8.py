"""128x128 block-scaled E4M3FN weight-only GEMM on MI355X.

Drop-in for hydraserve/kernels/fp8.py: same function names, arguments,
validation order, messages and exception types (fp8.py:24-62), including the
staging of host-resident weights onto the activation's GPU (fp8.py:32-41);
page-locked host weights take the overlapped slab stream of fp8_stream.py.
Execution is the HIP kernels of libhydraserve_amd.so; unlike the reference
there is no CPU execution branch (fp8.py:51-53).
"""

from __future__ import annotations

from .. import _native
from ._device import device_guard, require_gpu
from .fp8_stream import PREFILL_ROWS, is_pinned_weight, streamed_fp8_gemm


def _check_scale_grid(weight) -> None:
    output_features, input_features = weight.original_shape
    block_n, block_k = weight.block_size
    expected = ((output_features + block_n - 1) // block_n, (input_features + block_k - 1) // block_k)
    if tuple(weight.scale_inv.shape) != expected:
        raise ValueError("FP8 inverse-scale grid does not match weight shape")


def _as_bytes(data):
    import torch

    if data.dtype != torch.float8_e4m3fn:
        raise TypeError("FP8 kernel requires torch.float8_e4m3fn weight storage")
    return data.view(torch.uint8)


def dequantize_fp8_weight(weight, *, dtype=None):
    """decode(W) * scale_inv (both cast to ``dtype``, default float32), as
    hydraserve/kernels/fp8.py:6-21 computes it; on the GPU via hs_fp8_dequant."""
    import torch

    _check_scale_grid(weight)
    require_gpu(weight.data, "dequantize_fp8_weight")
    if not weight.scale_inv.is_cuda or weight.scale_inv.device != weight.data.device:
        raise ValueError("FP8 data and scales must be on the same GPU")
    n, k = weight.original_shape
    data = _as_bytes(weight.data)
    if tuple(data.shape) != (n, k):
        raise ValueError("FP8 data does not match the weight's original_shape")
    out_dtype = dtype or torch.float32
    _native.dtype_code(out_dtype)
    with device_guard(data.device):
        return _native.fp8_dequant(data, weight.scale_inv, n, k, out_dtype)


def _streamed(hidden, weight):
    import torch

    _check_scale_grid(weight)
    n, k = weight.original_shape
    data = _as_bytes(weight.data)
    if tuple(data.shape) != (n, k) or not (data.is_contiguous() and weight.scale_inv.is_contiguous()):
        raise ValueError("FP8 data and scales must be contiguous tensors of the weight's shape")
    flattened = hidden.reshape(-1, k).contiguous()
    if flattened.dtype != torch.bfloat16:
        raise TypeError("hydraserve_amd quantized GEMMs take bfloat16 activations")
    _native.dtype_code(weight.scale_inv.dtype)
    shape = hidden.shape[:-1] + (n,)
    if k == 0:
        return torch.zeros(shape, device=hidden.device, dtype=hidden.dtype)
    with device_guard(hidden.device):
        return streamed_fp8_gemm(flattened, weight).reshape(shape)


def fp8_linear(hidden, weight):
    """Multiply BF16 activations by block-scaled E4M3 weights."""
    import torch

    if hidden.shape[-1] != weight.original_shape[1]:
        raise ValueError("activation width does not match FP8 weight")
    if weight.block_size != (128, 128):
        raise ValueError("HydraServe FP8 kernel currently requires 128x128 blocks")
    if hidden.device != weight.data.device:
        if not hidden.is_cuda or weight.data.device.type != "cpu":
            raise ValueError("unsupported activation/FP8 weight device placement")
        rows = hidden.numel() // max(hidden.shape[-1], 1)
        if is_pinned_weight(weight) and rows >= PREFILL_ROWS and not torch.compiler.is_compiling():
            # page-locked host weight: slab copies overlapped with slab GEMMs
            return _streamed(hidden, weight)
        staged = type(weight)(
            weight.data.to(hidden.device, non_blocking=True).contiguous(),
            weight.scale_inv.to(hidden.device, non_blocking=True).contiguous(),
            weight.original_shape,
            weight.block_size,
        )
        return fp8_linear(hidden, staged)
    _check_scale_grid(weight)
    output_features, input_features = weight.original_shape
    shape = hidden.shape[:-1] + (output_features,)
    flattened = hidden.reshape(-1, input_features).contiguous()
    require_gpu(hidden, "fp8_linear")
    if not (
        weight.data.is_cuda
        and weight.scale_inv.is_cuda
        and weight.data.is_contiguous()
        and weight.scale_inv.is_contiguous()
    ):
        raise ValueError("FP8 data and scales must be contiguous CUDA tensors")
    data = _as_bytes(weight.data)
    if tuple(data.shape) != (output_features, input_features):
        raise ValueError("FP8 data does not match the weight's original_shape")
    if flattened.dtype != torch.bfloat16:
        raise TypeError("hydraserve_amd quantized GEMMs take bfloat16 activations")
    _native.dtype_code(weight.scale_inv.dtype)
    if input_features == 0:
        return torch.zeros(shape, device=hidden.device, dtype=hidden.dtype)
    if torch.compiler.is_compiling():
        # Dynamo/Inductor: the opaque custom op (hydraserve_amd/ops.py)
        out = torch.ops.hydraserve_amd.fp8_gemm(flattened, data, weight.scale_inv, output_features, input_features)
        return out.reshape(shape)
    tiles = getattr(weight, "tiles", None)  # load-time tiled copy (kernels/tiles.py)
    if tiles is not None and not (tiles.is_cuda and tiles.device == hidden.device and tiles.is_contiguous()):
        raise ValueError("FP8 weight tiles must be a contiguous tensor on the activation's GPU")
    with device_guard(hidden.device):
        out = _native.fp8_gemm(flattened, data, weight.scale_inv, output_features, input_features, tiles)
    return out.reshape(shape)
