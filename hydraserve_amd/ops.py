"""torch.library registration of the native GEMMs (namespace ``hydraserve_amd``).

The reference's ``_linear`` runs eagerly, under CUDA-graph capture
(hydraserve/model/runtime.py:788-803) and, with
HYDRASERVE_TORCH_COMPILE_SCOPE=transactions, inside ``torch.compile``
(runtime.py:577, 592-596).  A raw ctypes call cannot be traced by Dynamo, so
each native entry point is also a custom op with a fake (meta) implementation:
Dynamo and Inductor see an opaque op with a known output shape and dtype, and
``fullgraph=True`` compiles without a graph break.  Eager callers skip the
dispatcher and call the library directly (the Python wrappers check
``torch.compiler.is_compiling()``), so the decode loop pays no extra per-call
cost.

Every op enqueues on the current stream of the input's device and allocates
its output through the caching allocator, as the eager path does.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native
from .kernels._device import device_guard


@torch.library.custom_op("hydraserve_amd::int4_gemm", mutates_args=(), device_types="cuda")
def int4_gemm(x: Tensor, packed: Tensor, scale: Tensor, zero_point: Tensor, n: int, k: int, group: int) -> Tensor:
    """Y[M, N] bf16 = x[M, K] . dequant(W)^T (hs_int4_gemm)."""
    with device_guard(x.device):
        return _native.int4_gemm(x, packed, scale, zero_point, n, k, group)


@int4_gemm.register_fake
def _int4_gemm_fake(x, packed, scale, zero_point, n, k, group):
    return x.new_empty(x.shape[0], n)


@torch.library.custom_op("hydraserve_amd::fp8_gemm", mutates_args=(), device_types="cuda")
def fp8_gemm(x: Tensor, data_u8: Tensor, scale_inv: Tensor, n: int, k: int) -> Tensor:
    """Y[M, N] bf16 = x[M, K] . (decode(W) * scale_inv)^T (hs_fp8_gemm)."""
    with device_guard(x.device):
        return _native.fp8_gemm(x, data_u8, scale_inv, n, k)


@fp8_gemm.register_fake
def _fp8_gemm_fake(x, data_u8, scale_inv, n, k):
    return x.new_empty(x.shape[0], n)


@torch.library.custom_op("hydraserve_amd::int4_gate_up_silu_mul", mutates_args=(), device_types="cuda")
def int4_gate_up_silu_mul(
    x: Tensor, packed: Tensor, scale: Tensor, zero_point: Tensor, n: int, k: int, group: int
) -> Tensor:
    """silu(gate) * up [M, N/2] on a gate/up-interleaved INT4 weight."""
    from .kernels.mlp import unfused_gate_up_silu_mul

    with device_guard(x.device):
        out = _native.int4_gemm_silu_mul(x, packed, scale, zero_point, n, k, group)
        if out is None:
            out = unfused_gate_up_silu_mul(x, packed, scale, zero_point, n, k, group)
        return out


@int4_gate_up_silu_mul.register_fake
def _int4_gate_up_silu_mul_fake(x, packed, scale, zero_point, n, k, group):
    return x.new_empty(x.shape[0], n // 2)
