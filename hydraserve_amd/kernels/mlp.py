"""The MLP's gate_up projection with SiLU-and-mul fused into the INT4 GEMM.

The reference runs, per decoder layer (hydraserve/model/runtime.py:1202-1210):

    gate, up = self._linear(hidden, weights.gate_up).chunk(2, dim=-1)
    activated = silu_and_mul(gate.contiguous(), up.contiguous())

with silu_and_mul = bf16(fp32(gate) * sigmoid(fp32(gate)) * fp32(up))
(hydraserve/kernels/activation.py:4-25, kernel :66-76).  Here the gate_up weight
is re-laid out once, at load time, so that every 16-row block of gate rows is
followed by the matching 16 up rows (interleave_gate_up, lossless); the GEMM
kernel then finds each gate/up pair inside one output tile and stores
silu(gate) * up directly (hs_int4_gemm_silu_mul), skipping the [M, N] bf16
round trip and the activation launch.  Gate and up are rounded to bf16 before
the activation, as in the reference's unfused sequence.

The fused store is in the row-partitioned decode kernels (1..16 rows), the
17..128-row streaming kernel and the 256x256-tile prefill kernel.  Where
neither applies (e.g. more than 128 rows), awq_gate_up_silu_mul runs hs_int4_gemm on the interleaved weight and the
activation as torch GPU ops on its output.
"""

from __future__ import annotations

from .. import _native
from ..model.weights import PackedInt4Weight
from ._device import device_guard, require_gpu
from .awq import _check_int4_storage

BLOCK = 16  # rows per gate / up block of the interleaved layout


def _row_order(n: int, device):
    """Rows of the fused gate_up weight in interleaved order."""
    import torch

    half = n // 2
    blocks = torch.arange(half // BLOCK, device=device).view(-1, 1, 1) * BLOCK
    within = torch.arange(BLOCK, device=device).view(1, 1, -1)
    side = torch.tensor([0, half], device=device).view(1, 2, 1)
    return (blocks + side + within).reshape(-1)


def interleave_gate_up(weight: PackedInt4Weight) -> PackedInt4Weight:
    """gate_up [N = 2H, K] -> the same weight with rows ordered gate 16j..16j+15,
    up 16j..16j+15 for j = 0 .. H/16 - 1.  Packed rows, scale rows and
    zero-point words (8 rows each, so a 16-row block is two whole words) move
    together; no value changes."""
    n, k = weight.original_shape
    if n % (2 * BLOCK) != 0:
        raise ValueError("gate_up interleave needs N (both halves) to be a multiple of 32")
    order = _row_order(n, weight.packed.device)
    zorder = order.view(-1, 8)[:, 0] // 8
    return PackedInt4Weight(
        weight.packed[:n].index_select(0, order).contiguous(),
        weight.scale[:n].index_select(0, order.to(weight.scale.device)).contiguous(),
        weight.zero_point[: n // 8].index_select(0, zorder.to(weight.zero_point.device)).contiguous(),
        (n, k),
        weight.group_size,
    )


def deinterleave_gate_up(weight: PackedInt4Weight) -> PackedInt4Weight:
    """Inverse of interleave_gate_up."""
    import torch

    n, k = weight.original_shape
    order = _row_order(n, weight.packed.device)
    inverse = torch.empty_like(order)
    inverse[order] = torch.arange(n, device=order.device)
    zinverse = inverse.view(-1, 8)[:, 0] // 8
    return PackedInt4Weight(
        weight.packed[:n].index_select(0, inverse).contiguous(),
        weight.scale[:n].index_select(0, inverse.to(weight.scale.device)).contiguous(),
        weight.zero_point[: n // 8].index_select(0, zinverse.to(weight.zero_point.device)).contiguous(),
        (n, k),
        weight.group_size,
    )


def silu_and_mul(gate, up):
    """silu(gate) * up in fp32, returned in gate's dtype (activation.py:4-25)."""
    import torch

    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate and up tensors must have matching shape and dtype")
    g = gate.float()
    return (g * torch.sigmoid(g) * up.float()).to(gate.dtype)


def awq_gate_up_silu_mul(hidden, weight: PackedInt4Weight):
    """silu(gate) * up for hidden [..., K] and an interleaved gate_up weight;
    shape hidden.shape[:-1] + (N/2,), dtype hidden.dtype."""
    if hidden.shape[-1] != weight.original_shape[1]:
        raise ValueError("activation width does not match packed INT4 weight")
    if weight.group_size != 128:
        raise ValueError("HydraServe AWQ kernel currently requires group_size=128")
    if hidden.device != weight.packed.device:
        raise ValueError("activation and packed weight must be on the same device")
    n, k = weight.original_shape
    if n % (2 * BLOCK) != 0:
        raise ValueError("gate_up interleave needs N (both halves) to be a multiple of 32")
    require_gpu(hidden, "awq_gate_up_silu_mul")
    if not all(
        tensor.is_cuda and tensor.is_contiguous()
        for tensor in (weight.packed, weight.scale, weight.zero_point)
    ):
        raise ValueError("packed INT4 tensors must be contiguous CUDA tensors")
    _check_int4_storage(weight)
    tiles = getattr(weight, "tiles", None)  # load-time tiled copy (kernels/tiles.py)
    if tiles is not None and not (tiles.is_cuda and tiles.device == hidden.device and tiles.is_contiguous()):
        raise ValueError("INT4 weight tiles must be a contiguous tensor on the activation's GPU")
    import torch

    flattened = hidden.reshape(-1, k).contiguous()
    if flattened.dtype != torch.bfloat16:
        raise TypeError("hydraserve_amd quantized GEMMs take bfloat16 activations")
    shape = hidden.shape[:-1] + (n // 2,)
    if k == 0:
        return torch.zeros(shape, device=hidden.device, dtype=hidden.dtype)
    args = (flattened, weight.packed, weight.scale, weight.zero_point, n, k, weight.group_size)
    if torch.compiler.is_compiling():
        # Dynamo/Inductor: the opaque custom op (hydraserve_amd/ops.py)
        return torch.ops.hydraserve_amd.int4_gate_up_silu_mul(*args).reshape(shape)
    with device_guard(hidden.device):
        out = _native.int4_gemm_silu_mul(*args, tiles=tiles)
        if out is None:
            out = unfused_gate_up_silu_mul(*args)
    return out.reshape(shape)


def unfused_gate_up_silu_mul(x, packed, scale, zero_point, n, k, group):
    """The GEMM on the interleaved weight, then the activation on its gate/up
    block pairs: for shapes the fused store does not cover."""
    m = x.shape[0]
    y = _native.int4_gemm(x, packed, scale, zero_point, n, k, group)
    pairs = y.view(m, n // (2 * BLOCK), 2, BLOCK)
    return silu_and_mul(pairs[:, :, 0], pairs[:, :, 1]).reshape(m, n // 2)
