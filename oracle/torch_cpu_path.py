"""The reference's CPU execution branch, restated in PyTorch for timing.

TEST INFRASTRUCTURE ONLY (the CPU baseline that ``bench.py`` times beside the
GPU kernels).  When ``hidden`` is a CPU tensor the reference's ``awq_linear``
and ``fp8_linear`` dequantize the whole weight and run one dense matmul in the
activation dtype:

* INT4: hydraserve/kernels/awq.py:36-38 with the dequant of awq.py:6-22
  (shift/mask unpack, zero-point gather, ``(q - z).to(scale.dtype) * scale``);
* FP8:  hydraserve/kernels/fp8.py:51-53 with the dequant of fp8.py:6-21 at
  ``dtype=hidden.dtype`` (bf16).

The dequant is included per call, exactly as the reference does.
"""

from __future__ import annotations


def int4_cpu_linear(hidden, packed, scale, zero_point, original_shape, group_size=128):
    import torch

    n, k = original_shape
    shifts = torch.arange(8, dtype=torch.int32) * 4
    q = ((packed.unsqueeze(-1) >> shifts) & 0xF).reshape(n, -1)[:, :k]
    z = ((zero_point.unsqueeze(-1) >> shifts) & 0xF).permute(0, 2, 1).reshape(-1, scale.shape[1])[:n]
    groups = torch.arange(k) // group_size
    dense = (q - z[:, groups]).to(scale.dtype) * scale[:, groups]
    flat = hidden.reshape(-1, k).contiguous()
    return flat @ dense.transpose(0, 1)


def fp8_cpu_linear(hidden, data, scale_inv, original_shape):
    import torch

    n, k = original_shape
    ob = torch.arange(n) // 128
    ib = torch.arange(k) // 128
    scales = scale_inv[ob[:, None], ib[None, :]]
    dense = data.to(hidden.dtype) * scales.to(hidden.dtype)
    flat = hidden.reshape(-1, k).contiguous()
    return flat @ dense.transpose(0, 1)
