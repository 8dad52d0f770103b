"""Device plumbing shared by the quantized ops."""

from __future__ import annotations

import contextlib


def require_gpu(tensor, op: str) -> None:
    """The ops run only as HIP kernels; CPU tensors are an error, not a fallback."""
    if not tensor.is_cuda:
        raise RuntimeError(
            f"{op}: hydraserve_amd executes on a ROCm GPU only (got a {tensor.device.type} tensor); "
            "move the activation and weight to the GPU"
        )


@contextlib.contextmanager
def device_guard(device):
    import torch

    if device.index is None or device.index == torch.cuda.current_device():
        yield
        return
    with torch.cuda.device(device):
        yield
