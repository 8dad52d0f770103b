"""Host-resident FP8 weights streamed to the GPU with the copy overlapping the GEMM.

The reference's memory-aware loader keeps some FP8 projections in host memory
when the GPU is short (hydraserve/model/runtime.py:182-236) and fp8_linear
stages such a weight onto the activation's GPU on every call, the whole
weight first and the GEMM after it (hydraserve/kernels/fp8.py:32-41).

Here the weight is cut along N into slabs of whole 128-row scale blocks.  A
row slab of the row-major [N, K] E4M3 matrix is one contiguous host range, so
each slab is one host-to-device copy (data rows plus their scale rows) on a
side stream, into one of two device staging buffers, while the current stream
runs hs_fp8_gemm on the previous slab and writes its columns of Y in place
(row stride N).  Events order the two streams: a slab's GEMM waits for its
copy, and a buffer's next copy waits for the GEMM that read it.  Both streams
have the default priority.

Overlap needs page-locked host memory: a pageable source makes the copy
synchronous.  ``pin_fp8_weight`` makes a page-locked copy of a host-resident
weight once, at load time (a newly allocated pinned tensor, never a
registration of existing memory); ``fp8_linear`` takes this path for pinned
host weights at PREFILL_ROWS activation rows or more, and the reference's
staging otherwise (for decode the copy is ~99 % of the time, and one copy on
the current stream measured faster than the side-stream sequence).
"""

from __future__ import annotations

import threading

from .. import _native
from ..model.weights import BlockScaledFP8Weight

# Slab choice.  Copies run at ~55 GB/s for one large transfer and a few GB/s
# less for 20-30 MB pieces, while a decode GEMM is ~1 % of the copy time: at
# fewer than PREFILL_ROWS activation rows the whole weight is one slab (one
# copy, then the GEMM).  From there, about SLABS slabs of whole 128-row scale
# blocks (at least MIN_SLAB_ROWS rows), so all but the last slab's GEMM hide
# under the copies.
PREFILL_ROWS = 128
SLABS = 6
MIN_SLAB_ROWS = 4096


def auto_slab_rows(m: int, n: int) -> int:
    if m < PREFILL_ROWS:
        return ((n + 127) // 128) * 128
    rows = -(-n // SLABS)
    return max(MIN_SLAB_ROWS, ((rows + 127) // 128) * 128)


_copy_streams: dict[int, object] = {}
_lock = threading.Lock()


def _copy_stream(device):
    import torch

    with _lock:
        s = _copy_streams.get(device.index)
        if s is None:
            s = torch.cuda.Stream(device=device)  # default priority
            _copy_streams[device.index] = s
        return s


def pin_fp8_weight(weight: BlockScaledFP8Weight) -> BlockScaledFP8Weight:
    """Page-locked host copy of a host-resident FP8 weight (load time, once)."""
    if weight.data.device.type != "cpu":
        raise ValueError("pin_fp8_weight takes a host-resident weight")
    return BlockScaledFP8Weight(
        weight.data.contiguous().pin_memory(),
        weight.scale_inv.contiguous().pin_memory(),
        weight.original_shape,
        weight.block_size,
    )


def is_pinned_weight(weight) -> bool:
    return weight.data.device.type == "cpu" and weight.data.is_pinned() and weight.scale_inv.is_pinned()


def streamed_fp8_gemm(flattened, weight: BlockScaledFP8Weight, slab_rows: int | None = None):
    """Y [M, N] for a contiguous bf16 ``flattened`` [M, K] on the GPU and a
    pinned host-resident weight, copies overlapped with the slab GEMMs
    (``slab_rows`` None: auto_slab_rows)."""
    import torch

    n, k = weight.original_shape
    if slab_rows is None:
        slab_rows = auto_slab_rows(flattened.shape[0], n)
    if slab_rows <= 0 or slab_rows % 128 != 0:
        raise ValueError("slab_rows must be a positive multiple of 128")
    dev = flattened.device
    m = flattened.shape[0]
    y = torch.empty(m, n, device=dev, dtype=flattened.dtype)
    if m == 0 or n == 0:
        return y
    data = weight.data.view(torch.uint8)
    scale = weight.scale_inv
    compute = torch.cuda.current_stream(dev)
    copy = _copy_stream(dev)
    rows = min(slab_rows, n)
    srows = (rows + 127) // 128
    nbuf = 1 if rows >= n else 2
    bufs = [
        (torch.empty(rows, k, dtype=torch.uint8, device=dev), torch.empty(srows, scale.shape[1], dtype=scale.dtype, device=dev))
        for _ in range(nbuf)
    ]
    freed = [None] * nbuf  # event: the GEMM that last read buffer i finished
    copy.wait_stream(compute)  # the buffers were allocated on the compute stream
    starts = list(range(0, n, rows))
    for i, r0 in enumerate(starts):
        r1 = min(r0 + rows, n)
        b = i % nbuf
        dbuf, sbuf = bufs[b]
        s0, s1 = r0 // 128, (r1 + 127) // 128
        with torch.cuda.stream(copy):
            if freed[b] is not None:
                copy.wait_event(freed[b])
            dbuf[: r1 - r0].copy_(data[r0:r1], non_blocking=True)
            sbuf[: s1 - s0].copy_(scale[s0:s1], non_blocking=True)
            landed = torch.cuda.Event()
            landed.record(copy)
        compute.wait_event(landed)
        _native.fp8_gemm_into(flattened, dbuf, sbuf, y, r0, r1 - r0, k)
        done = torch.cuda.Event()
        done.record(compute)
        freed[b] = done
    for dbuf, sbuf in bufs:  # the copy stream wrote them: keep them alive for it
        dbuf.record_stream(copy)
        sbuf.record_stream(copy)
    return y
