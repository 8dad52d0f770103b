"""ctypes binding of libhydraserve_amd.so (C ABI in include/hydraserve_amd.h).

The library is loaded lazily on first use and every failure is loud: a
missing library raises, a non-zero return code raises ``RuntimeError`` with
the library's message.  There is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("HYDRASERVE_AMD_LIB", Path(__file__).resolve().parent / "libhydraserve_amd.so"))

HS_KIND_INT4 = 0
HS_KIND_FP8 = 1
HS_DT_BF16 = 0
HS_DT_F16 = 1
HS_DT_F32 = 2
HS_EUNSUPPORTED = 3

# (name, restype, argtypes) for every symbol the header declares.
_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_I = ctypes.c_int
SIGNATURES = {
    "hs_abi_version": (_I, []),
    "hs_error_string": (ctypes.c_char_p, [_I]),
    "hs_gemm_workspace_bytes": (_I64, [_I, _I, _I, _I]),
    "hs_int4_gemm": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P, _I64, _P]),
    "hs_int4_gemm_noalloc": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P]),
    "hs_int4_gemm_silu_mul": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P, _I64, _P]),
    "hs_int4_gemm_silu_mul_tiled": (
        _I, [_P, _I64, _P, _I64, _P, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P, _I64, _P]),
    "hs_fp8_gemm": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _P, _I64, _I, _I, _I, _P, _I64, _P]),
    "hs_int4_gemm_tiled": (_I, [_P, _I64, _P, _I64, _P, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P, _I64, _P]),
    "hs_fp8_gemm_tiled": (_I, [_P, _I64, _P, _I64, _P, _P, _I64, _I, _P, _I64, _I, _I, _I, _P, _I64, _P]),
    "hs_int4_dequant": (_I, [_P, _I64, _P, _I64, _I, _P, _I64, _P, _I64, _I, _I, _I, _I, _P]),
    "hs_fp8_dequant": (_I, [_P, _I64, _P, _I64, _I, _P, _I64, _I, _I, _I, _P]),
    "hs_hbm_read_probe": (_I, [_P, _I64, _P, _I64, _I, _P]),
}
ABI_VERSION = 1

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m hydraserve_amd.build` "
                    "(hydraserve_amd has no non-HIP execution path)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.hs_abi_version() != ABI_VERSION:
                raise RuntimeError("libhydraserve_amd.so ABI version mismatch; rebuild it")
            _lib = handle
    return _lib


def check(code: int, what: str) -> None:
    if code != 0:
        msg = lib().hs_error_string(code).decode()
        raise RuntimeError(f"{what} failed (code {code}): {msg}")


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.bfloat16:
        return HS_DT_BF16
    if dtype == torch.float16:
        return HS_DT_F16
    if dtype == torch.float32:
        return HS_DT_F32
    raise TypeError(f"unsupported scale/output dtype {dtype}")


class _Workspaces:
    """Zero-filled device workspaces, one per (device, stream).

    The kernels leave a workspace zero-filled when they finish, so a buffer is
    filled once at allocation and reused.  Calls on one stream are ordered, so
    sharing within a stream is safe; different streams get different buffers.
    A workspace only grows; growing allocates, so warm every shape up before
    capturing a HIP graph.
    """

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, int], object] = {}
        self._lock = threading.Lock()

    def get(self, device, stream_ptr: int, nbytes: int):
        import torch

        key = (device.index, stream_ptr)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                if buf is not None:
                    size = max(size, 2 * buf.numel())
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


workspaces = _Workspaces()


def int4_gemm(x, packed, scale, zero_point, n: int, k: int, group: int, tiles=None):
    """Y[M, N] (bf16) for a contiguous bf16 x [M, K] on the current stream
    (``tiles``: the load-time tiled copy of packed, kernels/tiles.py)."""
    import torch

    m = x.shape[0]
    y = torch.empty(m, n, device=x.device, dtype=x.dtype)
    if m == 0 or n == 0:
        return y
    L = lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    need = L.hs_gemm_workspace_bytes(HS_KIND_INT4, m, n, k)
    ws = workspaces.get(x.device, stream, need)
    if tiles is not None:
        check(
            L.hs_int4_gemm_tiled(
                x.data_ptr(), x.stride(0), packed.data_ptr(), packed.stride(0), tiles.data_ptr(),
                scale.data_ptr(), scale.stride(0), dtype_code(scale.dtype),
                zero_point.data_ptr(), zero_point.stride(0),
                y.data_ptr(), y.stride(0), m, n, k, group,
                ws.data_ptr(), ws.numel(), stream,
            ),
            "hs_int4_gemm_tiled",
        )
        return y
    check(
        L.hs_int4_gemm(
            x.data_ptr(), x.stride(0), packed.data_ptr(), packed.stride(0),
            scale.data_ptr(), scale.stride(0), dtype_code(scale.dtype),
            zero_point.data_ptr(), zero_point.stride(0),
            y.data_ptr(), y.stride(0), m, n, k, group,
            ws.data_ptr(), ws.numel(), stream,
        ),
        "hs_int4_gemm",
    )
    return y


def int4_gemm_silu_mul(x, packed, scale, zero_point, n: int, k: int, group: int, tiles=None):
    """silu(gate) * up [M, N/2] (bf16) on a gate/up-interleaved weight of N rows,
    or None where the fused kernel does not apply (HS_EUNSUPPORTED)
    (``tiles``: the load-time tiled copy of the interleaved packed words)."""
    import torch

    m = x.shape[0]
    y = torch.empty(m, n // 2, device=x.device, dtype=x.dtype)
    if m == 0 or n == 0:
        return y
    L = lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    need = L.hs_gemm_workspace_bytes(HS_KIND_INT4, m, n, k)
    ws = workspaces.get(x.device, stream, need)
    name = "hs_int4_gemm_silu_mul" if tiles is None else "hs_int4_gemm_silu_mul_tiled"
    w_args = (packed.data_ptr(), packed.stride(0)) if tiles is None else (
        packed.data_ptr(), packed.stride(0), tiles.data_ptr())
    rc = getattr(L, name)(
        x.data_ptr(), x.stride(0), *w_args,
        scale.data_ptr(), scale.stride(0), dtype_code(scale.dtype),
        zero_point.data_ptr(), zero_point.stride(0),
        y.data_ptr(), y.stride(0), m, n, k, group,
        ws.data_ptr(), ws.numel(), stream,
    )
    if rc == HS_EUNSUPPORTED:
        return None
    check(rc, name)
    return y


def fp8_gemm(x, data_u8, scale_inv, n: int, k: int, tiles=None):
    import torch

    m = x.shape[0]
    y = torch.empty(m, n, device=x.device, dtype=x.dtype)
    if m == 0 or n == 0:
        return y
    L = lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    need = L.hs_gemm_workspace_bytes(HS_KIND_FP8, m, n, k)
    ws = workspaces.get(x.device, stream, need)
    if tiles is not None:
        check(
            L.hs_fp8_gemm_tiled(
                x.data_ptr(), x.stride(0), data_u8.data_ptr(), data_u8.stride(0), tiles.data_ptr(),
                scale_inv.data_ptr(), scale_inv.stride(0), dtype_code(scale_inv.dtype),
                y.data_ptr(), y.stride(0), m, n, k,
                ws.data_ptr(), ws.numel(), stream,
            ),
            "hs_fp8_gemm_tiled",
        )
        return y
    check(
        L.hs_fp8_gemm(
            x.data_ptr(), x.stride(0), data_u8.data_ptr(), data_u8.stride(0),
            scale_inv.data_ptr(), scale_inv.stride(0), dtype_code(scale_inv.dtype),
            y.data_ptr(), y.stride(0), m, n, k,
            ws.data_ptr(), ws.numel(), stream,
        ),
        "hs_fp8_gemm",
    )
    return y


def fp8_gemm_into(x, data_u8, scale_inv, y, col0: int, n: int, k: int) -> None:
    """Y[:, col0:col0+n] = x . W^T for an FP8 row slab W [n, K] (its own scale
    rows), written in place into a wider bf16 output y (row stride y.stride(0))."""
    import torch

    m = x.shape[0]
    if m == 0 or n == 0:
        return
    L = lib()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    need = L.hs_gemm_workspace_bytes(HS_KIND_FP8, m, n, k)
    ws = workspaces.get(x.device, stream, need)
    check(
        L.hs_fp8_gemm(
            x.data_ptr(), x.stride(0), data_u8.data_ptr(), data_u8.stride(0),
            scale_inv.data_ptr(), scale_inv.stride(0), dtype_code(scale_inv.dtype),
            y.data_ptr() + col0 * y.element_size(), y.stride(0), m, n, k,
            ws.data_ptr(), ws.numel(), stream,
        ),
        "hs_fp8_gemm",
    )


def int4_dequant(packed, scale, zero_point, n: int, k: int, group: int, out_dtype):
    import torch

    out = torch.empty(n, k, device=packed.device, dtype=out_dtype)
    if n == 0 or k == 0:
        return out
    stream = torch.cuda.current_stream(packed.device).cuda_stream
    check(
        lib().hs_int4_dequant(
            packed.data_ptr(), packed.stride(0), scale.data_ptr(), scale.stride(0), dtype_code(scale.dtype),
            zero_point.data_ptr(), zero_point.stride(0), out.data_ptr(), out.stride(0), dtype_code(out_dtype),
            n, k, group, stream,
        ),
        "hs_int4_dequant",
    )
    return out


def fp8_dequant(data_u8, scale_inv, n: int, k: int, out_dtype):
    import torch

    out = torch.empty(n, k, device=data_u8.device, dtype=out_dtype)
    if n == 0 or k == 0:
        return out
    stream = torch.cuda.current_stream(data_u8.device).cuda_stream
    check(
        lib().hs_fp8_dequant(
            data_u8.data_ptr(), data_u8.stride(0), scale_inv.data_ptr(), scale_inv.stride(0),
            dtype_code(scale_inv.dtype), out.data_ptr(), out.stride(0), dtype_code(out_dtype), n, k, stream,
        ),
        "hs_fp8_dequant",
    )
    return out


def hbm_read_probe(src, sink, blocks: int) -> None:
    """One streaming read of every byte of ``src`` (a contiguous CUDA tensor)."""
    import torch

    stream = torch.cuda.current_stream(src.device).cuda_stream
    nbytes = src.numel() * src.element_size()
    check(
        lib().hs_hbm_read_probe(src.data_ptr(), nbytes, sink.data_ptr(), sink.numel() * sink.element_size(), blocks, stream),
        "hs_hbm_read_probe",
    )
