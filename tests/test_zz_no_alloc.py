"""hs_int4_gemm_noalloc (fixed per-GPU scratch, no allocation) against
hs_int4_gemm with a caller workspace, through the C ABI.

Both entry points run the same kernels with the same plan, so the outputs
must be bit-identical.  Two calls in a row, the second smaller, check that the
scratch's leftover contents from the first call do not leak into the second
(the counters return to zero at the end of every call; partial tiles are
overwritten before they are read).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from hydraserve_amd import _native

from . import test_gemm_gpu as tg

pytestmark = pytest.mark.gpu

HS_ESCRATCH = 4


def _noalloc(x, w, n, k):
    L = _native.lib()
    y = torch.empty(x.shape[0], n, device=x.device, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = L.hs_int4_gemm_noalloc(
        x.data_ptr(), x.stride(0), w.packed.data_ptr(), w.packed.stride(0),
        w.scale.data_ptr(), w.scale.stride(0), _native.dtype_code(w.scale.dtype),
        w.zero_point.data_ptr(), w.zero_point.stride(0), y.data_ptr(), y.stride(0),
        x.shape[0], n, k, 128, stream,
    )
    return rc, y


def _with_workspace(x, w, n, k):
    return _native.int4_gemm(x, w.packed, w.scale, w.zero_point, n, k, 128)


@pytest.mark.parametrize(
    "first,second",
    [
        ((64, 34816, 5120), (17, 4096, 2048)),   # streaming 17..128-row kernel, stream-K partials
        ((64, 5120, 17408), (9, 5120, 8192)),    # register-streamed kernel on narrow outputs
        ((128, 4096, 4096), (33, 1024, 1024)),
        ((16, 34816, 5120), (1, 2048, 1024)),    # row-partitioned kernels (no workspace use)
    ],
)
def test_noalloc_matches_workspace_entry_point(first, second):
    dev = tg._cuda()
    for i, (m, n, k) in enumerate((first, second)):
        print(f"noalloc case {i}: M={m} N={n} K={k}", flush=True)
        rng = np.random.default_rng(m * 31 + n + k)
        w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev)
        rc, y = _noalloc(x, w, n, k)
        assert rc == 0, _native.lib().hs_error_string(rc)
        torch.cuda.synchronize()
        want = _with_workspace(x, w, n, k)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"case {i}"
        if n * k <= 4096 * 4096:
            tg.assert_gemm_close(y, tg.int4_ref(xb, packed, scale, zero, n, k), what=f"noalloc {m}x{n}x{k}")


def test_noalloc_rejects_problems_larger_than_its_scratch():
    dev = tg._cuda()
    m, n, k = 2048, 34816, 5120  # the prefill plan's partial tiles exceed 40 MiB
    x = torch.zeros(m, k, device=dev, dtype=torch.bfloat16)
    w = type("W", (), {})()
    w.packed = torch.zeros(n, k // 8, device=dev, dtype=torch.int32)
    w.scale = torch.zeros(n, k // 128, device=dev, dtype=torch.bfloat16)
    w.zero_point = torch.zeros(n // 8, k // 128, device=dev, dtype=torch.int32)
    rc, _ = _noalloc(x, w, n, k)
    assert rc == HS_ESCRATCH
    assert b"scratch" in _native.lib().hs_error_string(rc)
