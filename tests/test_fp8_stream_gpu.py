"""Host-resident FP8 weights streamed with the copy overlapping the GEMM
(hydraserve_amd/kernels/fp8_stream.py; reference staging at
hydraserve/kernels/fp8.py:32-41, offload planner runtime.py:182-236).

The streamed result is checked against the float64 oracle with the bars of
tests/test_gemm_gpu.py, on ragged shapes (a partial last slab and a partial
last scale block), with many slabs (the two staging buffers reused), both
scale dtypes, and against the device-resident path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd.kernels import pin_fp8_weight
from hydraserve_amd.kernels.fp8_stream import is_pinned_weight, streamed_fp8_gemm
from hydraserve_amd.model.weights import BlockScaledFP8Weight

from . import test_gemm_gpu as tg
from . import _synth

pytestmark = pytest.mark.gpu


def _host_weight(rng, n, k, sdt):
    data, s = _synth.fp8_weight(rng, n, k)
    w = BlockScaledFP8Weight(torch.from_numpy(data).view(torch.float8_e4m3fn), torch.from_numpy(s).to(sdt), (n, k))
    return w, data


@pytest.mark.parametrize("m,n,k,slab", [(3, 300, 259, 128), (16, 1024, 1024, 256), (64, 4224, 640, 1024), (300, 640, 384, 128)])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
def test_streamed_matches_oracle(m, n, k, slab, sdt):
    dev = tg._cuda()
    rng = np.random.default_rng(m + n + k + slab)
    w, data = _host_weight(rng, n, k, sdt)
    pw = pin_fp8_weight(w)
    assert is_pinned_weight(pw) and not is_pinned_weight(w)
    xb = _synth.x_bf16(rng, m, k)
    x = tg.t_bf16(xb, dev)
    y = streamed_fp8_gemm(x, pw, slab_rows=slab)
    torch.cuda.synchronize()
    tg.assert_gemm_close(y, tg.fp8_ref(xb, data, pw.scale_inv, n, k), what=f"streamed {m}x{n}x{k} slab {slab}")
    # the drop-in (streamed for a pinned host weight from 128 rows, staged below)
    y2 = hs.fp8_linear(x, pw)
    tg.assert_gemm_close(y2, tg.fp8_ref(xb, data, pw.scale_inv, n, k), what="fp8_linear pinned")
    # and agrees with the device-resident weight
    wd = BlockScaledFP8Weight(pw.data.to(dev), pw.scale_inv.to(dev), (n, k))
    ref = hs.fp8_linear(x, wd).float()
    assert (y2.float() - ref).abs().max().item() <= 2e-2 * max(ref.abs().max().item(), 1e-6)


def test_streamed_repeated_calls_and_pageable_fallback():
    """Back-to-back streamed calls reuse the copy stream; a pageable host
    weight takes the reference's whole-weight staging."""
    dev = tg._cuda()
    rng = np.random.default_rng(5)
    n, k, m = 2048, 512, 8
    w, data = _host_weight(rng, n, k, torch.float32)
    pw = pin_fp8_weight(w)
    xb = _synth.x_bf16(rng, m, k)
    x = tg.t_bf16(xb, dev)
    ref = tg.fp8_ref(xb, data, pw.scale_inv, n, k)
    outs = [streamed_fp8_gemm(x, pw, slab_rows=128) for _ in range(4)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    tg.assert_gemm_close(outs[0], ref)
    tg.assert_gemm_close(hs.fp8_linear(x, w), ref, what="pageable staging")


def test_slab_rows_must_be_whole_scale_blocks():
    dev = tg._cuda()
    rng = np.random.default_rng(6)
    w, _ = _host_weight(rng, 256, 256, torch.float32)
    with pytest.raises(ValueError, match="multiple of 128"):
        streamed_fp8_gemm(torch.zeros(1, 256, dtype=torch.bfloat16, device=dev), pin_fp8_weight(w), slab_rows=100)
