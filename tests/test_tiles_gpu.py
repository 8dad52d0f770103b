"""Load-time tiled weight copies (hydraserve_amd/kernels/tiles.py) read by the
block-major decode kernel (hs_int4_gemm_tiled / hs_fp8_gemm_tiled), against
the oracle with the bars of tests/test_gemm_gpu.py: every M the kernel takes
(1..16), partitions of whole 16-row tiles, all scale dtypes, the full gate_up
shape, and shapes the kernel does not take (which fall back to the row-major
weight in the same call)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd.kernels import tile_fp8_weight, tile_int4_weight

from . import test_gemm_gpu as tg

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 17, 64, 300])
@pytest.mark.parametrize("n,k", [(4096, 1024), (2064, 2048)])
def test_int4_tiled_matches_oracle(m, n, k):
    dev = tg._cuda()
    rng = np.random.default_rng(31 * m + n)
    w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev)
    wt = tile_int4_weight(w)
    y = hs.awq_linear(x, wt)
    tg.assert_gemm_close(y, tg.int4_ref(xb, packed, scale, zero, n, k), what=f"tiled int4 {m}x{n}x{k}")


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_int4_tiled_other_scale_dtypes(sdt):
    dev = tg._cuda()
    rng = np.random.default_rng(77)
    m, n, k = 4, 2048, 2048
    w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, sdt)
    tg.assert_gemm_close(hs.awq_linear(x, tile_int4_weight(w)), tg.int4_ref(xb, packed, scale, zero, n, k))


@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
def test_fp8_tiled_matches_oracle(m, sdt):
    dev = tg._cuda()
    rng = np.random.default_rng(5 * m)
    n, k = 4096, 2048
    w, x, xb, data, scale = tg.fp8_case(rng, m, n, k, dev, sdt)
    tg.assert_gemm_close(hs.fp8_linear(x, tile_fp8_weight(w)), tg.fp8_ref(xb, data, scale, n, k), what=f"tiled fp8 {m}")


@pytest.mark.parametrize("m", [1, 4, 16])
def test_int4_tiled_gate_up_full_shape(m):
    dev = tg._cuda()
    n, k = 34816, 5120
    g = torch.Generator(device="cpu").manual_seed(700 + m)
    packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int32)
    zero = torch.randint(-(2**31), 2**31 - 1, (n // 8, k // 128), generator=g, dtype=torch.int32)
    scale = (torch.rand(n, k // 128, generator=g) * 9e-3 + 1e-3).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = hs.PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
    y = hs.awq_linear(x.to(dev), tile_int4_weight(w)).cpu()
    y0 = hs.awq_linear(x.to(dev), w).cpu()
    cols = tg._tile_columns(n, m)
    from oracle import quant_oracle as qo

    zp = qo.unpack_zero_points(zero.numpy(), n)[cols].astype(np.int32)
    q = qo.unpack_int4_rows(packed.numpy()[cols], k).astype(np.int32)
    s = scale.float().numpy()[cols]
    gi = np.arange(k) // 128
    w_exact = (q - zp[:, gi]).astype(np.float64) * s[:, gi]
    wd = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits((q - zp[:, gi]).astype(np.float32) * s[:, gi]))
    ref = qo.gemm_f64(x.float().numpy(), wd).view(tg.RefArray)
    ref.exact = x.float().numpy().astype(np.float64) @ w_exact.T
    tg.assert_gemm_close(y[:, cols], ref, what=f"tiled gate_up M={m}")
    # same per-row arithmetic as the row-major path: identical bits
    assert torch.equal(y.view(torch.int16), y0.view(torch.int16))
