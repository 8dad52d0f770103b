"""Seeded random shapes through the product path against the oracle (bars of
tests/test_gemm_gpu.py).  Each case draws M in 1..300 (every dispatch regime:
row-partitioned, register-streamed, 17..128-row streaming, prefill), N and K
anywhere from one partial 16-row block / 128-wide chunk to a few thousand
(ragged and aligned), the scale dtype, and whether the weight is a row view
of a larger fused weight (row strides) or a load-time tiled copy."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd.kernels import tile_fp8_weight, tile_int4_weight

from . import test_gemm_gpu as tg

pytestmark = pytest.mark.gpu

SDTS = (torch.bfloat16, torch.float16, torch.float32)


def _draw(seed):
    r = np.random.default_rng(seed)
    m = int(r.choice([1, 2, 3, 5, 8, 13, 16, 17, 31, 33, 48, 64, 65, 100, 128, 129, 200, 300]))
    if r.random() < 0.5:
        n = int(r.integers(1, 200)) * 16
        k = int(r.integers(1, 24)) * 128
    else:
        n = int(r.integers(1, 3000))
        k = int(r.integers(1, 3000))
    return r, m, n, k, SDTS[int(r.integers(0, 3))]


@pytest.mark.parametrize("seed", range(24))
def test_int4_random_shape(seed):
    dev = tg._cuda()
    r, m, n, k, sdt = _draw(1000 + seed)
    w, x, xb, packed, scale, zero, _ = tg.int4_case(np.random.default_rng(seed), m, n, k, dev, sdt)
    ref = tg.int4_ref(xb, packed, scale, zero, n, k)
    tg.assert_gemm_close(hs.awq_linear(x, w), ref, what=f"int4 seed {seed}: {m}x{n}x{k} {sdt}")
    if n % 16 == 0 and k % 128 == 0 and r.random() < 0.5:
        tg.assert_gemm_close(hs.awq_linear(x, tile_int4_weight(w)), ref, what=f"int4 tiled seed {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_fp8_random_shape(seed):
    dev = tg._cuda()
    r, m, n, k, sdt = _draw(2000 + seed)
    w, x, xb, data, scale = tg.fp8_case(np.random.default_rng(seed), m, n, k, dev, sdt)
    ref = tg.fp8_ref(xb, data, scale, n, k)
    tg.assert_gemm_close(hs.fp8_linear(x, w), ref, what=f"fp8 seed {seed}: {m}x{n}x{k} {sdt}")
    if n % 16 == 0 and k % 128 == 0 and r.random() < 0.5:
        tg.assert_gemm_close(hs.fp8_linear(x, tile_fp8_weight(w)), ref, what=f"fp8 tiled seed {seed}")


@pytest.mark.parametrize("seed", range(8))
def test_int4_random_split_views(seed):
    """Row views of a fused weight at random 8-aligned offsets (row strides)."""
    dev = tg._cuda()
    r = np.random.default_rng(3000 + seed)
    m = int(r.choice([1, 7, 16, 40, 64, 130]))
    k = int(r.integers(1, 12)) * 128
    sizes = tuple(int(v) * 8 for v in r.integers(1, 120, size=3))
    n = sum(sizes)
    w, x, xb, packed, scale, zero, _ = tg.int4_case(np.random.default_rng(seed), m, n, k, dev)
    ref = tg.int4_ref(xb, packed, scale, zero, n, k)
    start = 0
    for part in hs.split_linear_weight(w, sizes):
        y = hs.awq_linear(x, part)
        sub = np.asarray(ref)[:, start : start + part.original_shape[0]].view(tg.RefArray)
        sub.exact = ref.exact[:, start : start + part.original_shape[0]]
        tg.assert_gemm_close(y, sub, what=f"view seed {seed} rows {start}+{part.original_shape[0]}")
        start += part.original_shape[0]
