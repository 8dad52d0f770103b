"""Load-time tiled weight copies (hydraserve_amd/kernels/tiles.py) read by the
tiled decode kernel (hs_int4_gemm_tiled / hs_fp8_gemm_tiled,
csrc/qgemm_tiled.hip), against the oracle with the bars of
tests/test_gemm_gpu.py: every row-block count (1..64 rows, partial blocks),
the group rewrite (<= 32 rows) and exact dequantisation (33..64 rows), all
scale dtypes, tile groups with waves of 0..2 tiles, K split across
workgroups (settled partials) with chunk counts that leave a ring remainder,
the full BASELINE shapes, and shapes the kernel does not take (which fall
back to the row-major weight in the same call)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd.kernels import tile_fp8_weight, tile_int4_weight
from oracle import quant_oracle as qo

from . import test_gemm_gpu as tg

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("splits", [None, "3"])
def test_tiled_kernel_small_shapes_forced(splits):
    """Small shapes forced through the tiled kernel in a child process
    (tests/_tiles_check.py, HS_TM_MIN_M=1): the plan keeps them row-major by
    default.  HS_TM_S=3 forces three K ranges where the shape allows, so K
    ranges start at chunks that are not multiples of the 8-chunk scale
    rounds."""
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    env = dict(os.environ, HS_TM_MIN_M="1")
    if splits:
        env["HS_TM_S"] = splits
    res = subprocess.run([sys.executable, "-u", "-m", "tests._tiles_check"], cwd=ROOT, env=env,
                         capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert res.stdout.strip().endswith("ok"), res.stdout[-2000:]


@pytest.mark.parametrize("m", [1, 8, 300])
def test_int4_tiled_weight_default_dispatch(m):
    """A tiled weight through the default plan (row-major kernels for small
    weights and above 64 rows)."""
    dev = tg._cuda()
    rng = np.random.default_rng(17 * m)
    n, k = 2064, 2048
    w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev)
    tg.assert_gemm_close(hs.awq_linear(x, tile_int4_weight(w)), tg.int4_ref(xb, packed, scale, zero, n, k))


def _int4_full(n, k, m, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int32)
    zero = torch.randint(-(2**31), 2**31 - 1, (n // 8, k // 128), generator=g, dtype=torch.int32)
    scale = (torch.rand(n, k // 128, generator=g) * 9e-3 + 1e-3).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return packed, zero, scale, x


def _int4_sampled_ref(packed, zero, scale, x, n, k, cols):
    zp = qo.unpack_zero_points(zero.numpy(), n)[cols].astype(np.int32)
    q = qo.unpack_int4_rows(packed.numpy()[cols], k).astype(np.int32)
    s = scale.float().numpy()[cols]
    gi = np.arange(k) // 128
    wd = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits((q - zp[:, gi]).astype(np.float32) * s[:, gi]))
    ref = qo.gemm_f64(x.float().numpy(), wd).view(tg.RefArray)
    ref.exact = x.float().numpy().astype(np.float64) @ ((q - zp[:, gi]).astype(np.float64) * s[:, gi]).T
    return ref


@pytest.mark.parametrize("m", [1, 8, 16, 32, 64])
@pytest.mark.parametrize(
    "n,k", [(34816, 5120), (5120, 17408), (10240, 5120), (5120, 8192), (12288, 5120), (4096, 4096)]
)
def test_int4_tiled_baseline_shapes(m, n, k):
    """Every BASELINE decode shape through the tiled copy: one column in every
    16-row tile plus the edges of every 256-wide block (tg._tile_columns)."""
    dev = tg._cuda()
    packed, zero, scale, x = _int4_full(n, k, m, 700 + m + n)
    w = hs.PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
    y = hs.awq_linear(x.to(dev), tile_int4_weight(w)).cpu()
    cols = tg._tile_columns(n, m)
    tg.assert_gemm_close(y[:, cols], _int4_sampled_ref(packed, zero, scale, x, n, k, cols),
                         what=f"tiled {n}x{k} M={m}")


@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("n,k", [(34816, 5120), (5120, 17408)])
def test_fp8_tiled_baseline_shapes(m, n, k):
    dev = tg._cuda()
    g = torch.Generator(device="cpu").manual_seed(m + n + 11)
    data = torch.randint(0, 256, (n, k), generator=g, dtype=torch.int32).to(torch.uint8)
    data[(data & 0x7F) == 0x7F] = 0x00
    scale = torch.rand((n + 127) // 128, (k + 127) // 128, generator=g) * 0.099 + 0.001
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = hs.BlockScaledFP8Weight(data.to(dev).view(torch.float8_e4m3fn), scale.to(dev), (n, k))
    y = hs.fp8_linear(x.to(dev), tile_fp8_weight(w)).cpu()
    cols = tg._tile_columns(n, m)
    wd = qo.decode_e4m3fn(data.numpy()[cols]) * scale.numpy()[(cols // 128)][:, np.arange(k) // 128]
    ref = qo.gemm_f64(x.float().numpy(), wd.astype(np.float32))
    tg.assert_gemm_close(y[:, cols], ref, what=f"tiled fp8 {n}x{k} M={m}")


@pytest.mark.parametrize("m", [16, 64])
def test_tiled_and_row_major_agree_and_replay_bitwise(m):
    """The tiled call agrees with the row-major call on the same weight within
    the output bar, and repeated tiled calls (split-K settles included) give
    identical bits."""
    dev = tg._cuda()
    n, k = 5120, 17408
    packed, zero, scale, x = _int4_full(n, k, m, 4242 + m)
    w = hs.PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
    wt = tile_int4_weight(w)
    xd = x.to(dev)
    y0 = hs.awq_linear(xd, w).float()
    y1 = hs.awq_linear(xd, wt)
    y2 = hs.awq_linear(xd, wt)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    diff = (y1.float() - y0).abs().max().item() / y0.abs().max().item()
    assert diff < 1e-2, diff


@pytest.mark.parametrize("kind", ["int4", "fp8"])
def test_tiled_row_split_qkv_m192(kind):
    """129..192 rows on a wide output with a tiled copy: 128 rows row-major and
    the upper 64 rows through the tiled kernel, sampled columns against the
    oracle."""
    dev = tg._cuda()
    n, k, m = 12288, 5120, 192
    cols = tg._tile_columns(n, 16)
    if kind == "int4":
        packed, zero, scale, x = _int4_full(n, k, m, 1921)
        w = hs.PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
        y = hs.awq_linear(x.to(dev), tile_int4_weight(w)).cpu()
        ref = _int4_sampled_ref(packed, zero, scale, x, n, k, cols)
    else:
        g = torch.Generator(device="cpu").manual_seed(1922)
        data = torch.randint(0, 256, (n, k), generator=g, dtype=torch.int32).to(torch.uint8)
        data[(data & 0x7F) == 0x7F] = 0x00
        scale = torch.rand(n // 128, k // 128, generator=g) * 0.099 + 0.001
        x = torch.randn(m, k, generator=g).to(torch.bfloat16)
        w = hs.BlockScaledFP8Weight(data.to(dev).view(torch.float8_e4m3fn), scale.to(dev), (n, k))
        y = hs.fp8_linear(x.to(dev), tile_fp8_weight(w)).cpu()
        wd = qo.decode_e4m3fn(data.numpy()[cols]) * scale.numpy()[(cols // 128)][:, np.arange(k) // 128]
        ref = qo.gemm_f64(x.float().numpy(), wd.astype(np.float32))
    tg.assert_gemm_close(y[:, cols], ref, what=f"tiled split {kind} M={m}")


@pytest.mark.parametrize("kind,scale_dtype", [("int4", torch.bfloat16), ("int4", torch.float16),
                                              ("int4", torch.float32), ("fp8", torch.float32),
                                              ("fp8", torch.bfloat16)])
@pytest.mark.parametrize("m,n,k", [(200, 2064, 2048), (300, 1040, 1280), (513, 784, 384)])
def test_prefill_reads_tiles(kind, scale_dtype, m, n, k):
    """Above 192 rows (129 on narrow outputs) the 256x256 prefill kernel reads
    the tiled copy when one is given: its bits equal those of the same kernel
    on the row-major weight (the same products in the same order), and the
    result meets the oracle bar.  N here is a multiple of 16 but not of 256
    (clamped tile rows) and K ranges end at odd 128-wide chunks."""
    dev = tg._cuda()
    rng = np.random.default_rng(m * 7 + n)
    if kind == "int4":
        w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, scale_dtype)
        y0 = hs.awq_linear(x, w)
        y1 = hs.awq_linear(x, tile_int4_weight(w))
        ref = tg.int4_ref(xb, packed, scale, zero, n, k)
    else:
        w, x, xb, data, scale = tg.fp8_case(rng, m, n, k, dev, scale_dtype)
        y0 = hs.fp8_linear(x, w)
        y1 = hs.fp8_linear(x, tile_fp8_weight(w))
        ref = tg.fp8_ref(xb, data, scale, n, k)
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), f"{kind} tiled prefill bits differ"
    tg.assert_gemm_close(y1, ref, what=f"tiled prefill {kind} M={m}")


@pytest.mark.parametrize("kind", ["int4", "fp8"])
def test_prefill_reads_tiles_baseline_gate_up(kind):
    """BASELINE gate_up (34816 x 5120) at 2048 rows: tiled and row-major
    weights give identical bits (split tiles settled across workgroups)."""
    dev = tg._cuda()
    n, k, m = 34816, 5120, 2048
    g = torch.Generator(device="cpu").manual_seed(2048)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(dev)
    if kind == "int4":
        packed, zero, scale, _ = _int4_full(n, k, 1, 2049)
        w = hs.PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
        y0, y1 = hs.awq_linear(x, w), hs.awq_linear(x, tile_int4_weight(w))
    else:
        data = torch.randint(0, 256, (n, k), generator=g, dtype=torch.int32).to(torch.uint8)
        data[(data & 0x7F) == 0x7F] = 0x00
        scale = torch.rand(n // 128, k // 128, generator=g) * 0.099 + 0.001
        w = hs.BlockScaledFP8Weight(data.to(dev).view(torch.float8_e4m3fn), scale.to(dev), (n, k))
        y0, y1 = hs.fp8_linear(x, w), hs.fp8_linear(x, tile_fp8_weight(w))
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
