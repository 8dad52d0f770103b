"""Gate_up projection with fused SiLU-and-mul (hydraserve_amd/kernels/mlp.py).

CPU: the load-time interleave is a lossless row permutation (checked through
the oracle's unpack and dequantizer, and by its inverse), and the fused C
entry point validates its arguments like hs_int4_gemm.
GPU: hs_int4_gemm_silu_mul (1..16 rows in the block-major GEMV or the
row-partitioned kernel,
17..128 rows in the LDS-DMA streaming kernel, from 129 rows in the 256x256-tile
prefill kernel) and the unfused fallback against
the oracle, with the bars of tests/test_gemm_gpu.py applied to
silu(bf16(gate)) * bf16(up) computed from the float64 oracle GEMM, and
against the product path's own unfused sequence (awq_linear on the original
weight, chunk, silu_and_mul), which the reference runs
(hydraserve/model/runtime.py:1202-1210).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from hydraserve_amd import _native
from hydraserve_amd.kernels.mlp import deinterleave_gate_up, interleave_gate_up, silu_and_mul
from hydraserve_amd.model.weights import PackedInt4Weight
from oracle import quant_oracle as qo

from . import _synth


def _weight_cpu(rng, n, k):
    packed, scale_bits, zero, _, _ = _synth.int4_weight(rng, n, k)
    scale = torch.from_numpy(scale_bits.view(np.int16)).view(torch.bfloat16)
    return PackedInt4Weight(torch.from_numpy(packed.view(np.int32)), scale, torch.from_numpy(zero.view(np.int32)), (n, k))


def _dequant_np(w):
    n, k = w.original_shape
    s = w.scale.float().numpy()
    q = qo.unpack_int4_rows(w.packed.numpy().view(np.uint32), k).astype(np.int32)
    z = qo.unpack_zero_points(w.zero_point.numpy().view(np.uint32), n).astype(np.int32)
    g = np.arange(k) // 128
    return (q - z[:, g]).astype(np.float64) * s[:, g]


def test_interleave_is_a_lossless_row_permutation():
    rng = np.random.default_rng(5)
    n, k = 96, 256
    w = _weight_cpu(rng, n, k)
    wi = interleave_gate_up(w)
    dense, dense_i = _dequant_np(w), _dequant_np(wi)
    half = n // 2
    for j in range(half // 16):
        for r in range(16):
            np.testing.assert_array_equal(dense_i[32 * j + r], dense[16 * j + r])
            np.testing.assert_array_equal(dense_i[32 * j + 16 + r], dense[half + 16 * j + r])
    back = deinterleave_gate_up(wi)
    for a, b in ((w.packed, back.packed), (w.scale, back.scale), (w.zero_point, back.zero_point)):
        assert torch.equal(a, b)


def test_interleave_rejects_odd_halves():
    w = _weight_cpu(np.random.default_rng(6), 48, 128)
    with pytest.raises(ValueError, match="multiple of 32"):
        interleave_gate_up(w)


def test_silu_and_mul_reference_recipe():
    # tests/test_triton_kernels.py:27-33 (seed 21, shapes, atol = rtol = 2e-2)
    for shape in [(1, 1, 128), (4, 3, 9216)]:
        torch.manual_seed(21)
        gate = torch.randn(shape, dtype=torch.bfloat16)
        up = torch.randn_like(gate)
        expected = gate.float() * torch.sigmoid(gate.float()) * up.float()
        torch.testing.assert_close(silu_and_mul(gate, up).float(), expected, atol=2e-2, rtol=2e-2)


def test_fused_entry_point_validates_arguments():
    L = _native.lib()
    # N not a multiple of 32 -> HS_EINVAL; group != 128 -> HS_EUNSUPPORTED; M == 0 -> OK
    assert L.hs_int4_gemm_silu_mul(1, 256, 1, 32, 1, 2, 0, 1, 2, 1, 64, 20, 48, 256, 128, 1, 1 << 20, None) == 1
    assert L.hs_int4_gemm_silu_mul(1, 256, 1, 32, 1, 2, 0, 1, 2, 1, 64, 20, 64, 256, 64, 1, 1 << 20, None) == 3
    assert L.hs_int4_gemm_silu_mul(None, 256, None, 32, None, 2, 0, None, 2, None, 64, 20, 64, 256, 128, None, 0, None) == 1
    assert L.hs_int4_gemm_silu_mul(1, 256, 1, 32, 1, 2, 0, 1, 2, 1, 32, 0, 64, 256, 128, 1, 1 << 20, None) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4, 7, 8, 12, 16, 17, 32, 64, 100, 128, 130, 300])
@pytest.mark.parametrize("n,k", [(2048, 1024), (1536, 640), (2048, 5120)])
def test_fused_gate_up_silu_mul(m, n, k):
    _check_fused(m, n, k, torch.bfloat16)


# fp16 and fp32 scales run their own instances of every fused kernel (block-
# major and row-partitioned decode at 4 and 16 rows, streaming at 64, prefill
# at 300)
@pytest.mark.gpu
@pytest.mark.parametrize("m", [4, 16, 64, 300])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_fused_gate_up_silu_mul_scale_dtypes(m, scale_dtype):
    _check_fused(m, 2048, 5120, scale_dtype)


def _check_fused(m, n, k, scale_dtype):
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    import hydraserve_amd as hs
    from hydraserve_amd.kernels import awq_gate_up_silu_mul

    from . import test_gemm_gpu as tg

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7000 + m)
    w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, scale_dtype)
    wi = interleave_gate_up(w)
    out = awq_gate_up_silu_mul(x, wi)
    torch.cuda.synchronize()
    if k % 128 == 0 and k // 128 >= 8:  # the fused entry point itself takes these
        from hydraserve_amd import _native

        assert _native.int4_gemm_silu_mul(
            x.reshape(-1, k).contiguous(), wi.packed, wi.scale, wi.zero_point, n, k, 128
        ) is not None
    assert out.shape == (m, n // 2) and out.dtype == torch.bfloat16
    # oracle: bf16 gate/up from the float64 GEMM, then the activation in float64
    # (from the reference's bf16-rounded weights, and from the exact weights
    # that the decode kernels' group rewrite uses: either must meet the bar)
    y = tg.int4_ref(xb, packed, scale, zero, n, k)

    def act(yy):
        gu = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits(np.asarray(yy, dtype=np.float32))).astype(np.float64)
        g, u = gu[:, : n // 2], gu[:, n // 2 :]
        return g / (1.0 + np.exp(-g)) * u

    ref = act(y).view(tg.RefArray)
    ref.exact = act(y.exact)
    tg.assert_gemm_close(out, ref, what=f"fused silu_mul M={m} N={n} K={k} scales={scale_dtype}")
    # the product path's unfused sequence on the original weight
    gate, up = hs.awq_linear(x, w).chunk(2, dim=-1)
    unfused = silu_and_mul(gate.contiguous(), up.contiguous())
    # gate and up are bf16-rounded by two kernels with different summation
    # orders, so a 1-ulp flip of either moves the product by ~2^-8 of the
    # output's magnitude: the absolute bar scales with it
    mag = max(1.0, unfused.float().abs().max().item())
    torch.testing.assert_close(out.float(), unfused.float(), atol=2e-2 * mag, rtol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("m", [1, 8, 16, 64, 2048])
def test_fused_gate_up_silu_mul_full_shape(m, tiled):
    """The benchmarked shape, gate_up 5120 -> 34816: at 1..16 rows the
    block-major kernel's largest row partitions and the row-partitioned
    kernel's widest SiLU instance, at 64 the streaming kernel's two-column-block
    store, at 2048 the prefill SiLU instance.  ``tiled``: the tiled copy of the
    interleaved weight, read by the tiled decode kernel's fused store up to 64
    rows and by the prefill SiLU instance's tiled loads at 2048.  The oracle
    recomputes gate and up for the output columns of
    test_gemm_gpu._tile_columns (every tile)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    from hydraserve_amd.kernels import awq_gate_up_silu_mul

    from . import test_gemm_gpu as tg

    dev = torch.device("cuda", 0)
    n, k = 34816, 5120
    half = n // 2
    g = torch.Generator(device="cpu").manual_seed(900 + m)
    groups = k // 128
    packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int32)
    zero = torch.randint(-(2**31), 2**31 - 1, (n // 8, groups), generator=g, dtype=torch.int32)
    scale = (torch.rand(n, groups, generator=g) * 9e-3 + 1e-3).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = PackedInt4Weight(packed.to(dev), scale.to(dev), zero.to(dev), (n, k))
    wi = interleave_gate_up(w)
    from hydraserve_amd import _native

    if tiled:
        from hydraserve_amd.kernels import tile_int4_weight

        wi = tile_int4_weight(wi)
        assert _native.int4_gemm_silu_mul(
            x.to(dev), wi.packed, wi.scale, wi.zero_point, n, k, 128, tiles=wi.tiles) is not None
    else:
        assert _native.int4_gemm_silu_mul(x.to(dev), wi.packed, wi.scale, wi.zero_point, n, k, 128) is not None
    out = awq_gate_up_silu_mul(x.to(dev), wi).cpu()
    assert out.shape == (m, half)
    cols = tg._tile_columns(half, m)
    rows = np.concatenate([cols, half + cols])
    zp = qo.unpack_zero_points(zero.numpy(), n)[rows].astype(np.int32)
    q = qo.unpack_int4_rows(packed.numpy()[rows], k).astype(np.int32)
    s = scale.float().numpy()[rows]
    gi = np.arange(k) // 128
    xf = x.float().numpy()
    w_exact = (q - zp[:, gi]).astype(np.float64) * s[:, gi]
    wd = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits((q - zp[:, gi]).astype(np.float32) * s[:, gi]))
    y = qo.gemm_f64(xf, wd)
    y_exact = xf.astype(np.float64) @ w_exact.T

    def act(yy):
        gu = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits(np.asarray(yy, dtype=np.float32))).astype(np.float64)
        gate, up = gu[:, : len(cols)], gu[:, len(cols) :]
        return gate / (1.0 + np.exp(-gate)) * up

    ref = act(y).view(tg.RefArray)
    ref.exact = act(y_exact)
    tg.assert_gemm_close(out[:, cols], ref, what=f"fused silu_mul full shape M={m}")
