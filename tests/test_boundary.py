"""CPU tests of the drop-in boundary: the C ABI, validation, fusion helpers.

No HIP kernel runs here.  Validation order and messages follow
hydraserve/kernels/awq.py:28-43 and hydraserve/kernels/fp8.py:28-62.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd import _native
from hydraserve_amd.model.weights import BlockScaledFP8Weight, PackedInt4Weight

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "hydraserve_amd.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(hs_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    syms = header_symbols()
    assert len(syms) >= 7
    handle = ctypes.CDLL(str(_native.LIB_PATH))
    for name in syms:
        assert hasattr(handle, name), name
    assert set(syms) == set(_native.SIGNATURES)


def test_abi_version_and_errors():
    L = _native.lib()
    assert L.hs_abi_version() == _native.ABI_VERSION
    assert L.hs_error_string(0) == b"success"
    assert b"workspace" in L.hs_error_string(2)


def test_c_validation_rejects_bad_args_without_launching():
    L = _native.lib()
    # group != 128
    assert L.hs_int4_gemm(1, 256, 1, 32, 1, 2, 0, 1, 2, 1, 64, 1, 64, 256, 64, 1, 1 << 20, None) == 3
    # null pointers
    assert L.hs_int4_gemm(None, 256, None, 32, None, 2, 0, None, 2, None, 64, 1, 64, 256, 128, None, 0, None) == 1
    # stride too small
    assert L.hs_fp8_gemm(1, 10, 1, 256, 1, 2, 0, 1, 64, 1, 64, 256, 1, 1 << 20, None) == 1
    # bad scale dtype code
    assert L.hs_fp8_gemm(1, 256, 1, 256, 1, 2, 7, 1, 64, 1, 64, 256, 1, 1 << 20, None) == 1
    # missing workspace is reported before any launch
    assert L.hs_fp8_gemm(16, 256, 16, 256, 16, 2, 0, 16, 64, 1, 64, 256, None, 0, None) == 2
    # empty problems are no-ops
    assert L.hs_int4_gemm(None, 0, None, 0, None, 0, 0, None, 0, None, 0, 0, 64, 256, 128, None, 0, None) == 0


def test_operands_of_2gib_or_more_are_refused_not_truncated():
    """Buffer resources address 32-bit byte ranges; the C ABI refuses larger
    operands (HS_EUNSUPPORTED) before touching the device."""
    L = _native.lib()
    big_ld = 1 << 30  # X row stride in elements: the second row starts at 2 GiB
    ws = 1 << 30
    # X spans 2^31 bytes
    assert L.hs_int4_gemm(16, big_ld, 16, 32, 16, 2, 0, 16, 2, 16, 64, 2, 64, 256, 128, 16, ws, None) == 3
    assert L.hs_int4_gemm_silu_mul(16, big_ld, 16, 32, 16, 2, 0, 16, 2, 16, 64, 2, 64, 256, 128, 16, ws, None) == 3
    assert L.hs_fp8_gemm(16, big_ld, 16, 256, 16, 2, 0, 16, 64, 2, 64, 256, 16, ws, None) == 3
    # FP8 weight of 2^20 x 4096 bytes = 4 GiB
    n, k = 1 << 20, 4096
    assert L.hs_fp8_gemm(16, k, 16, k, 16, 32, 2, 16, n, 1, n, k, 16, ws, None) == 3
    # INT4 packed rows with a 2^29-word stride
    assert L.hs_int4_gemm(16, 256, 16, 1 << 29, 16, 2, 0, 16, 2, 16, 64, 1, 64, 256, 128, 16, ws, None) == 3
    # output stride
    assert L.hs_int4_gemm(16, 256, 16, 32, 16, 2, 0, 16, 2, 16, big_ld, 2, 64, 256, 128, 16, ws, None) == 3
    # just under the limit is accepted by the check (missing workspace is reported instead)
    assert L.hs_fp8_gemm(16, 256, 16, 256, 16, 2, 0, 16, 64, 1, 64, 256, None, 0, None) == 2


def test_workspace_size_is_deterministic_and_covers_counters():
    L = _native.lib()
    a = L.hs_gemm_workspace_bytes(0, 1, 34816, 5120)
    assert a == L.hs_gemm_workspace_bytes(0, 1, 34816, 5120) and a > 0
    assert L.hs_gemm_workspace_bytes(0, 0, 64, 64) == 0
    assert L.hs_gemm_workspace_bytes(9, 1, 64, 64) == 0


def _int4_weight(n=64, k=256, group=128):
    g = (k + group - 1) // group
    return PackedInt4Weight(
        torch.zeros(n, k // 8, dtype=torch.int32),
        torch.ones(n, g, dtype=torch.bfloat16),
        torch.zeros(n // 8, g, dtype=torch.int32),
        (n, k),
        group,
    )


def _fp8_weight(n=129, k=129):
    return BlockScaledFP8Weight(
        torch.zeros(n, k, dtype=torch.float8_e4m3fn),
        torch.ones((n + 127) // 128, (k + 127) // 128, dtype=torch.bfloat16),
        (n, k),
    )


def test_awq_validation_order_and_messages():
    w = _int4_weight()
    with pytest.raises(ValueError, match="activation width does not match packed INT4 weight"):
        hs.awq_linear(torch.zeros(2, 128, dtype=torch.bfloat16), w)
    w64 = _int4_weight(group=64)
    with pytest.raises(ValueError, match="requires group_size=128"):
        hs.awq_linear(torch.zeros(2, 256, dtype=torch.bfloat16), w64)


def test_awq_cpu_activation_is_an_error_not_a_fallback():
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        hs.awq_linear(torch.zeros(2, 256, dtype=torch.bfloat16), _int4_weight())


def test_fp8_validation_order_and_messages():
    w = _fp8_weight()
    with pytest.raises(ValueError, match="activation width does not match FP8 weight"):
        hs.fp8_linear(torch.zeros(1, 128), w)
    bad_block = BlockScaledFP8Weight(w.data, w.scale_inv, w.original_shape, (64, 64))
    with pytest.raises(ValueError, match="128x128 blocks"):
        hs.fp8_linear(torch.zeros(1, 129), bad_block)
    # the reference test tests/test_fp8_kernel.py:117-123
    invalid = BlockScaledFP8Weight(w.data, w.scale_inv[:1, :1], w.original_shape)
    with pytest.raises(ValueError, match="scale grid"):
        hs.fp8_linear(torch.randn(1, 129), invalid)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        hs.fp8_linear(torch.zeros(1, 129, dtype=torch.bfloat16), w)


def test_dequantize_validates_scale_grid_first():
    w = _fp8_weight()
    invalid = BlockScaledFP8Weight(w.data, w.scale_inv[:1, :1], w.original_shape)
    with pytest.raises(ValueError, match="scale grid"):
        hs.dequantize_fp8_weight(invalid)


def test_concat_split_round_trip_int4_and_fp8():
    # tests/test_runtime.py:394-431 in the reference: concat then split returns the parts.
    g = torch.Generator().manual_seed(0)
    parts = []
    for n in (16, 8, 24):
        parts.append(
            PackedInt4Weight(
                torch.randint(-(2**31), 2**31 - 1, (n, 32), generator=g, dtype=torch.int32),
                torch.rand(n, 2, generator=g).to(torch.bfloat16),
                torch.randint(-(2**31), 2**31 - 1, (n // 8, 2), generator=g, dtype=torch.int32),
                (n, 256),
            )
        )
    fused = hs.concatenate_linear_weights(parts)
    assert fused.original_shape == (48, 256)
    for a, b in zip(parts, hs.split_linear_weight(fused, (16, 8, 24))):
        assert b.original_shape == a.original_shape
        assert torch.equal(a.packed, b.packed) and torch.equal(a.scale, b.scale)
        assert torch.equal(a.zero_point, b.zero_point)
    # N % 8 != 0 cannot be fused (zero points pack 8 rows per word)
    odd = PackedInt4Weight(parts[0].packed[:12], parts[0].scale[:12], parts[0].zero_point[:2], (12, 256))
    assert hs.concatenate_linear_weights([odd, parts[1]]) is None

    f_parts = [
        BlockScaledFP8Weight(
            torch.randint(0, 120, (n, 200), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn),
            torch.rand(n // 128, 2, generator=g).to(torch.bfloat16),
            (n, 200),
        )
        for n in (128, 256)
    ]
    fused = hs.concatenate_linear_weights(f_parts)
    assert fused.original_shape == (384, 200) and fused.scale_inv.shape == (3, 2)
    for a, b in zip(f_parts, hs.split_linear_weight(fused, (128, 256))):
        assert torch.equal(a.data.view(torch.uint8), b.data.view(torch.uint8))
        assert torch.equal(a.scale_inv, b.scale_inv)
    bad = BlockScaledFP8Weight(f_parts[0].data[:100], f_parts[0].scale_inv, (100, 200))
    assert hs.concatenate_linear_weights([bad, f_parts[1]]) is None


def test_split_views_share_storage_and_reject_misaligned_rows():
    g = torch.Generator().manual_seed(1)
    n = 48
    w = PackedInt4Weight(
        torch.randint(-(2**31), 2**31 - 1, (n, 32), generator=g, dtype=torch.int32),
        torch.rand(n, 2, generator=g).to(torch.bfloat16),
        torch.randint(-(2**31), 2**31 - 1, (n // 8, 2), generator=g, dtype=torch.int32),
        (n, 256),
    )
    a, b = hs.split_linear_weight(w, (16, 32))
    assert a.packed.data_ptr() == w.packed.data_ptr()
    assert b.zero_point.data_ptr() == w.zero_point[2:].data_ptr() and b.zero_point.shape == (4, 2)
    with pytest.raises(ValueError, match="zero_point"):
        hs.split_linear_weight(w, (12, 36))
    # a ragged FP8 tail keeps its partial scale row (ceil(N/128) rows per part)
    f = BlockScaledFP8Weight(
        torch.zeros(300, 128, dtype=torch.float8_e4m3fn), torch.rand(3, 1).to(torch.bfloat16), (300, 128)
    )
    head, tail = hs.split_linear_weight(f, (256, 44))
    assert head.scale_inv.shape == (2, 1) and tail.scale_inv.shape == (1, 1)
    assert torch.equal(tail.scale_inv, f.scale_inv[2:])
    # mixed formats or dense + quantized do not fuse
    assert hs.concatenate_linear_weights([w, f]) is None
    assert hs.concatenate_linear_weights([torch.zeros(8, 256), w]) is None
    assert hs.concatenate_linear_weights([]) is None


def test_linear_dispatch_dense_branch():
    w = torch.randn(5, 7)
    x = torch.randn(3, 7)
    torch.testing.assert_close(hs.linear(x, w), x @ w.T)


def test_custom_ops_are_registered_with_fake_implementations():
    """torch.compile sees opaque ops (hydraserve_amd/ops.py); their fake
    implementations give the output shape and dtype without a device."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    for name in ("int4_gemm", "fp8_gemm", "int4_gate_up_silu_mul"):
        assert hasattr(torch.ops.hydraserve_amd, name)
    with FakeTensorMode():
        x = torch.empty(3, 256, dtype=torch.bfloat16)
        packed = torch.empty(64, 32, dtype=torch.int32)
        scale = torch.empty(64, 2, dtype=torch.bfloat16)
        zero = torch.empty(8, 2, dtype=torch.int32)
        y = torch.ops.hydraserve_amd.int4_gemm(x, packed, scale, zero, 64, 256, 128)
        assert y.shape == (3, 64) and y.dtype == torch.bfloat16
        y = torch.ops.hydraserve_amd.int4_gate_up_silu_mul(x, packed, scale, zero, 64, 256, 128)
        assert y.shape == (3, 32)
        data = torch.empty(64, 256, dtype=torch.uint8)
        y = torch.ops.hydraserve_amd.fp8_gemm(x, data, torch.empty(1, 2), 64, 256)
        assert y.shape == (3, 64) and y.dtype == torch.bfloat16


def test_noalloc_entry_point_validates_before_touching_the_device():
    L = _native.lib()
    # group != 128, null pointers, short strides, bad dtype: rejected on the host
    assert L.hs_int4_gemm_noalloc(16, 256, 16, 32, 16, 2, 0, 16, 2, 16, 64, 1, 64, 256, 64, None) == 3
    assert L.hs_int4_gemm_noalloc(None, 256, None, 32, None, 2, 0, None, 2, None, 64, 1, 64, 256, 128, None) == 1
    assert L.hs_int4_gemm_noalloc(16, 100, 16, 32, 16, 2, 0, 16, 2, 16, 64, 1, 64, 256, 128, None) == 1
    assert L.hs_int4_gemm_noalloc(16, 256, 16, 32, 16, 2, 9, 16, 2, 16, 64, 1, 64, 256, 128, None) == 1
    assert L.hs_int4_gemm_noalloc(None, 0, None, 0, None, 0, 0, None, 0, None, 0, 0, 64, 256, 128, None) == 0
    assert b"scratch" in L.hs_error_string(4)


def test_tiled_copies_round_trip_and_are_dropped_by_fuse_split():
    from hydraserve_amd.kernels.tiles import TiledInt4Weight, tile_fp8_weight, tile_int4_weight, untile_int4

    g = torch.Generator().manual_seed(3)
    n, k = 48, 384
    w = PackedInt4Weight(
        torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int32),
        torch.rand(n, 3, generator=g).to(torch.bfloat16),
        torch.randint(-(2**31), 2**31 - 1, (n // 8, 3), generator=g, dtype=torch.int32),
        (n, k),
    )
    t = tile_int4_weight(w)
    assert isinstance(t, TiledInt4Weight) and isinstance(t, PackedInt4Weight)
    assert t.tiles.shape == (3, 3, 16, 16)
    assert torch.equal(untile_int4(t.tiles, n, k), w.packed)
    # tiles are chunk-major: tiles[c, t] = rows 16t..16t+15 of chunk c.
    # Tile (t=1, c=2) = rows 16..31, words 32..47, nibbles paired: K offset i
    # of a word sits at nibble i/2 (even i) or 4 + i/2 (odd i)
    src = w.packed[16:32, 32:48].to(torch.int64) & 0xFFFFFFFF
    dst = t.tiles[2, 1].to(torch.int64) & 0xFFFFFFFF
    for i in range(8):
        pos = i // 2 if i % 2 == 0 else 4 + i // 2
        assert torch.equal((src >> (4 * i)) & 15, (dst >> (4 * pos)) & 15)
    f = BlockScaledFP8Weight(
        torch.randint(0, 120, (32, 256), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn),
        torch.ones(1, 2), (32, 256),
    )
    tf = tile_fp8_weight(f)
    # FP8 tile (t=1, c=1): rows 16..31, K 128..255; byte j of row r at K
    # 64h + 16p + j sits at tiles[c, t, h, p, r, j]
    src8 = f.data.view(torch.uint8)[16:32, 128:256].reshape(16, 2, 4, 16)
    assert torch.equal(tf.tiles[1, 1], src8.permute(1, 2, 0, 3))
    src8 = f.data.view(torch.uint8)[16:32, 0:128].reshape(16, 2, 4, 16)
    assert torch.equal(tf.tiles[0, 1], src8.permute(1, 2, 0, 3))
    parts = hs.split_linear_weight(t, (16, 32))
    assert all(type(p) is PackedInt4Weight for p in parts)
    fused = hs.concatenate_linear_weights([t, t])
    assert type(fused) is PackedInt4Weight and fused.original_shape == (96, k)
    with pytest.raises(ValueError, match="N % 16"):
        tile_int4_weight(PackedInt4Weight(w.packed[:8], w.scale[:8], w.zero_point[:1], (8, k)))
