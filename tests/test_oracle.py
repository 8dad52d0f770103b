"""Pins the CPU oracle (oracle/quant_oracle.py) to independent results.

Each check is chosen so that a plausible mistake in the oracle (wrong nibble
order, wrong zero-point transpose, truncation instead of round-to-nearest-even,
wrong E4M3 bias or subnormal handling, transposed GEMM) fails it.
"""

import numpy as np
import pytest

from oracle import quant_oracle as qo


def test_bf16_rounding_matches_torch(golden_dir):
    d = np.load(golden_dir / "bf16_round.npz")
    got = qo.f32_to_bf16_bits(d["f32"])
    np.testing.assert_array_equal(got, d["bf16"])
    np.testing.assert_array_equal(qo.bf16_bits_to_f32(got).view(np.uint32) & 0xFFFF, 0)


def test_bf16_nan_stays_nan():
    assert np.isnan(qo.bf16_bits_to_f32(qo.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


def test_unpack_brute_force_every_value_every_position():
    # Word with value v in nibble position p and 0 elsewhere -> k = 8j + p holds v.
    rows = []
    for v in range(16):
        for p in range(8):
            rows.append(np.uint32(v) << np.uint32(4 * p))
    words = np.array(rows, dtype=np.uint32).reshape(-1, 1).view(np.int32)
    q = qo.unpack_int4_rows(words, 8)
    for r, (v, p) in enumerate((v, p) for v in range(16) for p in range(8)):
        expect = np.zeros(8, np.uint8)
        expect[p] = v
        np.testing.assert_array_equal(q[r], expect)


def test_zero_point_unpack_transposes_rows():
    # zero word [r, g] nibble j belongs to output row 8r + j, group g.
    z = np.zeros((2, 3), dtype=np.uint32)
    z[1, 2] = np.uint32(0xA) << np.uint32(4 * 5)  # row 13, group 2
    out = qo.unpack_zero_points(z.view(np.int32), 16)
    expect = np.zeros((16, 3), np.uint8)
    expect[13, 2] = 0xA
    np.testing.assert_array_equal(out, expect)


def test_pack_unpack_round_trip_and_truncation():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, (24, 40), dtype=np.uint8)
    np.testing.assert_array_equal(qo.unpack_int4_rows(qo.pack_int4_rows(q), 40), q)
    np.testing.assert_array_equal(qo.unpack_int4_rows(qo.pack_int4_rows(q), 37), q[:, :37])
    z = rng.integers(0, 16, (24, 5), dtype=np.uint8)
    np.testing.assert_array_equal(qo.unpack_zero_points(qo.pack_zero_points(z), 24), z)
    np.testing.assert_array_equal(qo.unpack_zero_points(qo.pack_zero_points(z), 21), z[:21])


def test_int4_dequant_matches_reference_test_expression(golden_dir):
    d = np.load(golden_dir / "int4_case_s41.npz")
    # packers agree with the reference test's packers
    np.testing.assert_array_equal(qo.pack_int4_rows(d["q"]), d["packed"])
    np.testing.assert_array_equal(qo.pack_zero_points(d["z"]), d["zero_point"])
    w = qo.dequant_int4_bf16(d["packed"], d["scale"], d["zero_point"], (64, 256), 128)
    np.testing.assert_array_equal(w, d["w_bf16"])  # bit-exact, like awq test atol=0


def test_int4_dequant_group_boundary_and_sign():
    # q=0, z=15 -> -15*s ; q=15, z=0 -> 15*s ; group switch at k=128.
    n, k = 8, 256
    q = np.zeros((n, k), np.uint8)
    q[:, 128:] = 15
    z = np.zeros((n, 2), np.uint8)
    z[:, 0] = 15
    s = qo.f32_to_bf16_bits(np.full((n, 2), 0.5, np.float32))
    w = qo.bf16_bits_to_f32(qo.dequant_int4_bf16(qo.pack_int4_rows(q), s, qo.pack_zero_points(z), (n, k)))
    assert np.all(w[:, :128] == -7.5) and np.all(w[:, 128:] == 7.5)


def test_e4m3fn_decode_matches_torch_for_all_codes(golden_dir):
    d = np.load(golden_dir / "e4m3fn_codes.npz")
    got = qo.decode_e4m3fn(d["codes"])
    nan = np.isnan(d["values"])
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], d["values"][~nan])
    assert nan.sum() == 2  # 0x7F and 0xFF


def test_e4m3fn_known_values():
    v = qo.decode_e4m3fn(np.array([0x01, 0x07, 0x08, 0x38, 0x7E, 0xFE, 0x80], np.uint8))
    np.testing.assert_array_equal(v, np.array([2.0**-9, 7 * 2.0**-9, 2.0**-6, 1.0, 448.0, -448.0, -0.0], np.float32))


def test_fp8_dequant_matches_torch(golden_dir):
    d = np.load(golden_dir / "fp8_case_143x259.npz")
    w32 = qo.dequant_fp8(d["data"], d["scale"], (143, 259), out="f32")
    np.testing.assert_array_equal(w32, d["w_f32"])
    # the Triton semantics: bf16 of the fp32 product
    wb = qo.dequant_fp8(d["data"], d["scale"], (143, 259), out="bf16")
    np.testing.assert_array_equal(wb, qo.f32_to_bf16_bits(d["w_f32"]))


def test_fp8_scale_grid_validation():
    with pytest.raises(ValueError, match="scale grid"):
        qo.dequant_fp8(np.zeros((129, 129), np.uint8), np.ones((1, 2), np.float32), (129, 129))


def test_fp8_quantizer_mean_error_bound():
    # tests/test_fp8_kernel.py:48-52: quantize->dequantize mean abs error < 0.02
    rng = np.random.default_rng(41)
    dense = rng.standard_normal((143, 259)).astype(np.float32)
    codes, scales = qo.quantize_fp8_blocks(dense)
    restored = qo.dequant_fp8(codes, scales, dense.shape)
    assert np.abs(restored - dense).mean() < 0.02
    # exact grid points survive the round trip
    assert np.all(np.abs(restored) <= np.abs(dense).max() * 1.0001)


def test_gemm_f64_brute_force():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 7)).astype(np.float32)
    w = rng.standard_normal((4, 7)).astype(np.float32)
    y = qo.gemm_f64(x, w)
    for m in range(3):
        for n in range(4):
            assert abs(y[m, n] - sum(float(x[m, k]) * float(w[n, k]) for k in range(7))) < 1e-12


def test_int4_linear_ref_matches_golden(golden_dir):
    d = np.load(golden_dir / "int4_case_s41.npz")
    y = qo.int4_linear_ref(d["x"], d["packed"], d["scale"], d["zero_point"], (64, 256))
    np.testing.assert_allclose(y, d["y"], rtol=0, atol=1e-12)


def test_fp8_linear_ref_matches_golden(golden_dir):
    d = np.load(golden_dir / "fp8_case_143x259.npz")
    y = qo.fp8_linear_ref(d["x"], d["data"], d["scale"], (143, 259))
    np.testing.assert_allclose(y, d["y"], rtol=0, atol=1e-9)


def test_weight_byte_formulas():
    assert qo.int4_weight_bytes(34816, 5120) == 92_610_560
    assert qo.int4_weight_bytes(5120, 17408) == 46_305_280
    assert qo.fp8_weight_bytes(34816, 5120) == 178_301_440
    assert qo.fp8_weight_bytes(5120, 17408) == 89_150_720
