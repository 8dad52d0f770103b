"""CPU oracle for HydraServe's quantized linear-layer path (numpy only).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
use it, and only as the checker.  It restates, in numpy, the arithmetic of the
reference's grouped asymmetric INT4 GEMM and 128x128 block-scaled E4M3FN GEMM:

* ``unpack_int4_rows``      -> hydraserve/kernels/awq.py:11-14
* ``unpack_zero_points``    -> hydraserve/kernels/awq.py:15-17
* ``dequant_int4_bf16``     -> hydraserve/kernels/awq.py:18-22 (and the in-kernel
                               dequant at awq.py:136-137, which is bit-identical)
* ``decode_e4m3fn``         -> hydraserve/kernels/fp8.py:144-152
* ``dequant_fp8``           -> hydraserve/kernels/fp8.py:6-21 (``dtype=None`` ->
                               fp32) and fp8.py:160-161 (Triton: fp32 product
                               rounded to bf16)
* ``pack_int4_rows`` / ``pack_zero_points`` -> tests/test_awq_kernel.py:11-24
* ``quantize_fp8_blocks``   -> tests/test_fp8_kernel.py:13-45 and
                               scripts/quantize_fp8.py:64-81 (amax/448 per block)
* ``gemm_f64``              -> the fp32-accumulate GEMM ``X @ W^T`` every kernel
                               computes (awq.py:36-38, fp8.py:51-53), evaluated in
                               float64 so it serves as the tolerance reference.

How each function is pinned (tests/test_oracle.py):
* nibble unpack / packers: brute force over every value 0..15 at every nibble
  position, plus round trip with the reference test's packers;
* bf16 rounding: against PyTorch's own float32 -> bfloat16 conversion on
  random and special values (ties, subnormals, inf, nan);
* INT4 dequant: against the reference test's own expected-weight expression
  evaluated by PyTorch (tests/test_awq_kernel.py:57-63, asserted atol=0);
* E4M3FN decode: all 256 codes against PyTorch's float8_e4m3fn conversion
  (tests/golden/e4m3fn_codes.npz, written by tests/golden/make_golden.py);
* FP8 dequant: closed form on identity scales and powers of two, plus the
  reference test's quantize->dequantize mean-error bound (< 0.02);
* GEMM: brute-force triple loop on tiny shapes and numpy's float64 matmul.

bf16 values are carried as ``uint16`` bit patterns throughout.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "unpack_int4_rows",
    "unpack_zero_points",
    "pack_int4_rows",
    "pack_zero_points",
    "dequant_int4_bf16",
    "decode_e4m3fn",
    "dequant_fp8",
    "quantize_fp8_blocks",
    "gemm_f64",
    "int4_linear_ref",
    "fp8_linear_ref",
    "int4_weight_bytes",
    "fp8_weight_bytes",
]


# --------------------------------------------------------------------------
# bf16 <-> f32 (round to nearest even, NaN kept quiet)
# --------------------------------------------------------------------------
def f32_to_bf16_bits(values) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even (IEEE)."""
    x = np.ascontiguousarray(values, dtype=np.float32)
    bits = x.view(np.uint32)
    nan = np.isnan(x)
    lsb = (bits >> np.uint32(16)) & np.uint32(1)
    rounded = (bits + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    out = rounded.astype(np.uint16)
    out[nan] = ((bits[nan] >> np.uint32(16)) | np.uint32(0x0040)).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


# --------------------------------------------------------------------------
# compressed-tensors INT4 layout
# --------------------------------------------------------------------------
def unpack_int4_rows(packed: np.ndarray, input_features: int) -> np.ndarray:
    """packed int32 [N, ceil(K/8)] -> q uint8 [N, K]; nibble i of word j is k=8j+i.

    Follows hydraserve/kernels/awq.py:11-14 (shift by 4*i, mask 0xF, reshape,
    truncate to ``input_features``).
    """
    words = np.ascontiguousarray(packed).view(np.uint32)
    rows = words.shape[0]
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    nib = (words[:, :, None] >> shifts) & np.uint32(0xF)
    return nib.reshape(rows, -1)[:, :input_features].astype(np.uint8)


def unpack_zero_points(zero_point: np.ndarray, output_features: int) -> np.ndarray:
    """zero int32 [ceil(N/8), G] -> z uint8 [N, G]; nibble j of word [r, g] is row 8r+j.

    Follows hydraserve/kernels/awq.py:15-17 (unpack, permute(0,2,1), reshape,
    truncate to ``output_features``).
    """
    words = np.ascontiguousarray(zero_point).view(np.uint32)
    groups = words.shape[1]
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    nib = (words[:, :, None] >> shifts) & np.uint32(0xF)  # [R, G, 8]
    return nib.transpose(0, 2, 1).reshape(-1, groups)[:output_features].astype(np.uint8)


def pack_int4_rows(q: np.ndarray) -> np.ndarray:
    """q [N, K] (K % 8 == 0, values 0..15) -> int32 [N, K/8] (tests/test_awq_kernel.py:11-16)."""
    q = np.asarray(q, dtype=np.uint32)
    rows, cols = q.shape
    out = np.zeros((rows, cols // 8), dtype=np.uint32)
    for nibble in range(8):
        out |= (q[:, nibble::8] & np.uint32(0xF)) << np.uint32(4 * nibble)
    return out.view(np.int32)


def pack_zero_points(z: np.ndarray) -> np.ndarray:
    """z [N, G] (N % 8 == 0) -> int32 [N/8, G] (tests/test_awq_kernel.py:19-24)."""
    z = np.asarray(z, dtype=np.uint32)
    rows, groups = z.shape
    out = np.zeros((rows // 8, groups), dtype=np.uint32)
    for nibble in range(8):
        out |= (z[nibble::8] & np.uint32(0xF)) << np.uint32(4 * nibble)
    return out.view(np.int32)


def dequant_int4_bf16(packed, scale_bits, zero_point, original_shape, group_size=128):
    """Dequantized weight as bf16 bits [N, K]: bf16_rne((q - z) * s).

    (q - z) in [-15, 15] is exact in bf16 and the product of a 4-bit integer and
    an 8-bit-mantissa scale is exact in float32, so a single RNE to bf16 gives
    the bits the reference produces (awq.py:18-22 on CPU, awq.py:136-137 in
    Triton).
    """
    n, k = original_shape
    q = unpack_int4_rows(packed, k).astype(np.int32)
    z = unpack_zero_points(zero_point, n).astype(np.int32)
    s = bf16_bits_to_f32(scale_bits)
    groups = np.arange(k) // group_size
    prod = (q - z[:, groups]).astype(np.float32) * s[:, groups]
    return f32_to_bf16_bits(prod)


# --------------------------------------------------------------------------
# E4M3FN
# --------------------------------------------------------------------------
def decode_e4m3fn(codes) -> np.ndarray:
    """uint8 E4M3FN codes -> float32, closed form of hydraserve/kernels/fp8.py:144-152.

    exponent field e = (b >> 3) & 0xF, mantissa m = b & 7;
    e == 0: m * 2^-9 (subnormal); else (1 + m/8) * 2^(e-7); sign bit 0x80.
    Codes 0x7F / 0xFF are NaN in E4M3FN (the Triton decode does not special-case
    them; PyTorch and the hardware return NaN).
    """
    b = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    e = (b >> 3) & 0xF
    m = (b & 7).astype(np.float64)
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((b & 0x80) != 0, -mag, mag)
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return val.astype(np.float32)


def _scale_grid_f32(scale_inv, scale_is_bf16: bool) -> np.ndarray:
    if scale_is_bf16:
        return bf16_bits_to_f32(scale_inv)
    return np.asarray(scale_inv, dtype=np.float32)


def dequant_fp8(data, scale_inv, original_shape, *, scale_is_bf16=False, out="f32"):
    """Block-scaled dequant.

    out="f32":  decode(b) * s in float32 (fp8.py:6-21 with dtype=None).
    out="bf16": bf16_rne(float32(decode(b) * s)) as bits, the Triton kernel's
                weight (fp8.py:153-161).
    """
    n, k = original_shape
    s = _scale_grid_f32(scale_inv, scale_is_bf16)
    exp_shape = ((n + 127) // 128, (k + 127) // 128)
    if s.shape != exp_shape:
        raise ValueError("FP8 inverse-scale grid does not match weight shape")
    w = decode_e4m3fn(np.asarray(data, dtype=np.uint8).reshape(n, k))
    grid = s[(np.arange(n) // 128)[:, None], (np.arange(k) // 128)[None, :]]
    prod = (w * grid).astype(np.float32)
    if out == "f32":
        return prod
    if out == "bf16":
        return f32_to_bf16_bits(prod)
    raise ValueError(out)


def quantize_fp8_blocks(dense: np.ndarray):
    """Reference test quantizer: per 128x128 block scale = max|block| / 448.

    Returns (codes uint8 [N, K], scale float32 grid).  Encoding to E4M3FN uses
    round-to-nearest-even on the finite grid (saturation cannot trigger because
    |block / scale| <= 448).  Mirrors tests/test_fp8_kernel.py:13-45.
    """
    dense = np.asarray(dense, dtype=np.float32)
    n, k = dense.shape
    gn, gk = (n + 127) // 128, (k + 127) // 128
    scales = np.empty((gn, gk), dtype=np.float32)
    codes = np.empty((n, k), dtype=np.uint8)
    table = decode_e4m3fn(np.arange(256, dtype=np.uint8))
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F and c != 0x80])
    order = np.argsort(table[finite], kind="stable")
    sorted_codes = finite[order]
    sorted_vals = table[sorted_codes].astype(np.float64)
    for bi in range(gn):
        for bj in range(gk):
            blk = dense[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            sc = np.float32(max(float(np.abs(blk).max()), 1e-6) / 448.0)
            scales[bi, bj] = sc
            v = (blk / sc).astype(np.float32).astype(np.float64)
            idx = np.clip(np.searchsorted(sorted_vals, v), 1, len(sorted_vals) - 1)
            lo, hi = sorted_vals[idx - 1], sorted_vals[idx]
            pick_hi = (hi - v) < (v - lo)
            tie = (hi - v) == (v - lo)
            # ties to even mantissa (code LSB 0)
            hi_even = (sorted_codes[idx] & 1) == 0
            pick_hi = pick_hi | (tie & hi_even)
            chosen = np.where(pick_hi, sorted_codes[idx], sorted_codes[idx - 1])
            chosen = np.where(v == 0.0, 0, chosen)
            codes[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128] = chosen
    return codes, scales


# --------------------------------------------------------------------------
# GEMM references
# --------------------------------------------------------------------------
def gemm_f64(x_f32: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    """Y = X @ W^T accumulated in float64 (the tolerance reference)."""
    return np.asarray(x_f32, np.float64) @ np.asarray(w_f32, np.float64).T


def int4_linear_ref(x_bf16_bits, packed, scale_bits, zero_point, original_shape, group_size=128):
    """Reference output (float64) of awq_linear on identical inputs."""
    w = bf16_bits_to_f32(dequant_int4_bf16(packed, scale_bits, zero_point, original_shape, group_size))
    return gemm_f64(bf16_bits_to_f32(x_bf16_bits), w)


def fp8_linear_ref(x_bf16_bits, data, scale_inv, original_shape, *, scale_is_bf16=False):
    """Reference output (float64) of fp8_linear with the fp32 dequantized weight."""
    w = dequant_fp8(data, scale_inv, original_shape, scale_is_bf16=scale_is_bf16, out="f32")
    return gemm_f64(bf16_bits_to_f32(x_bf16_bits), w)


def int4_weight_bytes(n: int, k: int, group: int = 128) -> int:
    """Packed + bf16 scale + packed zero bytes of one INT4 weight."""
    g = (k + group - 1) // group
    return n * ((k + 7) // 8) * 4 + n * g * 2 + ((n + 7) // 8) * g * 4


def fp8_weight_bytes(n: int, k: int, scale_bytes: int = 4) -> int:
    return n * k + ((n + 127) // 128) * ((k + 127) // 128) * scale_bytes
