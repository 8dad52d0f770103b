"""Seeded synthetic quantized weights and activations (numpy, host side).

Draws follow the measurement spec: X ~ N(0,1) in bf16; INT4 q and zero points
uniform in 0..15, packed in the compressed-tensors layout; bf16 scales uniform
in [1e-3, 1e-2]; FP8 codes uniform over the 254 finite E4M3FN codes; fp32
block scales uniform in [1e-3, 1e-1].
"""

from __future__ import annotations

import numpy as np

from oracle import quant_oracle as qo


def x_bf16(rng, m, k):
    return qo.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))


def int4_weight(rng, n, k, group=128):
    g = (k + group - 1) // group
    q = rng.integers(0, 16, (n, k), dtype=np.uint8)
    z = rng.integers(0, 16, (n, g), dtype=np.uint8)
    kp = ((k + 7) // 8) * 8
    qp = np.zeros((n, kp), dtype=np.uint8)
    qp[:, :k] = q
    npad = ((n + 7) // 8) * 8
    zp = np.zeros((npad, g), dtype=np.uint8)
    zp[:n] = z
    scale = qo.f32_to_bf16_bits(rng.uniform(1e-3, 1e-2, (n, g)).astype(np.float32))
    return qo.pack_int4_rows(qp), scale, qo.pack_zero_points(zp), q, z


def fp8_codes(rng, shape):
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    return finite[rng.integers(0, len(finite), shape)]


def fp8_weight(rng, n, k, scale_dtype="f32"):
    data = fp8_codes(rng, (n, k))
    s = rng.uniform(1e-3, 1e-1, ((n + 127) // 128, (k + 127) // 128)).astype(np.float32)
    if scale_dtype == "bf16":
        s = qo.f32_to_bf16_bits(s)
    return data, s
