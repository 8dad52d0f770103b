"""Write the committed fixtures under tests/golden/.

    python tests/golden/make_golden.py

* e4m3fn_codes.npz   -- all 256 E4M3FN codes decoded by PyTorch's own
                        float8_e4m3fn -> float32 conversion (an independent
                        implementation: it pins oracle.decode_e4m3fn and the
                        GPU decode).
* bf16_round.npz     -- float32 inputs (random, ties, subnormals, specials) and
                        PyTorch's float32 -> bfloat16 conversion of them
                        (pins oracle.f32_to_bf16_bits).
* int4_case_s41.npz  -- the reference test's INT4 case (seed-41 shapes of
                        tests/test_awq_kernel.py:29-69: N=64, K=256, M=3) with
                        the dequantized bf16 weight computed by PyTorch using the
                        reference test's own expression ((q - z).to(bf16) * s),
                        plus the float64 output of X @ W^T.
* fp8_case_143x259.npz -- a partial-block FP8 case (N=143, K=259, M=5;
                        tests/test_fp8_kernel.py:48-56 shape) with fp32 and bf16
                        dequantized weights computed by PyTorch
                        (data.to(dtype) * scale.to(dtype)) and the float64 output.

PyTorch supplies the expected values; the oracle module is not used here.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    np.savez(HERE / "e4m3fn_codes.npz", codes=codes.numpy(), values=vals)

    g = np.random.default_rng(7)
    rnd = g.standard_normal(4096).astype(np.float32) * np.float32(10.0) ** g.integers(-40, 38, 4096).astype(np.float32)
    base = g.integers(0, 1 << 16, 512, dtype=np.uint32) << np.uint32(16)
    ties = (base | np.uint32(0x8000)).view(np.float32)  # exactly half an ulp
    near = (base | np.uint32(0x7FFF)).view(np.float32)
    sub = (g.integers(1, 1 << 23, 256, dtype=np.uint32)).view(np.float32)  # subnormals
    special = np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1.0, -1.0], dtype=np.float32)
    f = np.concatenate([rnd, ties, near, sub, special]).astype(np.float32)
    f = f[np.isfinite(f) | np.isinf(f)]
    np.savez(HERE / "bf16_round.npz", f32=f, bf16=bf16_bits(torch.from_numpy(f).to(torch.bfloat16)))

    # INT4 case: the reference test's recipe (seeded torch generator on CPU).
    gen = torch.Generator().manual_seed(41)
    n, k, group = 64, 256, 128
    q = torch.randint(0, 16, (n, k), generator=gen)
    z = torch.randint(0, 16, (n, k // group), generator=gen)
    s = torch.rand(n, k // group, generator=gen, dtype=torch.float32).to(torch.bfloat16) * 0.2
    hidden = torch.randn(3, k, generator=gen, dtype=torch.bfloat16)
    packed = torch.zeros(n, k // 8, dtype=torch.int64)
    for nib in range(8):
        packed |= q[:, nib::8].to(torch.int64) << (nib * 4)
    zp = torch.zeros(n // 8, k // group, dtype=torch.int64)
    for nib in range(8):
        zp |= z[nib::8].to(torch.int64) << (nib * 4)
    groups = torch.arange(k) // group
    w = (q - z[:, groups]).to(torch.bfloat16) * s[:, groups]
    y = hidden.double() @ w.double().T
    np.savez(
        HERE / "int4_case_s41.npz",
        q=q.numpy().astype(np.uint8), z=z.numpy().astype(np.uint8),
        packed=packed.to(torch.int32).numpy(), zero_point=zp.to(torch.int32).numpy(),
        scale=bf16_bits(s), x=bf16_bits(hidden), w_bf16=bf16_bits(w), y=y.numpy(),
    )

    # FP8 partial-block case.
    gen = torch.Generator().manual_seed(43)
    n, k = 143, 259
    data = torch.randint(0, 256, (n, k), generator=gen, dtype=torch.int32).to(torch.uint8)
    data[(data & 0x7F) == 0x7F] = 0  # no NaN codes
    sc = (torch.rand((n + 127) // 128, (k + 127) // 128, generator=gen) * 0.099 + 0.001).to(torch.float32)
    hidden = torch.randn(5, k, generator=gen, dtype=torch.bfloat16)
    fp8 = data.view(torch.float8_e4m3fn)
    ob, ib = torch.arange(n) // 128, torch.arange(k) // 128
    grid = sc[ob[:, None], ib[None, :]]
    w32 = fp8.to(torch.float32) * grid
    wb = fp8.to(torch.bfloat16) * grid.to(torch.bfloat16)
    y = hidden.double() @ w32.double().T
    np.savez(
        HERE / "fp8_case_143x259.npz",
        data=data.numpy(), scale=sc.numpy(), x=bf16_bits(hidden),
        w_f32=w32.numpy(), w_bf16=bf16_bits(wb), y=y.numpy(),
    )
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
