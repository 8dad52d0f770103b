"""Child process of tests/test_tiles_gpu.py: parity of the tiled decode
kernel (csrc/qgemm_tiled.hip) on small shapes.

By default the plan sends small weights (N*K below 32M) to the row-major
kernels; this child runs with HS_TM_MIN_M=1 (read once per
process), so every case below goes through the tiled kernel: every row-block
count (1..64 rows, partial blocks; 129..192 rows split into 128 row-major
rows and a tiled rest), waves holding 0..2 tiles (N = 64: four
tiles), K ranges split across workgroups, all scale dtypes.  The checks are
those of tests/test_gemm_gpu.py, plus a bit-identical second call.  The
"silu" cases run the fused gate_up SiLU-and-mul store of the tiled kernel
(awq_gate_up_silu_mul on the tiled copy of an interleaved weight) against
silu(bf16(gate)) * bf16(up) from the oracle GEMM, as tests/test_mlp.py does.
"""

from __future__ import annotations

import numpy as np
import torch

from tests import test_gemm_gpu as tg

import hydraserve_amd as hs
from hydraserve_amd.kernels import awq_gate_up_silu_mul, interleave_gate_up, tile_fp8_weight, tile_int4_weight
from oracle import quant_oracle as qo

# (kind, M, N, K, scale dtype)
CASES = (
    [("int4", m, n, k, torch.bfloat16) for m in (1, 2, 4, 5, 8, 16, 17, 33, 37, 64)
     for n, k in ((4096, 1024), (2064, 2048), (64, 384))]
    + [("int4", m, 2048, 2048, sdt) for m in (8, 64) for sdt in (torch.float16, torch.float32)]
    + [("fp8", m, 4096, 2048, sdt) for m in (1, 16, 33, 64) for sdt in (torch.float32, torch.bfloat16)]
    + [("fp8", m, 272, 1024, torch.float16) for m in (3, 40)]
    # 10 K chunks, 65 tiles: K ranges that end inside a ring round and an
    # 8-chunk scale round, a ragged last tile group
    + [("int4", m, 1040, 1280, torch.bfloat16) for m in (1, 16, 40)]
    + [("fp8", m, 1040, 1280, torch.bfloat16) for m in (1, 40)]
    # 129..192 rows: 128 rows row-major, the rest through the tiled kernel
    + [("int4", 160, 4096, 1024, torch.bfloat16), ("fp8", 192, 4096, 2048, torch.float32),
       ("int4", 190, 1024, 4096, torch.float16)]
    # fused SiLU store: 1..64 rows (each row-block count, the K-half pairing
    # at 33..64), 68 tiles of 10 chunks (an odd tile count per wave set, a
    # ragged last group), 4 tiles; fp16 / fp32 scales
    + [("silu", m, n, k, torch.bfloat16) for m in (1, 5, 16, 17, 33, 64)
       for n, k in ((2048, 1024), (1088, 1280), (64, 384))]
    + [("silu", m, 2048, 2048, sdt) for m in (8, 64) for sdt in (torch.float16, torch.float32)]
)


def _silu_ref(y, n):
    """silu(bf16(gate)) * bf16(up) in float64 from a GEMM result (and its
    exact-weight variant) on the original, non-interleaved weight."""

    def act(yy):
        gu = qo.bf16_bits_to_f32(qo.f32_to_bf16_bits(np.asarray(yy, dtype=np.float32))).astype(np.float64)
        g, u = gu[:, : n // 2], gu[:, n // 2 :]
        return g / (1.0 + np.exp(-g)) * u

    ref = act(y).view(tg.RefArray)
    ref.exact = act(y.exact)
    return ref


def main() -> int:
    dev = torch.device("cuda", 0)
    for i, (kind, m, n, k, sdt) in enumerate(CASES):
        rng = np.random.default_rng(31 * m + n + i)
        what = f"tiled {kind} M={m} N={n} K={k} {sdt}"
        print(what, flush=True)
        if kind == "silu":
            w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, sdt)
            wt = tile_int4_weight(interleave_gate_up(w))
            y = awq_gate_up_silu_mul(x, wt)
            y2 = awq_gate_up_silu_mul(x, wt)
            ref = _silu_ref(tg.int4_ref(xb, packed, scale, zero, n, k), n)
        elif kind == "int4":
            w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, sdt)
            wt = tile_int4_weight(w)
            y = hs.awq_linear(x, wt)
            y2 = hs.awq_linear(x, wt)
            ref = tg.int4_ref(xb, packed, scale, zero, n, k)
        else:
            w, x, xb, data, scale = tg.fp8_case(rng, m, n, k, dev, sdt)
            wt = tile_fp8_weight(w)
            y = hs.fp8_linear(x, wt)
            y2 = hs.fp8_linear(x, wt)
            ref = tg.fp8_ref(xb, data, scale, n, k)
        torch.cuda.synchronize()
        tg.assert_gemm_close(y, ref, what=what)
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), what
    print("ok", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
