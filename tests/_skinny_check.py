"""Child process of tests/test_skinny_gpu.py: parity of the register-streamed
decode kernel (csrc/qgemm_skinny.hip) under one forced layout.

The launch plan reads its tuning environment once per process, so each
forced layout runs in a child with HS_SKINNY=1 and HS_SKINNY_LAYOUT /
HS_SKINNY_XD set; the checks are those of tests/test_gemm_gpu.py.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

from tests import test_gemm_gpu as tg

import hydraserve_amd as hs

# (kind, M, N, K, scale dtype): ragged N, K that does or does not divide into
# the layout's K phases (the plan then falls back), multi-tile stream-K
# ranges, and the 64-row limit.
CASES = [
    ("int4", 1, 200, 1024, torch.bfloat16),
    ("int4", 5, 1000, 4096, torch.bfloat16),
    ("int4", 16, 5120, 2048, torch.bfloat16),
    ("int4", 16, 264, 640, torch.float16),
    ("int4", 12, 520, 1152, torch.float32),
    ("int4", 17, 2056, 3072, torch.bfloat16),
    ("int4", 33, 384, 2048, torch.bfloat16),
    ("int4", 64, 4096, 8192, torch.bfloat16),
    ("fp8", 1, 272, 1024, torch.float32),
    ("fp8", 9, 2048, 4096, torch.bfloat16),
    ("fp8", 16, 5120, 2048, torch.float32),
    ("fp8", 40, 1000, 3072, torch.float32),
    ("fp8", 64, 512, 1536, torch.float16),
]


def main() -> int:
    dev = torch.device("cuda", 0)
    layout = os.environ.get("HS_SKINNY_LAYOUT", "?")
    xd = int(os.environ.get("HS_SKINNY_XD", "0"))
    for i, (kind, m, n, k, sdt) in enumerate(CASES):
        if xd and m > xd:
            continue
        rng = np.random.default_rng(1000 + i)
        what = f"skinny layout={layout} xd={xd} {kind} M={m} N={n} K={k} {sdt}"
        print(what, flush=True)
        if kind == "int4":
            w, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev, sdt)
            y = hs.awq_linear(x, w)
            ref = tg.int4_ref(xb, packed, scale, zero, n, k)
        else:
            w, x, xb, data, scale = tg.fp8_case(rng, m, n, k, dev, sdt)
            y = hs.fp8_linear(x, w)
            ref = tg.fp8_ref(xb, data, scale, n, k)
        torch.cuda.synchronize()
        tg.assert_gemm_close(y, ref, what=what)
        # a second call reuses the workspace (arrival counters back at zero)
        y2 = hs.awq_linear(x, w) if kind == "int4" else hs.fp8_linear(x, w)
        torch.cuda.synchronize()
        assert torch.equal(y, y2), what + ": second call differs"
    print("ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
