"""GPU parity of the register-streamed decode kernel under every layout.

The launch plan picks this kernel only for some shapes (narrow outputs,
5..64 rows); here each layout (16-row blocks per wave x block groups x K
phases) and the per-wave X mode are forced in turn, in a child process
(tests/_skinny_check.py) since the plan reads HS_SKINNY* once per process.
Bars: those of tests/test_gemm_gpu.py, plus a bit-identical second call.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize(
    "layout,xd", [(0, 0), (1, 0), (2, 0), (3, 0), (4, 0), (5, 0), (0, 16), (2, 16)]
)
def test_skinny_layout(layout, xd):
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    env = dict(os.environ, HS_SKINNY="1", HS_SKINNY_LAYOUT=str(layout), HS_SKINNY_XD=str(xd))
    res = subprocess.run(
        [sys.executable, "-u", "-m", "tests._skinny_check"],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=110,
    )
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert res.stdout.strip().endswith("ok"), res.stdout[-2000:]
