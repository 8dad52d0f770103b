"""Build libhydraserve_amd.so in-tree with hipcc for gfx950.

    python -m hydraserve_amd.build        # or: from hydraserve_amd.build import build; build()

Every source is compiled on every call (no staleness heuristics), in parallel,
then linked into ``hydraserve_amd/libhydraserve_amd.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libhydraserve_amd.so"
BUILD_DIR = PKG / "_build"
SOURCES = ["qgemm_tiled.hip", "qgemm_skinny.hip", "qgemm_decode.hip", "qgemm_stream.hip", "qgemm_rows.hip", "qgemm_gemv.hip", "qgemm_prefill.hip", "qgemm_wide.hip", "qgemm_mid.hip", "qgemm_dequant.hip", "hbm_probe.hip", "qgemm_capi.hip"]
ARCH = os.environ.get("HS_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build hydraserve_amd)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Never emit packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result",
        f"-I{PKG.parent / 'include'}",
    ]


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)

    # HS_BUILD_INCREMENTAL=1 (development only): skip sources whose object is
    # newer than the source and every header; build() itself always compiles all.
    incremental = os.environ.get("HS_BUILD_INCREMENTAL") == "1"
    headers = [*CSRC.glob("*.h"), PKG.parent / "include" / "hydraserve_amd.h"]
    newest_header = max(h.stat().st_mtime for h in headers)

    def compile_one(src: str) -> Path:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        if incremental and obj.exists():
            t = obj.stat().st_mtime
            if t > (CSRC / src).stat().st_mtime and t > newest_header:
                return obj
        cmd = [hipcc, *_flags(), "-c", str(CSRC / src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
        if verbose:
            noise = "is not a recognized feature for this target"
            for line in (res.stdout + res.stderr).splitlines():
                if noise not in line:
                    print(line, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
