"""Reading the quantized linear weights of a safetensors checkpoint.

The formats are the reference's (hydraserve/model/weights.py:41-108 reads the
shards, hydraserve/model/runtime.py:170-276 assembles the weights):

* compressed-tensors asymmetric INT4: ``<base>.weight_packed`` (int32 [N, K/8]),
  ``<base>.weight_scale`` ([N, K/128], cast to the runtime dtype),
  ``<base>.weight_zero_point`` (int32 [N/8, K/128]) and ``<base>.weight_shape``
  (the two ints N, K) -> PackedInt4Weight;
* block-scaled FP8: ``<base>.weight`` (float8_e4m3fn [N, K]) with
  ``<base>.weight_scale_inv`` ([N/128, K/128], cast to the runtime dtype)
  -> BlockScaledFP8Weight;
* anything else (embeddings, norms, lm_head) -> a dense tensor in the runtime
  dtype.

A checkpoint is either one ``model.safetensors`` or shards listed in
``model.safetensors.index.json``.  Tensors are read on demand with
safetensors' own reader (nothing from the file is executed), one short-lived
handle per read.

``load_linear_weights`` is the load-time hook of this path: besides reading,
it can keep chosen FP8 projections in page-locked host memory (the offload
case, fp8_linear then streams them, kernels/fp8_stream.py), and it fuses an
MLP's gate and up projections along N (concatenate_linear_weights, as the
reference fuses at load, runtime.py:1404-1469) and re-lays the fused INT4
gate_up out once into the gate/up-interleaved order the fused SiLU-and-mul
kernel reads (kernels/mlp.py: interleave_gate_up, lossless).
"""

from __future__ import annotations

import json
import threading
from pathlib import Path
from typing import Any, Iterable

from .weights import BlockScaledFP8Weight, PackedInt4Weight

INT4_PARTS = (".weight_packed", ".weight_scale", ".weight_zero_point", ".weight_shape")


class CheckpointReader:
    """Tensor names -> shard files of a safetensors checkpoint directory."""

    def __init__(self, model_dir: str | Path) -> None:
        self.model_dir = Path(model_dir)
        if not self.model_dir.is_dir():
            raise NotADirectoryError(self.model_dir)
        index = self.model_dir / "model.safetensors.index.json"
        single = self.model_dir / "model.safetensors"
        if index.is_file():
            with index.open("r", encoding="utf-8") as f:
                self.shard_of = dict(json.load(f)["weight_map"])
        elif single.is_file():
            from safetensors import safe_open

            with safe_open(single, framework="np") as h:
                self.shard_of = {name: single.name for name in h.keys()}
        else:
            raise FileNotFoundError(f"no safetensors checkpoint found in {self.model_dir}")
        self._lock = threading.Lock()

    def __contains__(self, name: str) -> bool:
        return name in self.shard_of

    def names(self, prefix: str = "") -> tuple[str, ...]:
        return tuple(sorted(n for n in self.shard_of if n.startswith(prefix)))

    def _shard(self, name: str) -> Path:
        try:
            return self.model_dir / self.shard_of[name]
        except KeyError as exc:
            raise KeyError(f"checkpoint does not contain {name!r}") from exc

    def tensor(self, name: str, *, device: Any = "cpu", dtype: Any = None):
        from safetensors import safe_open

        with self._lock, safe_open(self._shard(name), framework="pt", device="cpu") as h:
            t = h.get_tensor(name)
        if dtype is not None:
            t = t.to(dtype=dtype)
        if str(device) != "cpu":
            t = t.to(device=device, non_blocking=True)
        return t

    def shape(self, name: str) -> tuple[int, ...]:
        from safetensors import safe_open

        with self._lock, safe_open(self._shard(name), framework="np") as h:
            return tuple(h.get_slice(name).get_shape())


def linear_bases(reader: CheckpointReader, prefix: str = "") -> dict[str, str]:
    """Base names (``<base>.weight``) of the linear weights under ``prefix`` ->
    their format: "int4", "fp8" or "dense"."""
    names = reader.names(prefix)
    out: dict[str, str] = {}
    for n in names:
        if n.endswith(".weight_packed"):
            out[n.removesuffix("_packed")] = "int4"
    for n in names:
        if n.endswith(".weight") and n not in out:
            out[n] = "fp8" if f"{n}_scale_inv" in reader else "dense"
    return out


def read_linear(reader: CheckpointReader, base: str, *, device: Any = "cuda:0", dtype: Any = None, host: bool = False):
    """One linear weight by its base name ``<prefix>.weight``.  ``host``: keep
    an FP8 weight in page-locked host memory instead of on ``device``."""
    import torch

    dtype = dtype or torch.bfloat16
    if f"{base}_packed" in reader:
        n, k = (int(v) for v in reader.tensor(f"{base}_shape").tolist())
        return PackedInt4Weight(
            packed=reader.tensor(f"{base}_packed", device=device).contiguous(),
            scale=reader.tensor(f"{base}_scale", device=device, dtype=dtype).contiguous(),
            zero_point=reader.tensor(f"{base}_zero_point", device=device).contiguous(),
            original_shape=(n, k),
        )
    if f"{base}_scale_inv" in reader:
        place = "cpu" if host else device
        w = BlockScaledFP8Weight(
            data=reader.tensor(base, device=place).contiguous(),
            scale_inv=reader.tensor(f"{base}_scale_inv", device=place, dtype=dtype).contiguous(),
            original_shape=reader.shape(base),
        )
        if host:
            from ..kernels.fp8_stream import pin_fp8_weight

            w = pin_fp8_weight(w)
        return w
    return reader.tensor(base, device=device, dtype=dtype)


def load_linear_weights(
    model_dir: str | Path,
    *,
    prefix: str = "",
    device: Any = "cuda:0",
    dtype: Any = None,
    host_fp8: Iterable[str] = (),
    fuse_gate_up: bool = False,
    tile: bool = False,
) -> dict[str, Any]:
    """Every linear weight under ``prefix`` by base name.

    ``host_fp8``: FP8 base names kept in page-locked host memory.
    ``fuse_gate_up``: for each ``<p>.gate_proj.weight`` / ``<p>.up_proj.weight``
    pair, also ``<p>.gate_up_proj.weight`` (fused along N) and, for INT4,
    ``<p>.gate_up_proj.weight.interleaved`` (the fused SiLU kernel's layout).
    ``tile``: device-resident INT4/FP8 weights (N % 16 == 0, K % 128 == 0),
    the interleaved gate_up included, come with the load-time tiled copy the
    tiled decode and 256x256 prefill kernels read (kernels/tiles.py).
    """
    from ..kernels.mlp import interleave_gate_up
    from ..kernels.tiles import tile_fp8_weight, tile_int4_weight
    from .linear import concatenate_linear_weights

    reader = CheckpointReader(model_dir)
    host = set(host_fp8)
    out = {base: read_linear(reader, base, device=device, dtype=dtype, host=base in host)
           for base in linear_bases(reader, prefix)}
    if fuse_gate_up:
        for base in [b for b in out if b.endswith(".gate_proj.weight")]:
            stem = base.removesuffix(".gate_proj.weight")
            up = out.get(f"{stem}.up_proj.weight")
            if up is None:
                continue
            fused = concatenate_linear_weights([out[base], up])
            if fused is None:
                continue
            out[f"{stem}.gate_up_proj.weight"] = fused
            if isinstance(fused, PackedInt4Weight) and fused.original_shape[0] % 32 == 0:
                out[f"{stem}.gate_up_proj.weight.interleaved"] = interleave_gate_up(fused)
    if tile:
        for name, w in list(out.items()):
            n_k = getattr(w, "original_shape", None)
            if n_k is None or n_k[0] % 16 or n_k[1] % 128:
                continue
            if isinstance(w, PackedInt4Weight) and w.group_size == 128:
                out[name] = tile_int4_weight(w)
            elif isinstance(w, BlockScaledFP8Weight) and name not in host:  # streamed weights stay row-major
                out[name] = tile_fp8_weight(w)
    return out
