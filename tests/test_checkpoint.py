"""The safetensors reader (hydraserve_amd/model/checkpoint.py) on synthetic
checkpoints in the reference's formats (hydraserve/model/weights.py:41-108,
hydraserve/model/runtime.py:170-276): compressed-tensors INT4 parts, FP8 +
scale_inv, dense tensors; sharded (index json) and single-file layouts.

CPU: every field read back bit-exact, formats recognised, gate/up fusion and
the interleaved layout lossless.  GPU: the loaded weights through linear()
against the oracle, an FP8 projection kept in page-locked host memory.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from hydraserve_amd.kernels.mlp import deinterleave_gate_up
from hydraserve_amd.model.checkpoint import CheckpointReader, linear_bases, load_linear_weights
from hydraserve_amd.model.weights import BlockScaledFP8Weight, PackedInt4Weight
from oracle import quant_oracle as qo

from . import _synth

P = "model.language_model.layers.0"


def _int4_parts(rng, base, n, k):
    packed, scale_bits, zero, _, _ = _synth.int4_weight(rng, n, k)
    return {
        f"{base}_packed": torch.from_numpy(packed.view(np.int32).copy()),
        f"{base}_scale": torch.from_numpy(scale_bits.view(np.int16).copy()).view(torch.bfloat16),
        f"{base}_zero_point": torch.from_numpy(zero.view(np.int32).copy()),
        f"{base}_shape": torch.tensor([n, k], dtype=torch.int64),
    }


def _write(tmp_path, sharded, seed=0):
    rng = np.random.default_rng(seed)
    t = {}
    t.update(_int4_parts(rng, f"{P}.mlp.gate_proj.weight", 64, 256))
    t.update(_int4_parts(rng, f"{P}.mlp.up_proj.weight", 64, 256))
    t.update(_int4_parts(rng, f"{P}.mlp.down_proj.weight", 256, 128))
    data, s = _synth.fp8_weight(rng, 256, 384)
    t[f"{P}.self_attn.o_proj.weight"] = torch.from_numpy(data).view(torch.float8_e4m3fn)
    t[f"{P}.self_attn.o_proj.weight_scale_inv"] = torch.from_numpy(s)
    t["lm_head.weight"] = torch.randn(96, 256).to(torch.bfloat16)
    t[f"{P}.input_layernorm.weight"] = torch.ones(256, dtype=torch.bfloat16)
    if sharded:
        names = sorted(t)
        half = len(names) // 2
        shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
        weight_map = {}
        for fname, ns in shards.items():
            save_file({n: t[n].contiguous() for n in ns}, str(tmp_path / fname))
            weight_map.update({n: fname for n in ns})
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    else:
        save_file({n: v.contiguous() for n, v in t.items()}, str(tmp_path / "model.safetensors"))
    return t


@pytest.mark.parametrize("sharded", [False, True])
def test_reader_recognises_formats_and_reads_bit_exact(tmp_path, sharded):
    t = _write(tmp_path, sharded)
    reader = CheckpointReader(tmp_path)
    kinds = linear_bases(reader)
    assert kinds[f"{P}.mlp.gate_proj.weight"] == "int4"
    assert kinds[f"{P}.self_attn.o_proj.weight"] == "fp8"
    assert kinds["lm_head.weight"] == "dense"
    w = load_linear_weights(tmp_path, device="cpu")
    g = w[f"{P}.mlp.gate_proj.weight"]
    assert isinstance(g, PackedInt4Weight) and g.original_shape == (64, 256) and g.group_size == 128
    assert torch.equal(g.packed, t[f"{P}.mlp.gate_proj.weight_packed"])
    assert torch.equal(g.scale.view(torch.int16), t[f"{P}.mlp.gate_proj.weight_scale"].view(torch.int16))
    assert torch.equal(g.zero_point, t[f"{P}.mlp.gate_proj.weight_zero_point"])
    o = w[f"{P}.self_attn.o_proj.weight"]
    assert isinstance(o, BlockScaledFP8Weight) and o.original_shape == (256, 384)
    assert torch.equal(o.data.view(torch.uint8), t[f"{P}.self_attn.o_proj.weight"].view(torch.uint8))
    # scale_inv is cast to the runtime dtype, as the reference loader does (runtime.py:240-243)
    assert o.scale_inv.dtype == torch.bfloat16
    assert torch.equal(o.scale_inv, t[f"{P}.self_attn.o_proj.weight_scale_inv"].to(torch.bfloat16))
    assert torch.equal(w["lm_head.weight"], t["lm_head.weight"])
    with pytest.raises(KeyError, match="does not contain"):
        reader.tensor("nope")


def test_load_with_tiles(tmp_path):
    from hydraserve_amd.kernels.tiles import TiledFP8Weight, TiledInt4Weight, untile_int4

    _write(tmp_path, sharded=False)
    w = load_linear_weights(tmp_path, device="cpu", tile=True)
    g = w[f"{P}.mlp.gate_proj.weight"]
    assert isinstance(g, TiledInt4Weight)
    assert torch.equal(untile_int4(g.tiles, 64, 256), g.packed)
    assert isinstance(w[f"{P}.self_attn.o_proj.weight"], TiledFP8Weight)
    assert not hasattr(w["lm_head.weight"], "tiles")


def test_missing_checkpoint_is_an_error(tmp_path):
    with pytest.raises(FileNotFoundError):
        CheckpointReader(tmp_path)


def test_gate_up_fusion_and_interleave_at_load(tmp_path):
    _write(tmp_path, sharded=True)
    w = load_linear_weights(tmp_path, device="cpu", fuse_gate_up=True)
    fused = w[f"{P}.mlp.gate_up_proj.weight"]
    gate, up = w[f"{P}.mlp.gate_proj.weight"], w[f"{P}.mlp.up_proj.weight"]
    assert fused.original_shape == (128, 256)
    assert torch.equal(fused.packed, torch.cat([gate.packed, up.packed]))
    inter = w[f"{P}.mlp.gate_up_proj.weight.interleaved"]
    back = deinterleave_gate_up(inter)
    for a, b in ((fused.packed, back.packed), (fused.scale, back.scale), (fused.zero_point, back.zero_point)):
        assert torch.equal(a, b)
    # dequantized rows: interleaved block j = gate rows 16j.., then up rows 16j..
    qi = qo.unpack_int4_rows(inter.packed.numpy().view(np.uint32), 256)
    qf = qo.unpack_int4_rows(fused.packed.numpy().view(np.uint32), 256)
    np.testing.assert_array_equal(qi[16:32], qf[64:80])


@pytest.mark.gpu
def test_loaded_weights_run_through_linear(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    import hydraserve_amd as hs

    from . import test_gemm_gpu as tg

    t = _write(tmp_path, sharded=True, seed=3)
    dev = torch.device("cuda", 0)
    w = load_linear_weights(tmp_path, device=dev, host_fp8=[f"{P}.self_attn.o_proj.weight"], fuse_gate_up=True)
    o = w[f"{P}.self_attn.o_proj.weight"]
    assert o.data.device.type == "cpu" and o.data.is_pinned()
    rng = np.random.default_rng(9)
    for m in (4, 200):
        xb = _synth.x_bf16(rng, m, 384)
        y = hs.linear(tg.t_bf16(xb, dev), o)
        ref = tg.fp8_ref(xb, t[f"{P}.self_attn.o_proj.weight"].view(torch.uint8).numpy(), o.scale_inv, 256, 384)
        tg.assert_gemm_close(y, ref, what=f"host fp8 M={m}")
        base = f"{P}.mlp.down_proj.weight"
        xb = _synth.x_bf16(rng, m, 128)
        y = hs.linear(tg.t_bf16(xb, dev), w[base])
        ref = tg.int4_ref(xb, t[f"{base}_packed"].numpy(), t[f"{base}_scale"], t[f"{base}_zero_point"].numpy(), 256, 128)
        tg.assert_gemm_close(y, ref, what=f"int4 M={m}")
    x = torch.randn(8, 256, device=dev, dtype=torch.bfloat16)
    lm = w["lm_head.weight"]
    torch.testing.assert_close(hs.linear(x, lm).float(), x.float() @ lm.float().T, atol=5e-2, rtol=2e-2)
