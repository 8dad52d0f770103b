"""The drop-in in the reference runtime's call contexts (GPU).

QwenTextRuntime._linear (hydraserve/model/runtime.py:1263-1270) is the only
caller; it runs eagerly, inside CUDA-graph capture of the decode step
(runtime.py:788-803) and inside torch.compile (runtime.py:577, 592-596).
Fused projections are split into narrow() views (runtime.py:1477-1506).
Everything here calls the product path; bars as in tests/test_gemm_gpu.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hydraserve_amd as hs
from hydraserve_amd.kernels import awq_gate_up_silu_mul, interleave_gate_up
from hydraserve_amd.model.weights import BlockScaledFP8Weight

from . import test_gemm_gpu as tg

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16)


def test_linear_dispatches_both_weight_types_and_dense():
    dev = tg._cuda()
    rng = np.random.default_rng(11)
    m, n, k = 5, 384, 1024
    w4, x, xb, packed, scale, zero, _ = tg.int4_case(rng, m, n, k, dev)
    tg.assert_gemm_close(hs.linear(x, w4), tg.int4_ref(xb, packed, scale, zero, n, k), what="linear int4")
    w8, x8, xb8, data, s8 = tg.fp8_case(rng, m, n, k, dev)
    tg.assert_gemm_close(hs.linear(x8, w8), tg.fp8_ref(xb8, data, s8, n, k), what="linear fp8")
    assert torch.equal(_bits(hs.linear(x, w4)), _bits(hs.awq_linear(x, w4)))
    assert torch.equal(_bits(hs.linear(x8, w8)), _bits(hs.fp8_linear(x8, w8)))
    # batched leading dims keep their shape through the dispatch
    y3 = hs.linear(x8.view(1, m, k), w8)
    assert y3.shape == (1, m, n)
    dense = torch.randn(n, k, device=dev, dtype=torch.bfloat16)
    torch.testing.assert_close(hs.linear(x, dense), x @ dense.T)


@pytest.mark.parametrize("m", [1, 16, 64, 300])
def test_fp8_split_views_match_separate_weights(m):
    """Fuse three FP8 projections, split them back into views (scale rows are
    narrowed by 128-row block), run each view: equal to the separate weight."""
    dev = tg._cuda()
    rng = np.random.default_rng(77 + m)
    k = 1024
    parts, xs = [], None
    for n in (256, 128, 384):
        w, x, xb, data, s = tg.fp8_case(rng, m, n, k, dev)
        parts.append((w, data, s))
        xs = (x, xb) if xs is None else xs
    x, xb = xs
    fused = hs.concatenate_linear_weights([p[0] for p in parts])
    assert fused is not None and fused.original_shape == (768, k)
    views = hs.split_linear_weight(fused, (256, 128, 384))
    start = 0
    for (w, data, s), v in zip(parts, views):
        n = w.original_shape[0]
        assert v.data.data_ptr() == fused.data.data_ptr() + start * k
        y = hs.fp8_linear(x, v)
        assert torch.equal(_bits(y), _bits(hs.fp8_linear(x, w)))
        tg.assert_gemm_close(y, tg.fp8_ref(xb, data, s, n, k), what=f"fp8 view rows {start}..{start + n}")
        start += n


def test_torch_compile_fullgraph_two_linears():
    """runtime.py:577 (fullgraph) / 592-596: the ops are opaque custom ops
    with fake implementations, so Dynamo traces through without a break."""
    dev = tg._cuda()
    rng = np.random.default_rng(19)
    m, n, k = 16, 512, 1024
    w4, x, *_ = tg.int4_case(rng, m, n, k, dev)
    w8, *_ = tg.fp8_case(rng, m, k, n, dev)
    wi = interleave_gate_up(tg.int4_case(rng, m, 2 * k, k, dev)[0])

    def two_linears(h):
        a = hs.linear(h, w4)  # [m, n]
        b = hs.fp8_linear(a, w8)  # [m, k]
        return awq_gate_up_silu_mul(b, wi)  # [m, k]

    torch._dynamo.reset()
    compiled = torch.compile(two_linears, fullgraph=True)
    got = compiled(x)
    want = two_linears(x)
    assert got.shape == want.shape == (m, k)
    assert torch.equal(_bits(got), _bits(want))
    # a second shape recompiles (dynamic M) and still matches
    x2 = x[:3].contiguous()
    assert torch.equal(_bits(compiled(x2)), _bits(two_linears(x2)))


@pytest.mark.parametrize("m", [1, 16, 64, 300])
def test_hip_graph_replay_matches_eager(m):
    """runtime.py:788-803: the decode step is captured once and replayed.
    Warm up eagerly (workspace growth allocates), capture INT4 + FP8 + fused
    calls, replay several times with eager work in between, and compare every
    replay bit for bit with the eager result."""
    dev = tg._cuda()
    rng = np.random.default_rng(500 + m)
    n, k = 2048, 1024
    w4, x, *_ = tg.int4_case(rng, m, n, k, dev)
    w8, *_ = tg.fp8_case(rng, m, n, k, dev)
    wi = interleave_gate_up(w4)
    x_static = x.clone()

    def step():
        return hs.awq_linear(x_static, w4), hs.fp8_linear(x_static, w8), awq_gate_up_silu_mul(x_static, wi)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = [t.clone() for t in step()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    for i in range(4):
        # unrelated eager work between replays
        hs.awq_linear(torch.randn(7, k, device=dev, dtype=torch.bfloat16), w4)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(_bits(e), _bits(o)), f"replay {i}"
    # new input values flow through the captured graph
    x_static.copy_(torch.randn_like(x_static))
    g.replay()
    torch.cuda.synchronize()
    fresh = step()
    for e, o in zip(fresh, outs):
        assert torch.equal(_bits(e), _bits(o))
