"""Benchmark of the quantized linear-layer hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--sweep] [--no-cpu]

Headline workload: INT4 group-128 asymmetric decode GEMMs,
M in {1, 4, 16, 64} x {gate_up 5120->34816, down 17408->5120}.  One "step" is
one pass over those 8 GEMMs through the product entry point
(hydraserve_amd.awq_linear -> C ABI -> HIP).  Inputs are synthetic and
resident in HBM before timing; weights rotate over several independent copies
(> 256 MB MALL) so every GEMM streams its weights from HBM.  Steps are
captured in a HIP graph (as the reference's decode loop does,
hydraserve/model/runtime.py:788-803) and timed with events around graph
replays, bracketed by synchronizations.

`value` = weight bytes (packed + scale + zero) of all GEMMs / step time, GB/s.
`roofline` = the dominant kernel's algorithmic weight bytes / its mean launch
duration (events around graph replays of back-to-back launches of that GEMM).
`cpu_baseline` = the reference's CPU torch path (dequant + bf16 matmul,
oracle/torch_cpu_path.py) timed on a bounded sample on the host cores.

--sweep additionally measures every BASELINE config (INT4/FP8, decode and
prefill, the config-4 layer) and prints one JSON object per shape to stderr;
--sweep-json PATH also writes the whole result there.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

GATE_UP = (34816, 5120)  # (N, K)
DOWN = (5120, 17408)
C0 = (4096, 4096)
QKV = (10240, 5120)
O_PROJ = (5120, 8192)
GDN_IN = (12288, 5120)


def int4_bytes(n, k):
    g = (k + 127) // 128
    return n * k // 2 + n * g * 2 + ((n + 7) // 8) * g * 4


def fp8_bytes(n, k, scale_bytes=4):
    return n * k + ((n + 127) // 128) * ((k + 127) // 128) * scale_bytes


def copies_for(bytes_per_copy, floor_bytes=900 << 20, max_copies=8):
    """Enough independent weight copies that a reused copy has left the 256 MB MALL."""
    return int(max(2, min(max_copies, -(-floor_bytes // max(bytes_per_copy, 1)))))


def make_int4(torch, n, k, copies, gen, dev):
    from hydraserve_amd import PackedInt4Weight

    g = (k + 127) // 128
    out = []
    for _ in range(copies):
        packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=gen, dtype=torch.int32, device=dev)
        zero = torch.randint(-(2**31), 2**31 - 1, ((n + 7) // 8, g), generator=gen, dtype=torch.int32, device=dev)
        scale = (torch.rand(n, g, generator=gen, device=dev) * 9e-3 + 1e-3).to(torch.bfloat16)
        out.append(PackedInt4Weight(packed, scale, zero, (n, k)))
    return out


def make_fp8(torch, n, k, copies, gen, dev):
    from hydraserve_amd import BlockScaledFP8Weight

    out = []
    for _ in range(copies):
        data = torch.randint(0, 254, (n, k), generator=gen, dtype=torch.int32, device=dev)
        data = torch.where(data >= 0x7F, data + 1, data).to(torch.uint8)  # skip 0x7F; 0xFF never drawn
        scale = torch.rand((n + 127) // 128, (k + 127) // 128, generator=gen, device=dev) * 0.099 + 0.001
        out.append(BlockScaledFP8Weight(data.view(torch.float8_e4m3fn), scale, (n, k)))
    return out


# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of
# `bench.py --profile KIND:SHAPE:M` (KiB per dispatch), scaled by what the same
# counters read for a 512 MiB copy: FETCH x2.0, WRITE x1.0.  Kept beside the
# summaries under profiles/; shapes not listed report null.
PMC_TRAFFIC_KIB = {("int4", "gate_up", 64): (69799.2, 28954.0)}
FETCH_CAL, WRITE_CAL = 2.0, 1.0


def pmc_traffic(kind, name, m):
    kib = PMC_TRAFFIC_KIB.get((kind, name, m))
    if kib is None:
        return None
    return int((kib[0] * FETCH_CAL + kib[1] * WRITE_CAL) * 1024)


def graph_time_ms(torch, fn, reps, inner):
    """Capture `inner` calls of fn(i) in one graph, replay `reps` times; ms per call."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(inner):  # warm: allocations, workspaces
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(inner):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * inner), g


class Case:
    def __init__(self, kind, name, n, k, m, weights, x):
        self.kind, self.name, self.n, self.k, self.m = kind, name, n, k, m
        self.weights, self.x = weights, x

    @property
    def wbytes(self):
        return int4_bytes(self.n, self.k) if self.kind == "int4" else fp8_bytes(self.n, self.k)

    @property
    def flops(self):
        return 2.0 * self.m * self.n * self.k

    def call(self, i):
        import hydraserve_amd as hs

        w = self.weights[i % len(self.weights)]
        return hs.awq_linear(self.x, w) if self.kind == "int4" else hs.fp8_linear(self.x, w)

    def regime(self):
        return "decode" if self.m <= 64 else "prefill"

    def report(self, ms):
        gbs = self.wbytes / (ms * 1e-3) / 1e9
        tfl = self.flops / (ms * 1e-3) / 1e12
        bound = "hbm" if self.regime() == "decode" else "mfma"
        frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tfl / BF16_PEAK_TFLOPS
        return {
            "kind": self.kind, "shape": self.name, "M": self.m, "N": self.n, "K": self.k,
            "us": round(ms * 1e3, 2), "weight_GBps": round(gbs, 1), "TFLOPs": round(tfl, 2),
            "bound": bound, "roofline_frac": round(frac, 4),
        }


def cpu_baseline(sample_shapes, m):
    """Reference CPU path on the host: dequant + bf16 matmul per call (kind 'port')."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.torch_cpu_path import int4_cpu_linear

    cores = os.cpu_count() or 1
    cores = min(cores, int(os.environ.get("HS_CPU_THREADS", cores)))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    total_bytes, total_s = 0, 0.0
    for (n, k) in sample_shapes:
        gg = (k + 127) // 128
        packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), generator=g, dtype=torch.int32)
        zero = torch.randint(-(2**31), 2**31 - 1, ((n + 7) // 8, gg), generator=g, dtype=torch.int32)
        scale = (torch.rand(n, gg, generator=g) * 9e-3 + 1e-3).to(torch.bfloat16)
        x = torch.randn(m, k, generator=g).to(torch.bfloat16)
        int4_cpu_linear(x, packed, scale, zero, (n, k))  # warmup
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            int4_cpu_linear(x, packed, scale, zero, (n, k))
            times.append(time.perf_counter() - t0)
        total_s += min(times)
        total_bytes += int4_bytes(n, k)
        del packed, zero, scale
    return {
        "value": round(total_bytes / total_s / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"INT4 dequant+bf16 matmul (reference CPU branch) at M={m} on "
        + ", ".join(f"{n}x{k}" for n, k in sample_shapes)
        + f"; best of 2 after 1 warmup; {total_s * 1e3:.0f} ms per pass",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=6)
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep-json", metavar="PATH", help="with --sweep: also write the result to PATH")
    ap.add_argument("--profile", metavar="KIND:SHAPE:M",
                    help="eager launches of one GEMM (e.g. int4:gate_up:64; int4silu:gate_up:M for the fused "
                    "SiLU-and-mul store) plus a plain copy kernel of "
                    "known size, for rocprofv3 counter passes; prints one JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized GEMM path has no multi-GPU mode in this build "
              "(column-parallel along N needs no communication, row-parallel along K one all-reduce of Y); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    import hydraserve_amd  # noqa: F401  (fails loudly if the library is missing)
    from hydraserve_amd import _native

    _native.lib()
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(0)

    if args.profile:
        profile(torch, gen, dev, args.profile, max(args.steps, 1))
        return

    # ---- headline: config 1 ------------------------------------------------
    ms_list = [1, 4, 16, 64]
    shapes = {"gate_up": GATE_UP, "down": DOWN}
    per_copy = sum(int4_bytes(n, k) for n, k in shapes.values())
    copies = copies_for(per_copy)
    weights = {name: make_int4(torch, n, k, copies, gen, dev) for name, (n, k) in shapes.items()}
    xs = {(name, m): torch.randn(m, shapes[name][1], generator=gen, device=dev).to(torch.bfloat16)
          for name in shapes for m in ms_list}
    cases = [Case("int4", name, *shapes[name], m, weights[name], xs[(name, m)]) for m in ms_list for name in shapes]

    def step(i):
        for c in cases:
            c.call(i)

    # warmup (eager) then one graph holding `copies` steps (each on another copy)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    reps = max(1, -(-args.steps // copies))
    steps = reps * copies
    t_ms, _ = graph_time_ms(torch, step, reps, copies)
    step_bytes = sum(c.wbytes for c in cases)
    step_flops = sum(c.flops for c in cases)
    value = step_bytes / (t_ms * 1e-3) / 1e9

    # per-kernel times: graphs of back-to-back launches of one GEMM
    per = []
    for c in cases:
        ms, _ = graph_time_ms(torch, c.call, 10, 2 * copies)
        per.append((c, ms, c.report(ms)))
    dom_c, dom_ms, dom_r = max(per, key=lambda t: t[1])
    roofline = {
        "bound": "hbm",
        "achieved": dom_r["weight_GBps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(dom_r["weight_GBps"] / HBM_PEAK_GBS, 4),
        "traffic": pmc_traffic("int4", dom_c.name, dom_c.m),
        "kernel": f"INT4 decode {dom_c.name} M={dom_c.m} ({dom_c.n}x{dom_c.k})",
        "bytes_per_launch": dom_c.wbytes,
        "us_per_launch": dom_r["us"],
    }

    result = {
        "metric": "INT4/FP8 GEMM TFLOP/s + weight HBM GB/s (% roofline), M=1..2048, 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform int4 nibbles/zero points, bf16 scales U[1e-3,1e-2], X~N(0,1)); "
        f"weights rotated over {copies} copies",
        "config": {
            "workload": "config 1: INT4 g128 asymmetric decode GEMMs, M in {1,4,16,64} x "
            "{gate_up 5120->34816, down 17408->5120}, 8 GEMMs per step",
            "weight_bytes_per_step": step_bytes,
            "tflops": round(step_flops / (t_ms * 1e-3) / 1e12, 3),
            "weight_copies": copies,
            "launch": "HIP graph replay",
        },
        "roofline": roofline,
        "per_shape": [r for _, _, r in per],
    }

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline([GATE_UP, DOWN], 16)

    if args.sweep:
        result["sweep"] = sweep(torch, gen, dev)
    print(json.dumps(result), flush=True)
    if args.sweep and args.sweep_json:
        with open(args.sweep_json, "w") as f:
            json.dump(result, f, indent=1)


SHAPES = {"gate_up": GATE_UP, "down": DOWN, "c0": C0, "qkv": QKV, "o_proj": O_PROJ, "gdn_in": GDN_IN}
COPY_CAL_BYTES = 512 << 20


def profile(torch, gen, dev, spec, launches):
    """One GEMM launched eagerly `launches` times over rotated weight copies, then a
    512 MiB device-to-device copy launched 4 times.  Under rocprofv3 --pmc the copy's
    FETCH_SIZE / WRITE_SIZE per dispatch calibrate the counters against known bytes."""
    kind, name, m = spec.split(":")
    n, k = SHAPES[name]
    m = int(m)
    # kind "int4silu": gate_up with the fused SiLU-and-mul store, on weights
    # interleaved at load time (awq_gate_up_silu_mul)
    fused = kind == "int4silu"
    if fused:
        kind = "int4"
    make = make_int4 if kind == "int4" else make_fp8
    per_copy = int4_bytes(n, k) if kind == "int4" else fp8_bytes(n, k)
    ws = make(torch, n, k, copies_for(per_copy), gen, dev)
    x = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
    if fused:
        from hydraserve_amd.kernels import awq_gate_up_silu_mul, interleave_gate_up

        ws = [interleave_gate_up(w) for w in ws]
    c = Case(kind, name, n, k, m, ws, x)
    for i in range(launches):
        if fused:
            awq_gate_up_silu_mul(x, ws[i % len(ws)])
        else:
            c.call(i)
    src = torch.empty(COPY_CAL_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile": spec, "launches": launches, "weight_bytes_per_launch": c.wbytes,
                      "copy_bytes_per_launch": COPY_CAL_BYTES}), flush=True)


def sweep(torch, gen, dev):
    out = []

    def run(kind, name, n, k, m_list):
        make = make_int4 if kind == "int4" else make_fp8
        per_copy = int4_bytes(n, k) if kind == "int4" else fp8_bytes(n, k)
        copies = copies_for(per_copy)
        ws = make(torch, n, k, copies, gen, dev)
        for m in m_list:
            x = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
            c = Case(kind, name, n, k, m, ws, x)
            reps = 10 if m <= 64 else 4
            ms, _ = graph_time_ms(torch, c.call, reps, copies)
            r = c.report(ms)
            print(json.dumps(r), file=sys.stderr, flush=True)
            out.append(r)
        del ws
        torch.cuda.empty_cache()

    run("int4", "c0", *C0, [8])
    run("int4", "gate_up", *GATE_UP, [1, 4, 16, 64, 512, 1024, 2048])
    run("int4", "down", *DOWN, [1, 4, 16, 64, 512, 1024, 2048])
    run("fp8", "gate_up", *GATE_UP, [1, 16, 256, 2048])
    run("fp8", "down", *DOWN, [1, 16, 256, 2048])
    # gate_up followed by SiLU-and-mul: fused epilogue on the interleaved
    # weight vs the reference's sequence (GEMM, chunk, activation launch).
    from hydraserve_amd.kernels import awq_gate_up_silu_mul, interleave_gate_up, silu_and_mul

    per_copy = int4_bytes(*GATE_UP)
    ws = make_int4(torch, *GATE_UP, copies_for(per_copy), gen, dev)
    wis = [interleave_gate_up(w) for w in ws]
    for m in (1, 4, 16, 64, 128, 2048):
        x = torch.randn(m, GATE_UP[1], generator=gen, device=dev).to(torch.bfloat16)

        def unfused(i):
            import hydraserve_amd as hs

            gate, up = hs.awq_linear(x, ws[i % len(ws)]).chunk(2, dim=-1)
            return silu_and_mul(gate.contiguous(), up.contiguous())

        def fused(i):
            return awq_gate_up_silu_mul(x, wis[i % len(wis)])

        ms_u, _ = graph_time_ms(torch, unfused, 10, len(ws))
        ms_f, _ = graph_time_ms(torch, fused, 10, len(ws))
        r = {"kind": "int4", "shape": "gate_up+silu_and_mul", "M": m, "N": GATE_UP[0], "K": GATE_UP[1],
             "unfused_us": round(ms_u * 1e3, 2), "fused_us": round(ms_f * 1e3, 2)}
        print(json.dumps(r), file=sys.stderr, flush=True)
        out.append(r)
    del ws, wis
    torch.cuda.empty_cache()
    run("int4", "qkv", *QKV, [64, 1024])
    run("int4", "o_proj", *O_PROJ, [64, 1024])
    run("int4", "gdn_in", *GDN_IN, [64, 1024])
    layer = {}
    for r in out:
        if r["kind"] == "int4" and r["shape"] in ("qkv", "o_proj", "gdn_in", "gate_up", "down") and r["M"] in (64, 1024):
            layer.setdefault(r["M"], 0.0)
            layer[r["M"]] += r["us"]
    out.append({"config4_layer_us": {str(m): round(v, 2) for m, v in layer.items()}})
    print(json.dumps(out[-1]), file=sys.stderr, flush=True)
    return out


if __name__ == "__main__":
    main()
