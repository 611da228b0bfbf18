"""SparseFlow / dense crossover of the gfx950 kernels (MI355X routing thresholds).

The reference calibrates its routing on V100 measurements: SparseFlow when the
input sparsity exceeds 0.7 (catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524,
threshold in catfuse/sparseflow/config.py:15-61), the SparseFlow/DenseKeep
comparisons of experiments/results/sparsity_scan.csv.  This module repeats the
measurement for the gfx950 implementations on one fused Conv3x3 -> BN -> LIF
layer (config C1 by default: x [4, 32, 256, 14, 14], 256 -> 256 channels) and
inputs of several spike rates in two spatial patterns:

  iid      Bernoulli(rate) spikes;
  block    per (t, b, c) and 8x8 spatial block, the block is zero with
           probability 0.7, Bernoulli(rate) elsewhere (the granularity of
           the reference's tests/test_70_oracle_gap.py:112-124);
  spatial  per (t, b) and 8x8 spatial block, the block is zero in every
           channel with probability 0.7, Bernoulli(rate) elsewhere (silent
           regions, the structure channel-group skipping can exploit).

Routes timed per input (device time of one layer call):

  SparseFlow  activity scan + tile prescan + the chunk-skipping conv, forced
              (every nonzero input takes the sparse route);
  StreamFuse  the fused dense conv (z on chip);
  DenseKeep   the conv writing z, then the multi-step LIF (the reference's
              dense schedule);
  auto        STFusionConvBNLIF's device-side route with the profile's
              threshold.

Inputs come as a fused layer's output (its fp16 NHWC copy and count block:
how a SparseFlow layer sees its input inside a network; StaticZero then needs
no counting pass) or, with plain=True, as an fp32 tensor (the layer packs it).
Each route's call is captured `calls` times in a HIP graph and replayed
`reps` times; time per call = median replay time / calls.

    python -m catfuse_amd.sparseflow.crossover [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys
from typing import Dict, List, Optional, Sequence

import torch

RATES = (0.0, 0.001, 0.01, 0.05, 0.1, 0.2, 0.3, 0.5)
PATTERNS = ("iid", "block", "spatial")
ROUTES = ("SparseFlow", "StreamFuse", "DenseKeep", "auto")


def c1_input(rate: float, pattern: str, shape=(4, 32, 256, 14, 14), seed: int = 0,
             block: int = 8, p_zero_block: float = 0.7) -> torch.Tensor:
    """fp32 CPU spikes [T, B, C, H, W] of the given rate and pattern."""
    g = torch.Generator().manual_seed(seed)
    T, B, C, H, W = shape
    x = (torch.rand(shape, generator=g) < rate).float()
    if pattern in ("block", "spatial"):
        gh, gw = -(-H // block), -(-W // block)
        kc = C if pattern == "block" else 1
        keep = (torch.rand((T, B, kc, gh, gw), generator=g) >= p_zero_block).float()
        keep = keep.repeat_interleave(block, 3).repeat_interleave(block, 4)[..., :H, :W]
        x = x * keep
    elif pattern != "iid":
        raise ValueError(f"unknown pattern {pattern!r}")
    return x


def as_fused_output(x: torch.Tensor) -> torch.Tensor:
    """x (GPU fp32 spikes) re-expressed as a fused conv's output: an
    NHWC-backed tensor carrying the fp16 copy and a count block holding
    count_nonzero(x), as the producing conv would have published it."""
    from catfuse_amd import runtime
    T, B, C, H, W = x.shape
    cp = runtime.pad32(C)
    nhwc = torch.zeros((T * B, H, W, cp), dtype=torch.float16, device=x.device)
    nhwc[..., :C] = x.reshape(T * B, C, H, W).permute(0, 2, 3, 1).half()
    y = runtime.lazy_output(tuple(x.shape), nhwc, x.device)
    blk = runtime.count_block(x.device)
    blk[1] = int(torch.count_nonzero(x))
    runtime.attach_count(y, blk, [0])
    return y


def _layer(C_in: int, C_out: int, device, seed: int = 0):
    from catfuse_amd.implementations.base import ConvLIFParams, ConvLIFSpec
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(C_out, C_in, 3, 3, generator=g) * (2.0 / (C_in * 9)) ** 0.5
    mean = torch.randn(C_out, generator=g) * 0.1
    var = torch.rand(C_out, generator=g) + 0.5
    gamma = torch.rand(C_out, generator=g) * 0.4 + 0.8
    beta = torch.randn(C_out, generator=g) * 0.1
    scale = gamma / torch.sqrt(var + 1e-5)
    shift = beta - mean * scale
    spec = ConvLIFSpec(C_in, C_out, 3, 1, 1, has_conv_bias=False, has_bn=True, tau=2.0,
                       v_threshold=1.0, v_reset=0.0, decay_input=True)
    params = ConvLIFParams(w.to(device), None, scale.to(device), shift.to(device))
    return spec, params


def _implementations():
    from catfuse_amd.implementations.dense_keep import DenseKeep
    from catfuse_amd.implementations.sparse_flow import SparseFlow
    from catfuse_amd.implementations.stream_fuse import StreamFuse
    return {"SparseFlow": SparseFlow(sparsity_threshold=-1.0), "StreamFuse": StreamFuse(),
            "DenseKeep": DenseKeep(), "auto": SparseFlow()}


def _time_graph(fn, calls: int, reps: int, device) -> float:
    """Median microseconds per call of fn over `reps` replays of a graph
    holding `calls` calls."""
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        fn()
        fn()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize(device)
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize(device)
        times.append(e0.elapsed_time(e1) * 1e3 / calls)
    del graph
    return statistics.median(times)


def sweep(device=None, rates: Sequence[float] = RATES, patterns: Sequence[str] = PATTERNS,
          shape=(4, 32, 256, 14, 14), C_out: Optional[int] = None, plain: bool = False,
          calls: int = 20, reps: int = 5, seed: int = 0) -> List[Dict]:
    """One row per (pattern, rate): input density and the microseconds per
    call of every route."""
    from catfuse_amd.state import StateBuffer
    device = torch.device(device or "cuda:0")
    T, B, C, H, W = shape
    spec, params = _layer(C, C_out or C, device, seed)
    impls = _implementations()
    rows = []
    with torch.no_grad():
        for pattern in patterns:
            for rate in rates:
                xc = c1_input(rate, pattern, shape, seed=seed + 1)
                xd = xc.to(device)
                x = xd if plain else as_fused_output(xd)
                row = {"pattern": pattern, "rate": rate,
                       "density": float(torch.count_nonzero(xc)) / xc.numel()}
                ref = None
                for name in ROUTES:
                    impl = impls[name]

                    def call(impl=impl):
                        return impl.forward(x, spec, params, StateBuffer())
                    y = call()
                    if ref is None:
                        ref = y.clone()
                    elif not torch.equal(y, ref):
                        raise RuntimeError(f"{name} differs from SparseFlow at {pattern} {rate}")
                    row[name] = _time_graph(call, calls, reps, device)
                rows.append(row)
    return rows


def crossover(rows: List[Dict]) -> Dict[str, Optional[float]]:
    """Per pattern, the lowest input sparsity at which forced SparseFlow is
    faster than the best dense route (None: at no measured nonzero rate)."""
    out = {}
    for pattern in sorted({r["pattern"] for r in rows}):
        wins = [1.0 - r["density"] for r in rows
                if r["pattern"] == pattern and r["density"] > 0.0
                and r["SparseFlow"] < min(r["StreamFuse"], r["DenseKeep"])]
        out[pattern] = min(wins) if wins else None
    return out


def format_table(rows: List[Dict]) -> str:
    lines = ["| pattern | rate | density | " + " | ".join(f"{n} (us)" for n in ROUTES) + " |",
             "|---|---|---|" + "---|" * len(ROUTES)]
    for r in rows:
        lines.append(f"| {r['pattern']} | {r['rate']:g} | {r['density']:.4f} | "
                     + " | ".join(f"{r[n]:.1f}" for n in ROUTES) + " |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--rates", type=float, nargs="*", default=list(RATES))
    ap.add_argument("--patterns", nargs="*", default=list(PATTERNS))
    ap.add_argument("--shape", type=int, nargs=5, default=[4, 32, 256, 14, 14])
    ap.add_argument("--plain", action="store_true", help="fp32 inputs (the layer packs them)")
    ap.add_argument("--calls", type=int, default=20)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("the crossover sweep needs a GPU", file=sys.stderr)
        return 2
    rows = sweep(rates=args.rates, patterns=args.patterns, shape=tuple(args.shape),
                 plain=args.plain, calls=args.calls, reps=args.reps)
    print(format_table(rows))
    print("crossover (lowest sparsity where SparseFlow wins):", crossover(rows))
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"shape": args.shape, "plain": args.plain, "rows": rows,
                       "crossover": crossover(rows)}, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
