"""Benchmark: SEW-ResNet18 (ADD, LIF tau=2, v_th=1, hard reset) T=4, B=32,
3x224x224 direct-encoded input, fused by catfuse_amd.optimize on one MI355X.

One step = one full forward of the fused network over the batch (all T
steps, stem to logits) on synthetic inputs resident in HBM, with a
functional.reset_net before it: by default a replay of the HIP graph that
catfuse_amd.graph.capture records for reset_net + forward (the batch is
copied into the graph's input first, inside the timed step; the replay's
output is checked against the eager forward's); --eager times the eager
launches instead.  Prints ONE JSON line (rank 0):
  value      = images/s = B / (seconds per step)
  roofline   = dominant kernel (the MFMA conv, conv_halo_kernel behind
               cf_conv_mfma) achieved TFLOP/s over its launches that ran the
               MFMA K loop (dense route) vs the 2.5 PFLOP/s fp16 dense MFMA
               peak, timed with HIP events on the launch stream around every
               launch of an eager pass over the same steps (the kernels the
               graph replays); the launches that took the StaticZero route
               (all-zero input: no K loop) are reported apart, as output
               bytes written per second vs the 8 TB/s HBM peak
  lif_tails  = standalone LIF-family kernels' achieved HBM GB/s vs 8 TB/s
  cpu_baseline = the CPU oracle (SpikingJelly-equivalent PyTorch/C
               multi-step path, fp32) on a bounded sample of the same
               workload on this host's cores
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "SEW-ResNet18 T=4 images/s on 1 MI355X; fused-LIF HBM GB/s vs peak"
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBPS = 8000.0


def build_model(num_classes=1000, seed=0, workload="sew_resnet18"):
    import torch
    from catfuse_amd import snn
    g = torch.Generator().manual_seed(seed)
    if workload == "spikformer_8_384":
        # config C4: random init (seeded kaiming weights, config-0 BN statistics)
        m = snn.spikformer_8_384(num_classes=num_classes, T=4)
        snn.kaiming_init(m, g)
        snn.randomize_bn(m, g)
        return m.eval()
    m = snn.sew_resnet18(num_classes=num_classes, cnf="ADD", tau=2.0, v_threshold=1.0,
                         v_reset=0.0)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    return m.eval()


def traffic_from_profiles(name="conv_halo_sew_resnet18_traffic.json"):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 PMC summary profiles/<name>, or None when it has not been
    collected."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("hbm_bytes_per_launch")
    except Exception:
        return None


def measure_tails(dev, reps=20):
    """Standalone LIF-family kernels at SEW-RN18 / C1 shapes; GB/s from the
    algorithmic bytes of each launch and its HIP-event duration."""
    import torch
    from catfuse_amd import runtime
    out = []
    g = torch.Generator(device=dev).manual_seed(0)
    cases = [
        ("lif", (4, 32, 64, 56, 56), 0),        # C3 layer1 tail: (8T+8)N
        ("bn_lif", (4, 32, 64, 56, 56), 1),
        ("add_lif", (4, 32, 64, 56, 56), 3),    # (12T+8)N
        ("lif", (4, 32, 256, 14, 14), 0),       # C1 tail
    ]
    for name, shape, mode in cases:
        T, B, C, H, W = shape
        z = torch.randn(shape, device=dev, generator=g)
        z2 = torch.randn(shape, device=dev, generator=g) if mode in (2, 3, 4) else None
        sc = torch.rand(C, device=dev, generator=g) + 0.5
        sh = torch.randn(C, device=dev, generator=g) * 0.1
        v0 = torch.zeros(B, C, H, W, device=dev)
        for _ in range(3):
            runtime.lif_multistep(z, v0, mode=mode, z2=z2, scale=sc, shift=sh, channels=C, hw=H * W)
        timer = runtime.KernelTimer()
        runtime.set_timer(timer)
        for _ in range(reps):
            runtime.lif_multistep(z, v0, mode=mode, z2=z2, scale=sc, shift=sh, channels=C, hw=H * W)
        runtime.set_timer(None)
        s = next(iter(timer.summary().values()))
        gbps = s["bytes"] / (s["ms_total"] * 1e-3) / 1e9
        out.append({"kernel": f"cf_lif_multistep/{name}", "shape": list(shape),
                    "bytes_per_launch": s["bytes"] // s["launches"],
                    "us_per_launch": round(s["ms_avg"] * 1e3, 2), "GB/s": round(gbps, 1),
                    "frac": round(gbps / PEAK_HBM_GBPS, 4)})
        del z, z2
    x = torch.rand((4, 32, 128, 32, 32), device=dev, generator=g)
    for _ in range(3):
        runtime.avgpool2x2_lif(x)
    timer = runtime.KernelTimer()
    runtime.set_timer(timer)
    for _ in range(reps):
        runtime.avgpool2x2_lif(x)
    runtime.set_timer(None)
    s = next(iter(timer.summary().values()))
    gbps = s["bytes"] / (s["ms_total"] * 1e-3) / 1e9
    out.append({"kernel": "cf_avgpool2x2_lif", "shape": [4, 32, 128, 32, 32],
                "bytes_per_launch": s["bytes"] // s["launches"],
                "us_per_launch": round(s["ms_avg"] * 1e3, 2), "GB/s": round(gbps, 1),
                "frac": round(gbps / PEAK_HBM_GBPS, 4)})
    return out


def cpu_baseline(model, T, image, budget_s=12.0, forward=None):
    """Oracle forward (fp32 torch CPU conv + eval BN + C LIF, SpikingJelly
    multi-step semantics) on this host: 1 warm-up image, then batches of 2
    images until about budget_s seconds have been timed."""
    import torch
    import oracle
    fwd = forward or oracle.sew_resnet_forward
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1)
    x1 = torch.randn(1, 3, image, image, generator=g)
    fwd(model, x1.unsqueeze(0).expand(T, 1, 3, image, image), conv_dtype=torch.float32)
    x2 = torch.randn(2, 3, image, image, generator=g)
    xs = x2.unsqueeze(0).expand(T, 2, 3, image, image)
    imgs, t_total = 0, 0.0
    while t_total < budget_s:
        t0 = time.perf_counter()
        fwd(model, xs, conv_dtype=torch.float32)
        t_total += time.perf_counter() - t0
        imgs += 2
    return {"value": round(imgs / t_total, 3), "unit": "images/s", "cores": threads,
            "kind": "port",
            "sample": f"{imgs} images of 3x{image}x{image}, T={T}, in batches of 2 "
                      f"({t_total:.1f} s), after 1 warm-up image"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--image", type=int, default=224)
    ap.add_argument("--T", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-tails", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of the captured HIP graph")
    ap.add_argument("--workload", default="sew_resnet18",
                    choices=["sew_resnet18", "spikformer_8_384"],
                    help="sew_resnet18: the headline metric (config C3); spikformer_8_384: "
                         "config C4 (spiking transformer), its own metric line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every GPU box in this setup has a single "
              "MI355X; run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import catfuse_amd
    from catfuse_amd import graph as cf_graph
    from catfuse_amd import runtime, snn

    dev = torch.device("cuda", 0)
    T, B, HW = args.T, args.batch, args.image
    spikformer = args.workload == "spikformer_8_384"
    model = build_model(workload=args.workload)
    fused, stats = catfuse_amd.optimize(model, device=dev, T=T)
    fused.eval()
    g = torch.Generator(device=dev).manual_seed(0)
    img = torch.randn(B, 3, HW, HW, device=dev, generator=g)
    x = img.unsqueeze(0).expand(T, B, 3, HW, HW)      # direct encoding, resident in HBM

    with torch.no_grad():
        for _ in range(args.warmup):
            snn.functional.reset_net(fused)
            fused(x)
        torch.cuda.synchronize()
        catfuse_amd.check_status(dev)

        # Eager pass with HIP events around every launch (per-kernel times
        # for the roofline; the same kernels the graph replays).
        timer = runtime.KernelTimer()
        runtime.set_timer(timer)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            snn.functional.reset_net(fused)
            y = fused(x)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        runtime.set_timer(None)
        ms_eager = (t1 - t0) * 1e3 / args.steps
        ms = ms_eager
        mode = "eager"
        if not args.eager:
            # One step = copy the batch into the captured input + replay of
            # reset_net + the whole fused forward (HIP graph).
            graphed = cf_graph.capture(fused, x)
            y_ref = y.clone()
            for _ in range(args.warmup):
                graphed(img)
            torch.cuda.synchronize()
            if not torch.equal(graphed(img), y_ref):
                print("graph replay differs from the eager forward", file=sys.stderr)
                sys.exit(1)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                y = graphed(img)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            ms = (t1 - t0) * 1e3 / args.steps
            mode = "hip_graph"
        catfuse_amd.check_status(dev)
    kern = timer.summary()
    ips = B / (ms * 1e-3)

    def agg(names):
        ds = [kern.get(n, {}) for n in names]
        return (sum(d.get("ms_total", 0.0) for d in ds), sum(d.get("flops", 0) for d in ds),
                sum(d.get("bytes", 0) for d in ds), sum(d.get("launches", 0) for d in ds))

    tot_ms, tot_fl, _, launches = agg(["conv_mfma", "conv_mfma_sparse"])
    z_ms, _, z_bytes, z_launches = agg(["conv_mfma_staticzero", "conv_mfma_sparse_staticzero"])
    achieved = tot_fl / (tot_ms * 1e-3) / 1e12 if tot_ms else 0.0
    roofline = {"kernel": "conv_halo_kernel (cf_conv_mfma fused Conv-BN-LIF), launches that run "
                          "the MFMA K loop",
                "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                "traffic": traffic_from_profiles(),
                "flops_per_launch_avg": tot_fl // max(1, launches),
                "us_per_launch_avg": round(tot_ms * 1e3 / max(1, launches), 2),
                "launches_per_step": launches // args.steps}
    z_gbps = z_bytes / (z_ms * 1e-3) / 1e9 if z_ms else 0.0
    # route of each conv launch of one forward, in launch order (D: MFMA K
    # loop, Z: StaticZero), decided on the device and read back here
    conv_recs = [r for r in timer.records if r[0].startswith("conv_mfma")]
    per_fwd = len(conv_recs) // max(1, args.steps)
    route_seq = "".join("Z" if (r[5] is not None and r[5].is_zero()) else "D"
                        for r in conv_recs[:per_fwd])
    staticzero = {"kernel": "conv_halo_kernel on the StaticZero route (all-zero input: BN bias "
                            "-> LIF, no K loop)",
                  "bound": "hbm", "launches_per_step": z_launches // args.steps,
                  "us_per_launch_avg": round(z_ms * 1e3 / max(1, z_launches), 2),
                  "bytes_per_launch_avg": z_bytes // max(1, z_launches),
                  "achieved": round(z_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                  "frac": round(z_gbps / PEAK_HBM_GBPS, 4),
                  "conv_route_sequence": route_seq}
    per_kernel = {k: {"launches_per_step": v["launches"] // args.steps,
                      "ms_per_step": round(v["ms_total"] / args.steps, 4)}
                  for k, v in kern.items()}

    if spikformer:
        # token linears (1x1 convs over the token rows) and the attention core
        l_ms, l_fl, _, l_n = agg(["linear_tokens"])
        lz_ms, _, _, lz_n = agg(["linear_tokens_staticzero"])
        # route of each token-linear launch of one forward (D: MFMA K loop,
        # Z: StaticZero), decided on the device and read back here
        lin_recs = [r for r in timer.records if r[0].startswith("linear_tokens")]
        per_fwd_l = len(lin_recs) // max(1, args.steps)
        lin_seq = "".join("Z" if (r[5] is not None and r[5].is_zero()) else "D"
                          for r in lin_recs[:per_fwd_l])
        a_ms, a_fl, a_b, a_n = agg(["spike_attention"])
        # the dominant MFMA work is the patch splitter's 3x3 convs (the token
        # linears take StaticZero when their input is all zero)
        roofline["kernel"] = ("conv_halo_kernel 3x3 (cf_conv_mfma: the SPS Conv-BN-LIF stages), "
                              "launches that run the MFMA K loop")
        roofline["traffic"] = traffic_from_profiles("conv_halo_spikformer_8_384_traffic.json")
        roofline["conv_route_sequence"] = route_seq
        ach = l_fl / (l_ms * 1e-3) / 1e12 if l_ms else 0.0
        linears = {"kernel": "conv_halo_kernel 1x1 (cf_conv_mfma: fused Linear-BN1d-LIF over the "
                             "token rows)",
                   "launches_per_step": (l_n + lz_n) // args.steps,
                   "mfma_route": {"launches_per_step": l_n // args.steps,
                                  "us_per_launch_avg": round(l_ms * 1e3 / max(1, l_n), 2),
                                  "achieved": round(ach, 2), "unit": "TFLOP/s"},
                   "staticzero_route": {"launches_per_step": lz_n // args.steps,
                                        "us_per_launch_avg": round(lz_ms * 1e3 / max(1, lz_n), 2)},
                   "linear_route_sequence": lin_seq}
        a_gbps = a_b / (a_ms * 1e-3) / 1e9 if a_ms else 0.0
        attention = {"kernel": "spike_attention_kernel (cf_spike_attention_lif)",
                     "launches_per_step": a_n // args.steps,
                     "us_per_launch_avg": round(a_ms * 1e3 / max(1, a_n), 2),
                     "achieved": round(a_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(a_gbps / PEAK_HBM_GBPS, 4)}
    result = {
        "metric": METRIC, "value": round(ips, 2), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "mode": mode, "eager_ms_per_step": round(ms_eager, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (conv: fp16 hi/lo split weights x fp16-exact spikes on MFMA, fp32 acc)",
        "data": "synthetic (seeded N(0,1) images, random kaiming weights, config BN stats)",
        "config": {"workload": "sew_resnet18_adds_T4_B32_224", "T": T, "batch": B,
                   "image": [3, HW, HW], "encoding": "direct (input repeated over T)",
                   "fused_lif_nodes": stats["fused_lif_nodes"],
                   "total_lif_nodes": stats["total_lif_nodes"]},
        "roofline": roofline,
        "staticzero_convs": staticzero,
        "kernels": per_kernel,
    }
    if spikformer:
        result["metric"] = "Spikformer-8-384 T=4 images/s on 1 MI355X (config C4)"
        result["config"] = {"workload": "spikformer_8_384_T4_B32_224", "T": T, "batch": B,
                            "image": [3, HW, HW], "tokens": 196, "dim": 384, "heads": 12,
                            "blocks": 8, "encoding": "direct (input repeated over T)",
                            "fused_lif_nodes": stats["fused_lif_nodes"],
                            "total_lif_nodes": stats["total_lif_nodes"]}
        result["dtype"] = ("fp32 (linears/convs: fp16 hi/lo split weights x fp16-exact spikes on "
                           "MFMA, fp32 acc; attention: exact integer Q(K^T V), one fp32 rounding)")
        result["token_linears"] = linears
        result["attention"] = attention
    if not args.no_tails and not spikformer:
        result["lif_tails"] = measure_tails(dev)
    if not args.no_cpu_baseline:
        import oracle
        result["cpu_baseline"] = cpu_baseline(
            model, T, HW, args.cpu_budget,
            forward=oracle.spikformer_forward if spikformer else None)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
