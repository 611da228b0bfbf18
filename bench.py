"""Benchmark of the fused SNN inference path on one MI355X.

Workloads (--workload):
  sew_resnet18     the headline (config C3): SEW-ResNet18 (ADD, LIF tau=2,
                   v_th=1, hard reset), T=4, B=32, 3x224x224 direct-encoded,
                   random kaiming weights, config-0 BN statistics; plus its
                   "live" companion: the same network with v_th = 0.1, the
                   reference's own end-to-end setting
                   (benchmarks/bench_sew_resnet18_e2e.py:101-115) under its
                   liveness check (>= 80% of the SEW blocks with spike rate
                   > 1e-4, :268-287), reported in its own keys;
  spikformer_8_384 config C4 (spiking transformer), its own metric line;
  vgg11_bn         config C2: spiking VGG-11-BN, T=4, B=64, 3x32x32; plus
                   its live companion at v_th = 0.1 (the reference's VGG
                   setting, benchmarks/bench_vgg11_e2e.py:74-80) under that
                   harness's liveness check (>= 80% of the fused conv and
                   Linear-LIF layers with spike rate > 1e-4, :205-241);
  sf_crossover     the SparseFlow / dense crossover sweep of one fused
                   Conv3x3-BN-LIF layer (config C1 shapes) that sets the
                   MI355X routing threshold; prints a markdown table.

One step = one full forward of the fused network over the batch (all T
steps, stem to logits) on synthetic inputs resident in HBM, after a
functional.reset_net: by default a replay of the HIP graph that
catfuse_amd.capture records for reset_net + forward, on the batch resident
in the graph's input buffer (copied there once, before timing, by the
replay whose output is checked against the eager forward's; each timed step
replays the whole forward on it, with no copy); --eager times the eager
launches.
Prints ONE JSON line:
  value        images/s = B / (seconds per step)
  roofline     the dominant kernel (conv_halo_kernel behind cf_conv_mfma, the
               fused Conv-BN-LIF) over its launches that ran the MFMA K loop:
               dense-equivalent FLOPs / HIP-event time on the launch stream,
               vs the 2.5 PFLOP/s dense fp16 MFMA peak
  per_layer    every conv launch of one forward: layer, route, time, TFLOP/s
  staticzero_convs  the conv launches that took StaticZero (all-zero input)
  lif_tails    standalone LIF-family kernels' HBM GB/s vs 8 TB/s
  cpu_baseline the CPU oracle's forward (fp32 torch conv + eval BN + C LIF,
               SpikingJelly multi-step semantics) on this host's cores: 1
               warm-up forward, then >= 3 timed forwards of a stated batch,
               median; beside it the eager SpikingJelly-equivalent model
               (catfuse_amd.snn, LIFNode's recurrence in torch), same protocol
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "SEW-ResNet18 T=4 images/s on 1 MI355X; fused-LIF HBM GB/s vs peak"
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBPS = 8000.0
# spin ahead of each timed launch (torch.cuda._sleep cycles; ~40-80 us on
# gfx950), longer than the host's per-launch work
SETTLE_CYCLES = 200_000
LIVE_V_THRESHOLD = 0.1      # benchmarks/bench_sew_resnet18_e2e.py:101-115
LIVE_RATE = 1e-4            # a block is alive above this spike rate (:268-287)
LIVE_MIN_FRACTION = 0.8

# images per CPU-baseline forward (a bounded sample: ~10-30 s of host work)
CPU_BATCH = {"sew_resnet18": 8, "spikformer_8_384": 2, "vgg11_bn": 64}

WORKLOADS = {
    "sew_resnet18": dict(T=4, batch=32, image=224),
    "spikformer_8_384": dict(T=4, batch=32, image=224),
    "vgg11_bn": dict(T=4, batch=64, image=32),
}


# ---------------------------------------------------------------------------
# models and timing
# ---------------------------------------------------------------------------

def build_model(workload="sew_resnet18", v_threshold=1.0, seed=0, num_classes=None):
    """The unfused SpikingJelly-style model of a workload, seeded kaiming
    weights and config-0 BN statistics."""
    import torch
    from catfuse_amd import snn
    g = torch.Generator().manual_seed(seed)
    if workload == "spikformer_8_384":
        m = snn.spikformer_8_384(num_classes=num_classes or 1000, T=4, v_threshold=v_threshold)
    elif workload == "vgg11_bn":
        m = snn.spiking_vgg11_bn(num_classes=num_classes or 10, v_threshold=v_threshold)
    else:
        m = snn.sew_resnet18(num_classes=num_classes or 1000, cnf="ADD", tau=2.0,
                             v_threshold=v_threshold, v_reset=0.0)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    return m.eval()


def _conv_patterns():
    from catfuse_amd.patterns import PartialFusionConvBNLIF, PartialFusionConvLIF
    from catfuse_amd.sparseflow.ops.st_fusion_conv_bn_lif import STFusionConvBNLIF
    from catfuse_amd.patterns import FusedLinearLIF
    from catfuse_amd.transformer import FusedLinearBNLIF
    return (PartialFusionConvBNLIF, PartialFusionConvLIF, STFusionConvBNLIF, FusedLinearLIF,
            FusedLinearBNLIF)


def label_launches(model, timer):
    """Forward hooks on every fused conv / linear layer that attribute the
    timer records its call appended to the layer's module path.  Returns
    (spans, handles); spans: [(name, first record, end record)]."""
    spans, handles, stack = [], [], []
    kinds = _conv_patterns()
    for name, mod in model.named_modules():
        if isinstance(mod, kinds):
            handles.append(mod.register_forward_pre_hook(
                lambda m, a: stack.append(len(timer.records))))
            handles.append(mod.register_forward_hook(
                lambda m, a, o, name=name: spans.append((name, stack.pop(),
                                                         len(timer.records)))))
    return spans, handles


def time_forward(fused, x, img, steps, warmup, eager=False, label=False):
    """Warm-up, three timed eager passes of `steps` forwards (their median is
    ms_eager), an eager pass with HIP events around every launch (per-kernel
    times; the same kernels the graph replays), then (unless eager) `steps`
    replays of the captured graph.  Returns dict(ms, ms_eager, mode, timer,
    spans)."""
    import torch
    import catfuse_amd
    from catfuse_amd import graph as cf_graph
    from catfuse_amd import runtime, snn
    dev = x.device
    with torch.no_grad():
        for _ in range(warmup):
            snn.functional.reset_net(fused)
            fused(x)
        torch.cuda.synchronize()
        catfuse_amd.check_status(dev)
        # eager: the median of three passes of `steps` forwards (the host
        # launches them, so a pass also measures the host's other load)
        passes = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                snn.functional.reset_net(fused)
                y = fused(x)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            passes.append((t1 - t0) * 1e3 / steps)
        ms_eager = sorted(passes)[1]
        # per-launch times: a second eager pass with the GPU kept busy ahead
        # of every launch, so each event pair brackets the kernel alone
        timer = runtime.KernelTimer(settle_cycles=SETTLE_CYCLES)
        spans, handles = label_launches(fused, timer) if label else ([], [])
        runtime.set_timer(timer)
        for _ in range(steps):
            snn.functional.reset_net(fused)
            y = fused(x)
        torch.cuda.synchronize()
        runtime.set_timer(None)
        for h in handles:
            h.remove()
        ms, mode = ms_eager, "eager"
        if not eager:
            graphed = cf_graph.capture(fused, x)
            y_ref = y.clone()
            for _ in range(warmup):
                graphed(img)
            torch.cuda.synchronize()
            if not torch.equal(graphed(img), y_ref):
                raise SystemExit("graph replay differs from the eager forward")
            torch.cuda.synchronize()
            # the batch is resident in the captured graph's input buffer (the
            # check above copied it there): each timed step replays the whole
            # forward on it, without re-copying the same 3xHxW images
            t0 = time.perf_counter()
            for _ in range(steps):
                graphed()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            ms, mode = (t1 - t0) * 1e3 / steps, "hip_graph"
            del graphed
        catfuse_amd.check_status(dev)
    return dict(ms=ms, ms_eager=ms_eager, mode=mode, timer=timer, spans=spans, steps=steps)


def _agg(kern, names):
    ds = [kern.get(n, {}) for n in names]
    return (sum(d.get("ms_total", 0.0) for d in ds), sum(d.get("flops", 0) for d in ds),
            sum(d.get("bytes", 0) for d in ds), sum(d.get("launches", 0) for d in ds))


def conv_roofline(kern, steps, names=("conv_mfma", "conv_mfma_sparse", "conv_pair"),
                  traffic=None):
    tot_ms, tot_fl, _, launches = _agg(kern, names)
    achieved = tot_fl / (tot_ms * 1e-3) / 1e12 if tot_ms else 0.0
    return {"kernel": "conv_halo_kernel and conv_halo_pair_kernel (cf_conv_mfma / "
                      "cf_conv_halo_pair fused Conv-BN-LIF), launches that run the MFMA K loop",
            "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "flops_per_launch_avg": tot_fl // max(1, launches),
            "us_per_launch_avg": round(tot_ms * 1e3 / max(1, launches), 2),
            "launches_per_step": launches // max(1, steps)}


def launch_floor_us(dev, reps=20):
    """Duration of a launch that does nothing (cf_resolve_copy of a copy its
    descriptor records as written: every workgroup returns after one load),
    timed like the forward's launches: the per-launch floor of the box."""
    import torch
    from catfuse_amd import _hip, runtime
    buf = torch.zeros(64, dtype=torch.uint8, device=dev)
    desc = runtime.written_desc(dev)
    timer = runtime.KernelTimer(settle_cycles=SETTLE_CYCLES)
    st = _hip.stream(dev)
    for _ in range(reps):
        ev = timer.start()
        _hip.check(_hip.lib().cf_resolve_copy(buf.data_ptr(), 64, desc.data_ptr(), st),
                   "cf_resolve_copy")
        timer.stop("floor", ev)
    d = timer.summary()["floor"]
    return round(d["ms_total"] * 1e3 / d["launches"], 2)


def staticzero_summary(kern, steps, floor_us=None, names=("conv_mfma_staticzero",
                                                          "conv_mfma_sparse_staticzero",
                                                          "conv_pair_staticzero")):
    z_ms, _, z_bytes, z_n = _agg(kern, names)
    elided = sum(kern.get(n, {}).get("elided", 0) for n in names)
    gbps = z_bytes / (z_ms * 1e-3) / 1e9 if z_ms else 0.0
    return {"kernel": "conv_halo_kernel on the StaticZero route (all-zero input: BN bias -> "
                      "LIF, no K loop)",
            "launches_per_step": z_n // max(1, steps),
            "elided_per_step": elided // max(1, steps),
            "us_per_step": round(z_ms * 1e3 / max(1, steps), 2),
            "us_per_launch_avg": round(z_ms * 1e3 / max(1, z_n), 2),
            "launch_floor_us": floor_us,
            "bytes_per_step": z_bytes // max(1, steps),
            "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "note": "elided launches store no output (their descriptors record an all-zero "
                    "or identity-aliased copy and per-channel state): launch floor bound"}


CONV_LAUNCHES = ("conv_mfma", "conv_pair")   # timer names of the halo-kernel conv launches


def route_sequence(timer, prefix, steps):
    """Route of each launch named prefix* in one forward, in launch order
    (D: the MFMA K loop ran, Z: StaticZero), read back from the devices'
    count blocks after the timed region."""
    recs = [r for r in timer.records if r[0].startswith(prefix)]
    per = len(recs) // max(1, steps)
    return "".join("Z" if (r[5] is not None and r[5].is_zero()) else "D" for r in recs[:per])


def per_layer_table(res, kernels=("conv_mfma", "conv_pair", "conv_stem", "conv_direct",
                                  "linear_tokens")):
    """One row per conv / linear launch of one forward (averaged over the
    eager steps): layer path, kernel, route, us, dense-equivalent TFLOP/s and
    fraction of the MFMA peak."""
    timer, spans, steps = res["timer"], res["spans"], res["steps"]
    label = {}
    for name, a, b in spans:
        for i in range(a, b):
            label.setdefault(i, name)
    rows = {}
    order = []
    for i, (kname, e0, e1, fl, nb, route) in enumerate(timer.records):
        if not kname.startswith(kernels):
            continue
        key = (label.get(i, "?"), kname)
        if key not in rows:
            rows[key] = dict(layer=key[0], kernel=kname, n=0, ms=0.0, flops=0, zero=False)
            order.append(key)
        r = rows[key]
        r["n"] += 1
        r["ms"] += e0.elapsed_time(e1)
        r["flops"] += fl
        r["zero"] = bool(route is not None and route.is_zero())
    out = []
    for key in order:
        r = rows[key]
        us = r["ms"] * 1e3 / r["n"]
        fl = r["flops"] / r["n"]
        tf = 0.0 if r["zero"] else fl / (us * 1e-6) / 1e12
        out.append({"layer": r["layer"], "kernel": r["kernel"], "route": "Z" if r["zero"] else "D",
                    "us": round(us, 2), "gflop": round(fl / 1e9, 3),
                    "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_FP16_TFLOPS, 4)})
    return out


def traffic_from_profiles(name="conv_halo_sew_resnet18_traffic.json"):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 PMC summary profiles/<name>, or None when absent."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("hbm_bytes_per_launch")
    except Exception:
        return None


# modules whose outputs the reference's harnesses check for liveness:
# SEW blocks (benchmarks/bench_sew_resnet18_e2e.py:268-287); every fused
# conv and Linear-LIF (benchmarks/bench_vgg11_e2e.py:205-241)
LIVENESS_MODULES = {
    "sew_resnet18": ("CTFSEWBasicBlock",),
    "vgg11_bn": ("PartialFusionConvBNLIF", "PartialFusionConvBNAvgPoolLIF", "FusedLinearLIF"),
}


def liveness(fused, x, workload="sew_resnet18"):
    """Spike rate of every module the reference's harness checks (SEW blocks,
    or VGG's fused layers): (alive fraction, {module: rate})."""
    import torch
    from catfuse_amd import snn
    rates, hs = {}, []
    kinds = LIVENESS_MODULES[workload]
    for name, mod in fused.named_modules():
        if type(mod).__name__ in kinds:
            hs.append(mod.register_forward_hook(
                lambda m, a, o, name=name: rates.__setitem__(name, float(o.float().mean()))))
    with torch.no_grad():
        snn.functional.reset_net(fused)
        fused(x)
    for h in hs:
        h.remove()
    alive = sum(1 for r in rates.values() if r > LIVE_RATE)
    return alive / max(1, len(rates)), {k: round(v, 6) for k, v in rates.items()}


# ---------------------------------------------------------------------------
# LIF tails
# ---------------------------------------------------------------------------

def _tail_row(kernel, shape, nbytes, us):
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"kernel": kernel, "shape": list(shape), "bytes_per_launch": int(nbytes),
            "us_per_launch": round(us, 2), "GB/s": round(gbps, 1),
            "frac": round(gbps / PEAK_HBM_GBPS, 4)}


def _time_launches(fn, reps, dev):
    """Microseconds per call: `reps` calls captured in one HIP graph, the
    median over 5 replays of the replay time / reps (graph replay keeps the
    host's launch gaps out; each call still includes its dispatch)."""
    return _xo_time_graph(fn, reps, 5, dev)


TAIL_CASES = [
    # name, kernel shape [T, B, C, H, W], cf_lif_multistep mode (None: AvgPool2x2-LIF)
    ("lif", (4, 32, 64, 56, 56), 0),        # C3 layer1 tail: (8T+8)N bytes
    ("bn_lif", (4, 32, 64, 56, 56), 1),
    ("add_lif", (4, 32, 64, 56, 56), 3),    # (12T+8)N
    ("lif", (4, 32, 256, 14, 14), 0),       # C1 tail
    ("avgpool2x2_lif", (4, 32, 128, 32, 32), None),   # 20T+8 bytes per output neuron
]


# buffer sets a cold tail measurement rotates through: together above 1 GiB
# and at least 4, so no launch finds its inputs in the 256 MB Infinity Cache
# (every set is evicted by the others before it is reused)
COLD_BYTES = 3 << 29
COLD_MIN_SETS = 4


def measure_tails(dev, reps=50):
    """Standalone LIF-family kernels at SEW-RN18 / C1 / VGG shapes: GB/s from
    the algorithmic bytes of a launch and the average duration of `reps`
    launches captured back to back in one graph.  Cold (the row's main
    figures, HBM): the launches rotate through buffer sets (inputs, states
    and outputs) totalling more than 1 GiB.  Resident (`resident`): every
    launch on one buffer set, which for the smaller shapes stays in the
    Infinity Cache between launches."""
    import torch
    from catfuse_amd import _hip
    from catfuse_amd.runtime import _lif_args, check, ptr
    L = _hip.lib()
    lif = _lif_args(2.0, 1.0, 0.0, True)
    out = []
    g = torch.Generator(device=dev).manual_seed(0)
    for name, shape, mode in TAIL_CASES:
        T, B, C, H, W = shape
        if mode is None:
            n_out = B * C * (H // 2) * (W // 2)
            nbytes = T * n_out * 20 + 4 * n_out

            def make():
                return dict(x=torch.rand(shape, device=dev, generator=g),
                            s=torch.empty((T, B, C, H // 2, W // 2), device=dev),
                            v=torch.empty((B, C, H // 2, W // 2), device=dev))

            def launch(b):
                # (the stream current at the call: the capture stream inside
                # the timed graph)
                check(L.cf_avgpool2x2_lif(ptr(b["x"]), None, ptr(b["s"]), 0, ptr(b["v"]), T,
                                          B * C, H, W, *lif, _hip.stream(dev)),
                      "cf_avgpool2x2_lif")
            kernel = "cf_avgpool2x2_lif"
        else:
            N = B * C * H * W
            two = mode in (2, 3, 4)
            nbytes = (8 * T + 8) * N + (4 * T * N if two else 0)
            sc = torch.rand(C, device=dev, generator=g) + 0.5
            sh = torch.randn(C, device=dev, generator=g) * 0.1

            def make():
                return dict(z=torch.randn(shape, device=dev, generator=g),
                            z2=torch.randn(shape, device=dev, generator=g) if two else None,
                            v0=torch.zeros(B, C, H, W, device=dev),
                            s=torch.empty(shape, device=dev),
                            v=torch.empty(B, C, H, W, device=dev))

            def launch(b, mode=mode, N=N, sc=sc, sh=sh):
                check(L.cf_lif_multistep(ptr(b["z"]), ptr(b["z2"]), ptr(sc), ptr(sh), mode,
                                         ptr(b["v0"]), ptr(b["s"]), 0, ptr(b["v"]), T, N, C,
                                         H * W, *lif, _hip.stream(dev)), "cf_lif_multistep")
            kernel = f"cf_lif_multistep/{name}"
        nsets = max(COLD_MIN_SETS, -(-COLD_BYTES // nbytes))
        sets = [make() for _ in range(nsets)]
        cnt = [0]

        def rotate():
            launch(sets[cnt[0] % nsets])
            cnt[0] += 1
        us_cold = _time_launches(rotate, max(reps, 2 * nsets), dev)
        us_res = _time_launches(lambda: launch(sets[0]), reps, dev)
        row = _tail_row(kernel, shape, nbytes, us_cold)
        row["buffers"] = {"sets": nsets, "bytes_total": int(nsets * nbytes)}
        res = _tail_row(kernel, shape, nbytes, us_res)
        row["resident"] = {k: res[k] for k in ("us_per_launch", "GB/s", "frac")}
        out.append(row)
        del sets
    return out


def tails_main(args):
    """--workload lif_tails: the LIF-family tails alone (one JSON line per
    kernel), the command the tails' rocprofv3 summaries are taken from."""
    import torch
    dev = torch.device("cuda", 0)
    for row in measure_tails(dev, reps=args.steps * 10):
        print(json.dumps(row), flush=True)
    # a plain copy of known size in the same process: the scale of the HBM
    # traffic counters (FETCH_SIZE / WRITE_SIZE) for the tails' summaries
    x = torch.ones(64 * 1024 * 1024, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize(dev)
    print(json.dumps({"calibration_copy_bytes": x.numel() * 4}), flush=True)


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------

def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_forwards(fn, reps, budget_s):
    """1 warm-up call, then `reps` timed calls (up to 9 while under
    budget_s): (median seconds, all times)."""
    fn()
    times, spent = [], 0.0
    while len(times) < reps or (spent < budget_s and len(times) < 9):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
    return statistics.median(times), times


def cpu_baseline(model, workload, T, batch, image, reps=3, budget_s=10.0):
    """The CPU oracle's network forward (oracle.sew_resnet_forward /
    spikformer_forward / vgg_forward in fp32: torch CPU conv, eval BN, the C
    LIF of SpikingJelly's multi-step recurrence) on this host's threads,
    1 warm-up forward then >= `reps` timed forwards of `batch` images,
    median.  Beside it, the same protocol for the eager SpikingJelly-
    equivalent model (catfuse_amd.snn modules: LIFNode's recurrence in torch)."""
    import copy
    import torch
    import oracle
    from catfuse_amd import snn
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    m = copy.deepcopy(model).cpu().eval()
    g = torch.Generator().manual_seed(1)
    img = torch.randn(batch, 3, image, image, generator=g)
    x = img.unsqueeze(0).expand(T, batch, 3, image, image)
    fwd = {"spikformer_8_384": oracle.spikformer_forward,
           "vgg11_bn": oracle.vgg_forward}.get(workload, oracle.sew_resnet_forward)
    with torch.no_grad():
        med, times = _median_forwards(lambda: fwd(m, x, conv_dtype=torch.float32), reps,
                                      budget_s)
        xc = x.contiguous()

        def eager():
            snn.functional.reset_net(m)
            m(xc)
        emed, etimes = _median_forwards(eager, reps, budget_s)
    sample = (f"batch {batch} of 3x{image}x{image} at T={T}: median of {{n}} forwards "
              f"({{lo:.2f}}-{{hi:.2f}} s each) after 1 warm-up forward")
    return {"value": round(batch / med, 3), "unit": "images/s", "cores": threads,
            "kind": "port", "cpu": cpu_model_name(),
            "sample": f"oracle {fwd.__name__} (fp32 torch CPU conv + eval BN + C LIF), "
                      + sample.format(n=len(times), lo=min(times), hi=max(times)),
            "eager_sj_equivalent": {
                "value": round(batch / emed, 3), "unit": "images/s", "cores": threads,
                "sample": "eager catfuse_amd.snn model (SpikingJelly-equivalent torch multi-step "
                          "path, fp32), " + sample.format(n=len(etimes), lo=min(etimes),
                                                          hi=max(etimes))}}


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def run_network(workload, args, dev, v_threshold=1.0, label=True):
    """Optimize the workload's model, time it; returns (res, stats, model,
    fused, x)."""
    import torch
    import catfuse_amd
    T, B, HW = args.T, args.batch, args.image
    model = build_model(workload, v_threshold=v_threshold)
    fused, stats = catfuse_amd.optimize(model, device=dev, T=T)
    fused.eval()
    g = torch.Generator(device=dev).manual_seed(0)
    img = torch.randn(B, 3, HW, HW, device=dev, generator=g)
    x = img.unsqueeze(0).expand(T, B, 3, HW, HW)      # direct encoding, resident in HBM
    res = time_forward(fused, x, img, args.steps, args.warmup, args.eager, label)
    return res, stats, model, fused, x


def sew_result(args, dev):
    res, stats, model, fused, x = run_network("sew_resnet18", args, dev)
    kern = res["timer"].summary()
    roof = conv_roofline(kern, args.steps, traffic=traffic_from_profiles())
    sz = staticzero_summary(kern, args.steps, launch_floor_us(dev))
    sz["conv_route_sequence"] = route_sequence(res["timer"], CONV_LAUNCHES, args.steps)
    result = _base_result(args, res, stats, "sew_resnet18_adds_T4_B32_224")
    result.update(roofline=roof, staticzero_convs=sz, per_layer=per_layer_table(res),
                  kernels=_per_kernel(kern, args.steps))
    if not args.no_live:
        result["live"] = live_result(args, dev)
    return result, model


def live_result(args, dev, workload="sew_resnet18"):
    """The workload's network with v_th = 0.1 (every layer active, the
    reference's end-to-end setting): the dense MFMA route at every layer's
    shape."""
    res, stats, model, fused, x = run_network(workload, args, dev,
                                              v_threshold=LIVE_V_THRESHOLD)
    frac, rates = liveness(fused, x, workload)
    kern = res["timer"].summary()
    roof = conv_roofline(kern, args.steps)
    rows = per_layer_table(res)
    mfma3 = [r for r in rows if r["kernel"] in CONV_LAUNCHES and r["route"] == "D"]
    return {"v_threshold": LIVE_V_THRESHOLD,
            "liveness": {"alive_fraction": round(frac, 4), "required": LIVE_MIN_FRACTION,
                         "ok": frac >= LIVE_MIN_FRACTION, "module_spike_rates": rates},
            "images_per_s": round(args.batch / (res["ms"] * 1e-3), 2),
            "ms_per_step": round(res["ms"], 4), "mode": res["mode"],
            "eager_ms_per_step": round(res["ms_eager"], 4),
            "roofline": roof,
            "conv_route_sequence": route_sequence(res["timer"], CONV_LAUNCHES, args.steps),
            "min_conv_frac": min((r["frac"] for r in mfma3), default=None),
            "per_layer": rows, "kernels": _per_kernel(kern, args.steps)}


def spikformer_result(args, dev):
    res, stats, model, fused, x = run_network("spikformer_8_384", args, dev)
    timer, steps = res["timer"], args.steps
    kern = timer.summary()
    roof = conv_roofline(kern, steps,
                         traffic=traffic_from_profiles("conv_halo_spikformer_8_384_traffic.json"))
    roof["kernel"] = ("conv_halo_kernel 3x3 (cf_conv_mfma: the SPS Conv-BN-LIF stages), "
                      "launches that run the MFMA K loop")
    roof["conv_route_sequence"] = route_sequence(timer, "conv_mfma", steps)
    l_ms, l_fl, _, l_n = _agg(kern, ["linear_tokens"])
    lz_ms, _, _, lz_n = _agg(kern, ["linear_tokens_staticzero"])
    a_ms, a_fl, a_b, a_n = _agg(kern, ["spike_attention"])
    az_ms, _, az_b, az_n = _agg(kern, ["spike_attention_staticzero"])
    az_el = kern.get("spike_attention_staticzero", {}).get("elided", 0)
    ach = l_fl / (l_ms * 1e-3) / 1e12 if l_ms else 0.0
    a_gbps = a_b / (a_ms * 1e-3) / 1e9 if a_ms else 0.0
    result = _base_result(args, res, stats, "spikformer_8_384_T4_B32_224")
    result["metric"] = "Spikformer-8-384 T=4 images/s on 1 MI355X (config C4)"
    result["config"].update(tokens=196, dim=384, heads=12, blocks=8)
    result["dtype"] = ("fp32 (linears/convs: fp16 hi/lo split weights x fp16-exact spikes on "
                       "MFMA, fp32 acc; attention: exact integer Q(K^T V), one fp32 rounding)")
    result.update(roofline=roof, staticzero_convs=staticzero_summary(kern, steps),
                  per_layer=per_layer_table(res), kernels=_per_kernel(kern, steps))
    result["token_linears"] = {
        "kernel": "conv_halo_kernel 1x1 (cf_conv_mfma: fused Linear-BN1d-LIF over the token rows)",
        "launches_per_step": (l_n + lz_n) // steps,
        "mfma_route": {"launches_per_step": l_n // steps,
                       "us_per_launch_avg": round(l_ms * 1e3 / max(1, l_n), 2),
                       "achieved": round(ach, 2), "unit": "TFLOP/s"},
        "staticzero_route": {"launches_per_step": lz_n // steps,
                             "us_per_launch_avg": round(lz_ms * 1e3 / max(1, lz_n), 2)},
        "linear_route_sequence": route_sequence(timer, "linear_tokens", steps)}
    result["attention"] = {"kernel": "spike_attention_kernel (cf_spike_attention_lif)",
                           "launches_per_step": (a_n + az_n) // steps,
                           "full_route": {"launches_per_step": a_n // steps,
                                          "us_per_launch_avg": round(a_ms * 1e3 / max(1, a_n), 2),
                                          "achieved": round(a_gbps, 1), "peak": PEAK_HBM_GBPS,
                                          "unit": "GB/s",
                                          "frac": round(a_gbps / PEAK_HBM_GBPS, 4)},
                           "zero_route": {"launches_per_step": az_n // steps,
                                          "elided_per_step": az_el // steps,
                                          "bytes_per_step": az_b // steps,
                                          "us_per_launch_avg": round(az_ms * 1e3 / max(1, az_n), 2)}}
    return result, model


def vgg_result(args, dev):
    """Config C2 (reference: benchmarks/bench_vgg11_e2e.py:54-72,277-290):
    the convs, the in-network AvgPool->LIF tails and the Linear->LIF head."""
    res, stats, model, fused, x = run_network("vgg11_bn", args, dev)
    timer, steps = res["timer"], args.steps
    kern = timer.summary()
    result = _base_result(args, res, stats, "spiking_vgg11_bn_T4_B64_32")
    result["metric"] = "Spiking VGG-11-BN T=4 images/s on 1 MI355X (config C2)"
    roof = conv_roofline(kern, steps)
    pool_ms, _, pool_b, pool_n = _agg(kern, ["avgpool2x2_lif"])
    result.update(roofline=roof, per_layer=per_layer_table(res),
                  kernels=_per_kernel(kern, steps))
    gb = pool_b / (pool_ms * 1e-3) / 1e9 if pool_ms else 0.0
    result["avgpool_lif_tails"] = {"kernel": "avgpool2_lif_kernel (cf_avgpool2x2_lif)",
                                   "launches_per_step": pool_n // steps,
                                   "us_per_launch_avg": round(pool_ms * 1e3 / max(1, pool_n), 2),
                                   "achieved": round(gb, 1), "peak": PEAK_HBM_GBPS,
                                   "unit": "GB/s", "frac": round(gb / PEAK_HBM_GBPS, 4)}
    if not args.no_live:
        result["live"] = live_result(args, dev, "vgg11_bn")
    return result, model


def _per_kernel(kern, steps):
    return {k: {"launches_per_step": v["launches"] // steps,
                "ms_per_step": round(v["ms_total"] / steps, 4)} for k, v in kern.items()}


def _base_result(args, res, stats, workload):
    ips = args.batch / (res["ms"] * 1e-3)
    return {
        "metric": METRIC, "value": round(ips, 2), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["ms"], 4),
        "mode": res["mode"], "eager_ms_per_step": round(res["ms_eager"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (conv: fp16 hi/lo split weights x fp16-exact spikes on MFMA, fp32 acc)",
        "data": "synthetic (seeded N(0,1) images, resident in HBM, random kaiming weights, config BN stats)",
        "config": {"workload": workload, "T": args.T, "batch": args.batch,
                   "image": [3, args.image, args.image],
                   "spike_copy": getattr(args, "spike_copy", "f16"),
                   "encoding": "direct (input repeated over T)",
                   "fused_lif_nodes": stats["fused_lif_nodes"],
                   "total_lif_nodes": stats["total_lif_nodes"]},
    }


# ---------------------------------------------------------------------------
# SparseFlow / dense crossover (the MI355X routing threshold)
# ---------------------------------------------------------------------------

XO_RATES = (0.0, 0.001, 0.01, 0.05, 0.1, 0.2, 0.3, 0.5)
XO_PATTERNS = ("iid", "block", "spatial", "chgroup", "region")
XO_ROUTES = ("SparseFlow", "SparseFlow-linear", "SF+EGD", "StreamFuse", "DenseKeep", "auto")


def xo_input(rate, pattern, shape=(4, 32, 256, 14, 14), seed=0, block=8, p_zero_block=0.7):
    """fp32 CPU spikes [T, B, C, H, W] of one rate and spatial pattern:
    iid Bernoulli(rate); block: per (t, b, c) and 8x8 block, zero with
    probability 0.7, else Bernoulli(rate) (the granularity of the
    reference's tests/test_70_oracle_gap.py:112-124); spatial: per (t, b)
    and 8x8 block, zero in every channel with probability 0.7; chgroup:
    per image and 16-channel group, silent at every step and pixel with
    probability 0.7 (dead channel groups); region: per image, activity only
    inside one random window of half the height and width (a quarter of the
    area), at every step."""
    import torch
    g = torch.Generator().manual_seed(seed)
    T, B, C, H, W = shape
    x = (torch.rand(shape, generator=g) < rate).float()
    if pattern in ("block", "spatial"):
        gh, gw = -(-H // block), -(-W // block)
        kc = C if pattern == "block" else 1
        keep = (torch.rand((T, B, kc, gh, gw), generator=g) >= p_zero_block).float()
        keep = keep.repeat_interleave(block, 3).repeat_interleave(block, 4)[..., :H, :W]
        x = x * keep
    elif pattern == "chgroup":
        ng = -(-C // 16)
        keep = (torch.rand((1, B, ng, 1, 1), generator=g) >= p_zero_block).float()
        x = x * keep.repeat_interleave(16, 2)[:, :, :C]
    elif pattern == "region":
        keep = torch.zeros((1, B, 1, H, W))
        hh, hw = max(1, H // 2), max(1, W // 2)
        for b in range(B):
            r0 = int(torch.randint(0, H - hh + 1, (1,), generator=g))
            c0 = int(torch.randint(0, W - hw + 1, (1,), generator=g))
            keep[0, b, 0, r0:r0 + hh, c0:c0 + hw] = 1.0
        x = x * keep
    elif pattern != "iid":
        raise ValueError(f"unknown pattern {pattern!r}")
    return x


def xo_as_fused_output(x):
    """x (GPU fp32 spikes) as a fused conv's output: an NHWC-backed tensor
    with the fp16 copy and a count block holding count_nonzero(x)."""
    import torch
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


def _xo_layer(C_in, C_out, device, seed=0, k=3, stride=1):
    import torch
    from catfuse_amd.implementations.base import ConvLIFParams, ConvLIFSpec
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(C_out, C_in, k, k, generator=g) * (2.0 / (C_in * k * k)) ** 0.5
    mean = torch.randn(C_out, generator=g) * 0.1
    var = torch.rand(C_out, generator=g) + 0.5
    gamma = torch.rand(C_out, generator=g) * 0.4 + 0.8
    beta = torch.randn(C_out, generator=g) * 0.1
    scale = gamma / torch.sqrt(var + 1e-5)
    shift = beta - mean * scale
    spec = ConvLIFSpec(C_in, C_out, k, stride, k // 2, has_conv_bias=False, has_bn=True, tau=2.0,
                       v_threshold=1.0, v_reset=0.0, decay_input=True)
    return spec, ConvLIFParams(w.to(device), None, scale.to(device), shift.to(device))


def _xo_time_graph(fn, calls, reps, device):
    """Median microseconds per call over `reps` replays of a graph of
    `calls` calls."""
    import torch
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


def xo_sweep(device, rates=XO_RATES, patterns=XO_PATTERNS, shape=(4, 32, 256, 14, 14),
             plain=False, calls=20, reps=5, seed=0, k=3, stride=1, c_out=None):
    """One row per (pattern, rate): the input density and the microseconds
    per call of every route (each checked bitwise against the others) of a
    k x k / stride conv of shape's input (c_out output channels, default
    the input's)."""
    import torch
    from catfuse_amd.implementations.dense_keep import DenseKeep
    from catfuse_amd.implementations.sparse_flow import SparseFlow
    from catfuse_amd.implementations.stream_fuse import StreamFuse
    from catfuse_amd.state import StateBuffer
    T, B, C, H, W = shape
    spec, params = _xo_layer(C, c_out or C, device, seed, k=k, stride=stride)
    impls = {"SparseFlow": SparseFlow(sparsity_threshold=-1.0, egd=False),
             "SparseFlow-linear": SparseFlow(sparsity_threshold=-1.0, compact_tiles=False,
                                             egd=False),
             "SF+EGD": SparseFlow(sparsity_threshold=-1.0),
             "StreamFuse": StreamFuse(), "DenseKeep": DenseKeep(), "auto": SparseFlow()}
    rows = []
    with torch.no_grad():
        for pattern in patterns:
            for rate in rates:
                xc = xo_input(rate, pattern, shape, seed=seed + 1)
                xd = xc.to(device)
                x = xd if plain else xo_as_fused_output(xd)
                row = {"pattern": pattern, "rate": rate, "k": k, "stride": stride,
                       "shape": list(shape), "c_out": spec.out_channels,
                       "density": float(torch.count_nonzero(xc)) / xc.numel()}
                ref = None
                for name in XO_ROUTES:
                    impl = impls[name]

                    def call(impl=impl):
                        return impl.forward(x, spec, params, StateBuffer())
                    y = call()
                    if name == "SparseFlow":
                        row.update(xo_score(impl, spec, T, H, W))
                    if ref is None:
                        ref = y.clone()
                    elif not torch.equal(y, ref):
                        raise RuntimeError(f"{name} differs from SparseFlow at {pattern} {rate}")
                    row[name] = _xo_time_graph(call, calls, reps, device)
                rows.append(row)
                print(json.dumps(row), file=sys.stderr, flush=True)
    return rows


_POPCOUNT8 = None


def xo_score(impl, spec, T, H, W):
    """Dispatch score of the SparseFlow launch just run, as cf_compact_tiles
    computes it (the reference's catfuse/sparseflow/dispatch.py:868-935 over
    the tile's time steps): R = 1 - AGR of the tile masks OR-ed over the
    steps, I = dense MACs per image / tiles per image, S = R * I."""
    import torch
    global _POPCOUNT8
    _tc, ag = impl.last_tiles()
    if _POPCOUNT8 is None or _POPCOUNT8.device != ag.device:
        _POPCOUNT8 = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int64,
                                  device=ag.device)
    geo = impl.geometry(spec, H, W)
    G = -(-spec.in_channels // geo["group_size"])
    Ho, Wo = spec.output_hw(H, W)
    GH, GW = -(-Ho // geo["block_h"]), -(-Wo // geo["block_w"])
    steps = ag.view(T, -1)
    m = steps[0].clone()
    for t in range(1, T):
        m |= steps[t]
    pop = int(_POPCOUNT8[m.contiguous().view(torch.uint8).long()].sum())
    R = 1.0 - pop / (m.numel() * G)
    I = Ho * Wo * spec.out_channels * spec.in_channels * spec.kernel_size ** 2 / (GH * GW)
    return {"R": R, "I": I, "S": R * I}


def xo_egd_fit(rows):
    """The dispatch-score threshold tau that best separates the measured
    rows (nonzero inputs) where forced SparseFlow beat the best dense route
    from those where it did not: tau minimising the misclassified rows
    (SparseFlow iff S > tau, R >= r_min), with the misclassification count;
    tau is the midpoint between the scores on either side of it."""
    pts = sorted((r["S"], r["SparseFlow"] < min(r["StreamFuse"], r["DenseKeep"]))
                 for r in rows if r["density"] > 0.0 and "S" in r)
    if not pts:
        return None, 0
    best = (len(pts) + 1, None)
    cands = [pts[0][0] - 1.0] + [(a[0] + b[0]) / 2 for a, b in zip(pts, pts[1:])] + [pts[-1][0]]
    for tau in cands:
        err = sum((s > tau) != win for s, win in pts)
        if err < best[0]:
            best = (err, tau)
    return best[1], best[0]


def xo_rmin_fit(rows):
    """The silent-group fraction R_min that best separates the measured rows
    (nonzero inputs) where forced SparseFlow beat the best dense route from
    those where it did not (SparseFlow iff R >= R_min): the midpoint of the
    widest interval of thresholds with the fewest misclassified rows, and
    that count."""
    pts = sorted((r["R"], r["SparseFlow"] < min(r["StreamFuse"], r["DenseKeep"]))
                 for r in rows if r["density"] > 0.0 and "R" in r)
    if not pts:
        return None, 0
    edges = [0.0] + sorted({p[0] for p in pts}) + [1.0 + 1e-9]
    best = None
    for lo, hi in zip(edges, edges[1:]):
        thr = (lo + hi) / 2 if lo < hi else lo
        err = sum((R >= thr) != win for R, win in pts)
        key = (err, -(hi - lo))
        if best is None or key < best[0]:
            best = (key, thr)
    return best[1], best[0][0]


def xo_crossover(rows):
    """Per pattern, the lowest input sparsity at which forced SparseFlow
    (compacted tile order) is faster than the best dense route (None: at no
    measured nonzero rate)."""
    out = {}
    for pattern in sorted({r["pattern"] for r in rows}):
        wins = [1.0 - r["density"] for r in rows
                if r["pattern"] == pattern and r["density"] > 0.0
                and r["SparseFlow"] < min(r["StreamFuse"], r["DenseKeep"])]
        out[pattern] = min(wins) if wins else None
    return out


def xo_table(rows):
    lines = ["| pattern | rate | density | R | S | "
             + " | ".join(f"{n} (us)" for n in XO_ROUTES) + " |",
             "|---|---|---|---|---|" + "---|" * len(XO_ROUTES)]
    for r in rows:
        lines.append(f"| {r['pattern']} | {r['rate']:g} | {r['density']:.4f} | "
                     f"{r.get('R', float('nan')):.3f} | {r.get('S', float('nan')):.3g} | "
                     + " | ".join(f"{r[n]:.1f}" for n in XO_ROUTES) + " |")
    return "\n".join(lines)


def sf_crossover_main(args):
    import torch
    dev = torch.device("cuda", 0)
    shape = tuple(args.xo_shape)
    rows = xo_sweep(dev, shape=shape, plain=args.xo_plain, k=args.xo_kernel,
                    stride=args.xo_stride, c_out=args.xo_cout,
                    patterns=tuple(args.xo_patterns.split(",")))
    print(xo_table(rows))
    print("crossover (lowest input sparsity where SparseFlow wins):", xo_crossover(rows))
    n = sum(r["density"] > 0 for r in rows)
    tau, err = xo_egd_fit(rows)
    print(f"dispatch score fit: tau = {tau:.4g} ({err} misclassified of {n})"
          if tau is not None else "no score")
    r_min, err = xo_rmin_fit(rows)
    print(f"silent-group fraction fit: R_min = {r_min:.3f} ({err} misclassified of {n})"
          if r_min is not None else "no score")
    print("rows:", json.dumps(rows))


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--image", type=int, default=None)
    ap.add_argument("--T", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-tails", action="store_true")
    ap.add_argument("--no-live", action="store_true")
    ap.add_argument("--live-only", action="store_true",
                    help="only the live SEW line (v_th = 0.1), printed as its own JSON line "
                         "(the command of its rocprofv3 summary)")
    ap.add_argument("--cpu-batch", type=int, default=None,
                    help="images per CPU-baseline forward (default: CPU_BATCH[workload])")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of the captured HIP graph")
    ap.add_argument("--workload", default="sew_resnet18",
                    choices=list(WORKLOADS) + ["sf_crossover", "lif_tails"])
    ap.add_argument("--spike-copy", default="f16", choices=["f16", "u8"],
                    help="element of the NHWC spike copies between fused layers (one byte "
                         "per channel with u8; results are the same bit for bit)")
    ap.add_argument("--xo-shape", type=int, nargs=5, default=[4, 32, 256, 14, 14])
    ap.add_argument("--xo-kernel", type=int, default=3, choices=[1, 3])
    ap.add_argument("--xo-stride", type=int, default=1, choices=[1, 2])
    ap.add_argument("--xo-cout", type=int, default=None)
    ap.add_argument("--xo-patterns", default=",".join(XO_PATTERNS))
    ap.add_argument("--xo-plain", action="store_true",
                    help="crossover inputs as fp32 tensors (the layer packs them)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every GPU box in this setup has a single "
              "MI355X; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.workload == "lif_tails":
        tails_main(args)
        return
    if args.workload == "sf_crossover":
        sf_crossover_main(args)
        return
    for k, v in WORKLOADS[args.workload].items():
        if getattr(args, k) is None:
            setattr(args, k, v)

    import torch
    import catfuse_amd
    catfuse_amd.set_spike_copy(args.spike_copy)
    dev = torch.device("cuda", 0)
    if args.live_only:
        line = live_result(args, dev, args.workload)
        line["spike_copy"] = args.spike_copy
        print(json.dumps(line), flush=True)
        return
    if args.workload == "spikformer_8_384":
        result, model = spikformer_result(args, dev)
    elif args.workload == "vgg11_bn":
        result, model = vgg_result(args, dev)
    else:
        result, model = sew_result(args, dev)
    if not args.no_tails and args.workload == "sew_resnet18":
        result["lif_tails"] = measure_tails(dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, args.workload, args.T,
                                              args.cpu_batch or CPU_BATCH[args.workload],
                                              args.image)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
