"""catfuse_amd — MI355X-native CATFuse-SF: spatio-temporal fused SNN inference.

Drop-in surface of the reference package `catfuse` (hpcyhr/CATFuse):
``optimize(model, device, policy, T, use_sparseflow) -> (model, stats)``,
``substitute``, ``substitute_sf``, the pattern modules, ``StateBuffer``,
the ``Implementation`` plug-in point, ``policy`` and ``hardware``.  All
tensor math of the fused patterns runs in hand-written gfx950 HIP kernels
behind the C-ABI in include/catfuse_amd.h (library: catfuse_amd/_lib).
"""
from __future__ import annotations

__version__ = "0.1.0"


def optimize(model, device="cuda:0", policy=None, T=16, use_sparseflow=True,
             fuse_sew_add=True, fuse_stem=True, fuse_head=True):
    """Substitute the SpikingJelly model's fusible subgraphs with gfx950
    patterns.  `policy` may be a HardwareProfile for the static routing
    table (default: the reference's V100 table shape); `device`, when not
    None, is where the fused model is placed.  `fuse_stem` also folds a
    ResNet stem's MaxPool2d(3, 2, 1) into its Conv-BN-LIF kernel; `fuse_head`
    lets a global average pool read the last fused conv's fp16 NHWC copy."""
    from catfuse_amd.substitute import substitute, substitute_sf
    if use_sparseflow:
        fused, stats = substitute_sf(model, T=T, fuse_sew_add=fuse_sew_add, hwprof=policy,
                                     fuse_stem=fuse_stem, fuse_head=fuse_head)
    else:
        fused, stats = substitute(model)
    if device is not None:
        import torch
        if torch.cuda.is_available():
            fused = fused.to(device)
    return fused, stats


def check_status(device=None) -> None:
    """Raise if any fused layer received an input that its fp16 MFMA path
    could not represent exactly (sticky device flag; synchronises)."""
    from catfuse_amd import runtime
    st = runtime.read_status(device)
    if st & runtime.STATUS_INEXACT_FP16:
        raise RuntimeError("catfuse_amd: a fused layer on the fp16 MFMA path received inputs "
                           "that are not exactly representable in fp16")
    if st & runtime.STATUS_FP16_RANGE:
        raise RuntimeError("catfuse_amd: the fused stem received image values outside the "
                           "fp16 range (|x| > 65504 or not finite)")


def set_spike_copy(fmt: str) -> None:
    """Element of the NHWC spike copies the fused layers exchange: "f16"
    (two bytes per channel) or "u8" (one byte: the values are integers
    0..255).  Layers launched afterwards produce copies in that format;
    results are bit for bit the same in both."""
    from catfuse_amd import runtime
    runtime.set_spike_copy(fmt)


def capture(model, example, reset=True, warmup=2):
    """HIP-graph replay of ``reset_net(model); model(example)`` (see
    catfuse_amd.graph): returns a callable that copies its input into the
    captured input buffer and replays the whole fused forward."""
    from catfuse_amd import graph
    return graph.capture(model, example, reset=reset, warmup=warmup)


__all__ = ["optimize", "check_status", "capture", "set_spike_copy", "__version__"]
