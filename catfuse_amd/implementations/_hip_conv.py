"""Shared plumbing of the gfx950 Conv->(BN)->LIF implementations.

Owns the per-layer `ConvLIFRunner` (packed weights + workspaces) keyed by
the identity of the parameter tensors, and decides the input domain once
per layer: inputs exactly representable in fp16 (spikes, SEW sums, pooled
spikes) take the MFMA path; anything else (an analog image) takes the fp32
direct-convolution path.  The decision costs one host synchronisation on the
first forward of the layer; afterwards the pack kernel keeps OR-ing a sticky
device status bit if an input ever stops being fp16-exact, which
`catfuse_amd.check_status()` turns into an error.
"""
from __future__ import annotations

import torch

from catfuse_amd.implementations.base import Implementation
from catfuse_amd.runtime import ConvLIFRunner


class HipConvImplementation(Implementation):
    def __init__(self):
        super().__init__()
        self._runner = None
        self._runner_key = None
        self._exact_input = None

    def reset_caches(self) -> None:
        self._runner = None
        self._runner_key = None

    def runner(self, spec, params, device) -> ConvLIFRunner:
        key = (id(params.weight), id(params.bias), id(params.bn_scale), id(params.bn_bias),
               device if type(device) is torch.device else torch.device(device))
        if self._runner_key != key:
            self._runner = ConvLIFRunner(
                params.weight,
                params.bn_scale if spec.has_bn else None,
                params.bn_bias if spec.has_bn else None,
                params.bias if spec.has_conv_bias else None,
                spec.stride, spec.padding, spec.tau, spec.v_threshold, spec.v_reset,
                spec.decay_input)
            self._runner_key = key
        return self._runner

    def input_is_analog(self, x: torch.Tensor) -> bool:
        if self._exact_input is None:
            self._exact_input = bool((x.half().float() == x).all().item())
        return not self._exact_input

    @staticmethod
    def check_input(x: torch.Tensor, spec) -> None:
        if x.dim() != 5:
            raise ValueError(f"expected [T, B, C, H, W], got {tuple(x.shape)}")
        if not x.is_cuda or x.dtype != torch.float32:
            raise RuntimeError("catfuse_amd fused patterns take float32 GPU tensors "
                               "(there is no CPU path)")
        if x.shape[2] != spec.in_channels:
            raise ValueError(f"expected {spec.in_channels} channels, got {x.shape[2]}")
