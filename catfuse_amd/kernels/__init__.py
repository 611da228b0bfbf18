"""Functional fused-kernel API (mirrors catfuse/kernels/__init__.py and the
standalone tails in catfuse/kernels/*.py).

  partial_fusion_conv_lif(x, w, tau, v_th, v_reset, stride, padding, K_block)
  partial_fusion_conv_bn_lif(x, w_conv, bn_weight, bn_bias, running_mean,
                             running_var, eps, tau, v_th, v_reset, stride,
                             padding, K_block)
  partial_fusion_conv_bn_add_lif(x, identity, w_conv, bn_weight, bn_bias,
                                 running_mean, running_var, eps, tau, v_th,
                                 v_reset, stride, padding)
  add_lif(x1, x2, v_carry=None, ...), add_bn_lif(a, x, scale, bias, ...),
  avgpool_lif(x, v_carry=None, ...), linear_lif(x, w, bias=None, ...)

Each call starts from the initial membrane state (v = v_reset), like the
reference's single-block (K = T) launchers, unless a carry tensor is given;
the `*_lif` tails return (spikes, v_final).  Packed weights are cached by
tensor identity and version.
"""
from __future__ import annotations

import torch

from catfuse_amd.runtime import ID_ADD_Z, ConvLIFRunner, avgpool2x2_lif, lif_multistep

_RUNNERS: dict = {}


def _runner(w, scale, shift, bias, stride, padding, tau, v_th, v_reset, decay_input=True):
    key = tuple((id(t), t._version) if t is not None else None for t in (w, scale, shift, bias)) + \
        (stride, padding, tau, v_th, v_reset, decay_input)
    r = _RUNNERS.get(key)
    if r is None:
        if len(_RUNNERS) > 64:
            _RUNNERS.clear()
        r = ConvLIFRunner(w, scale, shift, bias, stride, padding, tau, v_th, v_reset, decay_input)
        r._keep = (w, scale, shift, bias)
        _RUNNERS[key] = r
    return r


def _fold(bn_weight, bn_bias, running_mean, running_var, eps):
    inv = 1.0 / torch.sqrt(running_var.float() + eps)
    scale = bn_weight.float() * inv
    return scale.contiguous(), (bn_bias.float() - running_mean.float() * scale).contiguous()


def _conv(x, r):
    if not bool((x.half().float() == x).all().item()):
        return r.run_direct(x, want_v_out=False)[0]
    return r.run_mfma(x.contiguous(), want_v_out=False)[0]


def partial_fusion_conv_lif(x, w, tau=2.0, v_th=1.0, v_reset=0.0, stride=1, padding=1,
                            K_block=None):
    """Conv -> LIF over [T, B, C_in, H, W]; returns spikes."""
    return _conv(x, _runner(w.float().contiguous(), None, None, None, stride, padding, tau, v_th,
                            v_reset))


def partial_fusion_conv_bn_lif(x, w_conv, bn_weight, bn_bias, running_mean, running_var,
                               eps=1e-5, tau=2.0, v_th=1.0, v_reset=0.0, stride=1, padding=1,
                               K_block=None):
    """Conv -> eval BN -> LIF; returns spikes."""
    sc, sh = _fold(bn_weight, bn_bias, running_mean, running_var, eps)
    return _conv(x, _runner(w_conv.float().contiguous(), sc, sh, None, stride, padding, tau,
                            v_th, v_reset))


def partial_fusion_conv_bn_add_lif(x, identity, w_conv, bn_weight, bn_bias, running_mean,
                                   running_var, eps=1e-5, tau=2.0, v_th=1.0, v_reset=0.0,
                                   stride=1, padding=1):
    """Conv -> eval BN -> (+ identity) -> LIF; returns spikes."""
    sc, sh = _fold(bn_weight, bn_bias, running_mean, running_var, eps)
    r = _runner(w_conv.float().contiguous(), sc, sh, None, stride, padding, tau, v_th, v_reset)
    return r.run_mfma(x.contiguous(), identity=identity.contiguous(), identity_mode=ID_ADD_Z,
                      want_v_out=False)[0]


def add_lif(x1, x2, v_carry=None, tau=2.0, v_th=1.0, v_reset=0.0, decay_input=True):
    """x1 + x2 -> LIF over [T, ...]; returns (spikes, v_final)."""
    return lif_multistep(x1.contiguous(), v_carry, mode=3, z2=x2.contiguous(), tau=tau,
                         v_threshold=v_th, v_reset=v_reset, decay_input=decay_input)


def add_bn_lif(a, x, scale, bias, v_carry=None, tau=2.0, v_th=1.0, v_reset=0.0,
               decay_input=True):
    """(a + x) * scale[c] + bias[c] -> LIF over [T, B, C, H, W]."""
    C = a.shape[2]
    hw = a[0, 0, 0].numel()
    return lif_multistep(a.contiguous(), v_carry, mode=4, z2=x.contiguous(),
                         scale=scale.float().contiguous(), shift=bias.float().contiguous(),
                         channels=C, hw=hw, tau=tau, v_threshold=v_th, v_reset=v_reset,
                         decay_input=decay_input)


def bn_lif(z, scale, bias, v_carry=None, tau=2.0, v_th=1.0, v_reset=0.0, decay_input=True):
    """z * scale[c] + bias[c] -> LIF over [T, B, C, H, W]."""
    C = z.shape[2]
    hw = z[0, 0, 0].numel()
    return lif_multistep(z.contiguous(), v_carry, mode=1, scale=scale.float().contiguous(),
                         shift=bias.float().contiguous(), channels=C, hw=hw, tau=tau,
                         v_threshold=v_th, v_reset=v_reset, decay_input=decay_input)


def avgpool_lif(x, v_carry=None, tau=2.0, v_th=1.0, v_reset=0.0, decay_input=True):
    """AvgPool2d(2, 2) -> LIF over [T, B, C, H, W]; returns (spikes, v_final)."""
    return avgpool2x2_lif(x.contiguous(), v_carry, tau=tau, v_threshold=v_th, v_reset=v_reset,
                          decay_input=decay_input)


def linear_lif(x, w, bias=None, v_carry=None, tau=2.0, v_th=1.0, v_reset=0.0, decay_input=True):
    """x [T, B, I] @ w[O, I]^T (+ bias) -> LIF; returns (spikes [T, B, O], v_final [B, O])."""
    T, B, I = x.shape
    O = w.shape[0]
    r = _runner(w.float().contiguous().view(O, I, 1, 1), None, None,
                None if bias is None else bias.float().contiguous(), 1, 0, tau, v_th, v_reset,
                decay_input)
    x5 = x.contiguous().view(T, B, I, 1, 1)
    v_in = None if v_carry is None else v_carry.contiguous().view(B, O, 1, 1)
    if not bool((x.half().float() == x).all().item()):
        s, v = r.run_direct(x5, v_in)
    else:
        s, v = r.run_mfma(x5, v_in)
    return s.view(T, B, O), v.view(B, O)


__all__ = ["partial_fusion_conv_lif", "partial_fusion_conv_bn_lif",
           "partial_fusion_conv_bn_add_lif", "add_lif", "add_bn_lif", "bn_lif", "avgpool_lif",
           "linear_lif"]
