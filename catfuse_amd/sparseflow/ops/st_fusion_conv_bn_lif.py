"""STFusionConvBNLIF — spatio-temporal fused Conv -> BN -> LIF with the
SparseFlow spatial backend (mirrors
catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:91-565).

Routing.  The reference counts nonzeros on the host every call
(`count_nonzero().item()`, :512-514) and picks StaticZero (nnz == 0),
SparseFlow (sparsity > 0.7) or DenseKeep.  Here the same decision, with the
same double-precision formula, is taken on the device inside the SparseFlow
implementation (routing="device", default): the forward never synchronises
and can be captured in a HIP graph.  routing="host" reproduces the
reference's host-side decision and dispatches to a separate dense
implementation.  All routes are bit-identical.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from catfuse_amd.hardware import runtime_profile
from catfuse_amd.implementations import ConvLIFParams, ConvLIFSpec, DenseKeep, SparseFlow, StreamFuse
from catfuse_amd.patterns import CTFPattern, conv_geometry, lif_params
from catfuse_amd.runtime import ID_ADD_SPIKE
from catfuse_amd.state import StateBuffer


def _fold_bn_params(bn: nn.BatchNorm2d):
    """Eval BN as an affine: scale = gamma / sqrt(var + eps),
    offset = beta - mean * scale."""
    inv_std = 1.0 / torch.sqrt(bn.running_var + bn.eps)
    scale = inv_std if bn.weight is None else bn.weight * inv_std
    offset = -bn.running_mean * scale if bn.bias is None else bn.bias - bn.running_mean * scale
    return scale.detach(), offset.detach()


class STFusionConvBNLIF(CTFPattern):
    policy_row = "STFusionConvBNLIF"

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int = 3,
                 stride: int = 1, padding: int = 1, bias: bool = True,
                 bn_scale: Optional[torch.Tensor] = None, bn_bias: Optional[torch.Tensor] = None,
                 tau: float = 2.0, v_threshold: float = 1.0, v_reset: Optional[float] = 0.0,
                 decay_input: bool = True, K: int = 4, threshold: float = 1e-6,
                 routing: str = "device", sparsity_threshold: Optional[float] = None):
        super().__init__()
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = int(kernel_size), int(stride), int(padding)
        self.K = int(K)
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = v_reset
        self.decay_input = bool(decay_input)
        self.threshold = float(threshold)
        if routing not in ("device", "host"):
            raise ValueError("routing must be 'device' or 'host'")
        self.routing = routing
        self.weight = nn.Parameter(torch.empty(out_channels, in_channels, kernel_size, kernel_size))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_channels))
        else:
            self.register_parameter("bias", None)
        if bn_scale is not None:
            self.register_buffer("bn_scale", bn_scale.clone())
            self.register_buffer("bn_bias_folded", bn_bias.clone())
        else:
            self.register_buffer("bn_scale", None)
            self.register_buffer("bn_bias_folded", None)
        self.state = StateBuffer()
        self._register_state(self.state)
        self.spec = ConvLIFSpec(self.in_channels, self.out_channels, self.kernel_size, self.stride,
                                self.padding, has_conv_bias=bool(bias),
                                has_bn=bn_scale is not None, tau=self.tau,
                                v_threshold=self.v_threshold, v_reset=v_reset,
                                decay_input=self.decay_input)
        prof = runtime_profile()
        self._impl_dense = DenseKeep() if prof.dense_impl == "DenseKeep" else StreamFuse()
        # sparsity above which the SparseFlow route is taken: the profile's
        # measured value unless given (0.7 reproduces the reference's routing)
        self._impl_sparse = SparseFlow(sparsity_threshold)
        self._params = None
        self._params_key = None
        self.route_counts = {"StaticZero": 0, "SparseFlow": 0, "DenseKeep": 0}

    def _ensure_params(self) -> ConvLIFParams:
        P, B = self._parameters, self._buffers
        key = (id(P["weight"]), id(P.get("bias")), id(B.get("bn_scale")),
               id(B.get("bn_bias_folded")))
        if self._params_key != key or self._params is None:
            self._params = ConvLIFParams(self.weight, self.bias, self.bn_scale,
                                         self.bn_bias_folded)
            self._params_key = key
        return self._params

    def supports_sew_identity(self):
        return True

    def forward(self, x: torch.Tensor, sew_identity: Optional[torch.Tensor] = None):
        squeeze = x.ndim == 4
        if squeeze:
            x = x.unsqueeze(0)
        params = self._ensure_params()
        if self.routing == "host":
            nnz = int(x.count_nonzero().item())
            sparsity = 1.0 - nnz / x.numel()
            if nnz == 0 or sparsity > self._impl_sparse.sparsity_threshold:
                self.route_counts["StaticZero" if nnz == 0 else "SparseFlow"] += 1
                impl = self._impl_sparse
            else:
                self.route_counts["DenseKeep"] += 1
                impl = self._impl_dense
        else:
            impl = self._impl_sparse
        if sew_identity is not None:
            if isinstance(impl, DenseKeep):
                y = sew_identity + impl.forward(x, self.spec, params, self.state)
            else:
                y = self._forward_identity(impl, x, params, sew_identity)
        else:
            y = impl.forward(x, self.spec, params, self.state)
        return y.squeeze(0) if squeeze else y

    def _forward_identity(self, impl, x, params, identity):
        if isinstance(impl, SparseFlow):
            _, B, _, H, W = x.shape
            dev = x.device
            Ho, Wo = self.spec.output_hw(H, W)
            r = impl.runner(self.spec, params, dev)
            v_in = self.state.peek((B, self.out_channels, Ho, Wo), dev)
            if impl.input_is_analog(x):
                spikes, v_out = r.run_direct(x, v_in)
                spikes = identity + spikes
            else:
                sparse = impl.route_geometry(self.spec, H, W)
                spikes, v_out = r.run_mfma(x.contiguous(), v_in, identity=identity.contiguous(),
                                           identity_mode=ID_ADD_SPIKE, sparse=sparse,
                                           sparse_threshold=impl.sparsity_threshold)
            self.state.set(v_out)
            return spikes
        return impl.forward(x, self.spec, params, self.state, identity=identity.contiguous(),
                            identity_mode=ID_ADD_SPIKE)

    def forward_with_k(self, x, K=None):
        return self._impl_sparse.forward_with_k(x, self.spec, self._ensure_params(), self.state, K)

    def last_route(self) -> int:
        """Device route of the last forward (0 StaticZero, 1 SparseFlow, 2
        DenseKeep); synchronises."""
        return self._impl_sparse.last_route()

    @classmethod
    def from_sj_modules(cls, conv: nn.Conv2d, bn: nn.BatchNorm2d, lif, K: int = 4,
                        threshold: float = 1e-6, routing: str = "device",
                        sparsity_threshold: Optional[float] = None):
        k, s, p = conv_geometry(conv)
        bn.eval()
        scale, offset = _fold_bn_params(bn)
        lp = lif_params(lif)
        m = cls(conv.in_channels, conv.out_channels, k, s, p, bias=conv.bias is not None,
                bn_scale=scale, bn_bias=offset, K=K, threshold=threshold, routing=routing,
                sparsity_threshold=sparsity_threshold, **lp)
        with torch.no_grad():
            m.weight.copy_(conv.weight)
            if conv.bias is not None:
                m.bias.copy_(conv.bias)
        return m.to(conv.weight.device)

    def extra_repr(self):
        s = f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, K={self.K}"
        if self.bn_scale is not None:
            s += ", bn=folded"
        return s + f", tau={self.tau}, v_th={self.v_threshold}, routing={self.routing}"
