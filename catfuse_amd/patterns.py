"""Fused pattern modules (drop-in replacements for SpikingJelly subgraphs).

Mirrors catfuse/patterns.py:52-1063: every pattern takes SpikingJelly
multi-step tensors [T, B, ...] (fp32, on the GPU), owns its parameters and a
StateBuffer for the membrane potential, resets through `reset()` (so
`functional.reset_net` clears it), and is built from the original modules
with `from_sj_modules(...)` / `from_sj_block(...)`.  The math runs in the
gfx950 kernels through an Implementation (StreamFuse on MI355X by default,
DenseKeep available) or a direct kernel launcher.

Differences from the reference that are deliberate (the reference's
behaviour diverges from SpikingJelly there):
  * the conv bias of PartialFusionConvBNLIF and the Linear bias of
    FusedLinearLIF are kept (catfuse/patterns.py:299,326-331,594-595 drop them);
  * the first state of every pattern is SpikingJelly's (v_reset for hard
    reset, 0 for soft), also when v_reset != 0;
  * CTFSEWBasicBlock with cnf='ADD' computes identity + spikes in the second
    conv's epilogue instead of a separate elementwise add.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from catfuse_amd import runtime
from catfuse_amd.hardware import runtime_profile
from catfuse_amd.implementations import ConvLIFParams, ConvLIFSpec, DenseKeep, StreamFuse
from catfuse_amd.runtime import (EPI_POOL, EPI_Z, ID_ADD_SPIKE, ID_ADD_Z, ConvLIFRunner,
                                 GroupedConvLIFRunner, avgpool2x2_lif, desc_of,
                                 global_avgpool_nhwc, lif_multistep, pad32, shadow_of)
from catfuse_amd.state import StateBuffer

try:  # SpikingJelly's MemoryModule when available, so reset_net recognises us
    from spikingjelly.activation_based.base import MemoryModule as _BaseModule  # type: ignore
except Exception:  # pragma: no cover - SpikingJelly absent
    from catfuse_amd.snn import MemoryModule as _BaseModule


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _first(v):
    return v[0] if isinstance(v, (tuple, list)) else v


def _pair(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def conv_unsupported_reason(conv) -> Optional[str]:
    """Why the fused conv kernels cannot compute this nn.Conv2d, or None.
    They compute a dense (groups = 1), undilated, zero-padded convolution
    with a square kernel, stride and padding; anything else is left to the
    original module (the matchers refuse it)."""
    groups = int(getattr(conv, "groups", 1))
    if groups != 1:
        return f"groups={groups}"
    if isinstance(getattr(conv, "padding", 0), str):
        return f"padding='{conv.padding}'"
    if any(int(d) != 1 for d in _pair(getattr(conv, "dilation", 1))):
        return f"dilation={tuple(_pair(conv.dilation))}"
    mode = getattr(conv, "padding_mode", "zeros")
    if mode != "zeros":
        return f"padding_mode='{mode}'"
    for name in ("kernel_size", "stride", "padding"):
        a, b = _pair(getattr(conv, name))
        if int(a) != int(b):
            return f"non-square {name}=({a}, {b})"
    return None


def grouped_conv_supported(conv) -> bool:
    """A grouped convolution (groups > 1, depthwise included) that the fused
    grouped kernel computes: undilated, zero padding, square kernel, stride
    and padding, channels divisible by groups."""
    groups = int(getattr(conv, "groups", 1))
    if groups <= 1 or isinstance(getattr(conv, "padding", 0), str):
        return False
    if any(int(d) != 1 for d in _pair(getattr(conv, "dilation", 1))):
        return False
    if getattr(conv, "padding_mode", "zeros") != "zeros":
        return False
    if conv.in_channels % groups or conv.out_channels % groups:
        return False
    return all(int(_pair(getattr(conv, n))[0]) == int(_pair(getattr(conv, n))[1])
               for n in ("kernel_size", "stride", "padding"))


def conv_geometry(conv):
    """(kernel_size, stride, padding) of a conv the fused kernels compute;
    ValueError for any other (conv_unsupported_reason)."""
    why = conv_unsupported_reason(conv)
    if why is not None:
        raise ValueError(f"the fused conv kernels do not compute a Conv2d with {why}")
    return int(_first(conv.kernel_size)), int(_first(conv.stride)), int(_first(conv.padding))


def is_lif_node(m) -> bool:
    """SpikingJelly's LIFNode or the catfuse_amd.snn stand-in (duck-typed on
    the class name and the neuron attributes the fused kernels read).  Other
    neurons (IFNode, ParametricLIFNode, ...) are not LIF and stay unfused."""
    if type(m).__name__ != "LIFNode":
        return False
    return all(hasattr(m, a) for a in ("v_threshold", "v_reset"))


def lif_params(lif):
    v_reset = getattr(lif, "v_reset", 0.0)
    return dict(tau=float(getattr(lif, "tau", 2.0)),
                v_threshold=float(getattr(lif, "v_threshold", 1.0)),
                v_reset=None if v_reset is None else float(v_reset),
                decay_input=bool(getattr(lif, "decay_input", True)))


def fold_bn(weight, bias, running_mean, running_var, eps):
    """scale = gamma / sqrt(var + eps), shift = beta - mean * scale (eval BN)."""
    inv_std = 1.0 / torch.sqrt(running_var + eps)
    scale = inv_std if weight is None else weight * inv_std
    shift = -running_mean * scale if bias is None else bias - running_mean * scale
    return scale.detach(), shift.detach()


def _dense_impl():
    return DenseKeep() if runtime_profile().dense_impl == "DenseKeep" else StreamFuse()


def sew_function(identity, out, cnf):
    if cnf == "ADD":
        return identity + out
    if cnf == "AND":
        return identity * out
    if cnf == "IAND":
        return identity * (1.0 - out)
    raise NotImplementedError(f"Unknown cnf: {cnf}")


# ---------------------------------------------------------------------------
# base
# ---------------------------------------------------------------------------

class CTFPattern(_BaseModule):
    """Base of all fused patterns: StateBuffer registration and reset."""

    policy_row: Optional[int] = None

    def __init__(self):
        super().__init__()
        self._catfuse_states: list = []
        self.step_mode = "m"

    def _register_state(self, state) -> None:
        if not isinstance(state, StateBuffer):
            raise TypeError(f"_register_state expects a StateBuffer, got {type(state).__name__}")
        if getattr(self, "_catfuse_states", None) is None:
            self._catfuse_states = []
        self._catfuse_states.append(state)

    def forward(self, x):
        raise NotImplementedError

    @classmethod
    def from_sj_modules(cls, *sj_modules, **kwargs):
        raise NotImplementedError

    def reset(self):
        for s in getattr(self, "_catfuse_states", []):
            s.reset()

    def single_step_forward(self, x):
        return self.forward(x)

    def multi_step_forward(self, x_seq):
        return self.forward(x_seq)


class _ConvPattern(CTFPattern):
    """Shared parts of the Conv -> (BN) -> LIF patterns."""

    def _setup(self, in_channels, out_channels, kernel_size, stride, padding, tau, v_threshold,
               v_reset, decay_input, has_bn, bn_eps, conv_bias):
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = int(kernel_size), int(stride), int(padding)
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.bn_eps = float(bn_eps)
        self.weight = nn.Parameter(torch.empty(out_channels, in_channels, kernel_size, kernel_size))
        nn.init.kaiming_normal_(self.weight)
        self.conv_bias = nn.Parameter(torch.zeros(out_channels)) if conv_bias else None
        self.state = StateBuffer()
        self._register_state(self.state)
        self.spec = ConvLIFSpec(self.in_channels, self.out_channels, self.kernel_size, self.stride,
                                self.padding, has_conv_bias=bool(conv_bias), has_bn=has_bn,
                                tau=self.tau, v_threshold=self.v_threshold, v_reset=self.v_reset,
                                decay_input=self.decay_input, bn_eps=self.bn_eps)
        self._params = None
        self._params_key = None
        # a paired launch with a downsample of the same input (CTFSEWBasicBlock):
        # _pair_with = (partner, x) for the next call, _pair_result = (x, out)
        # left for the partner's call
        self._pair_with = None
        self._pair_result = None

    def _bn_tensors(self):
        return None

    def _ensure_params(self) -> ConvLIFParams:
        # parameters read from the module's own dict (attribute lookup goes
        # through nn.Module.__getattr__ on every call)
        P = self._parameters
        w, cb = P["weight"], P.get("conv_bias")
        bn = self._bn_tensors()
        key = (id(w), w._version, None if cb is None else (id(cb), cb._version),
               None if bn is None else tuple([(id(t), t._version) for t in bn if t is not None]))
        if self._params_key == key and self._params is not None:
            return self._params
        with torch.no_grad():
            if bn is not None:
                scale, shift = fold_bn(bn[0], bn[1], bn[2], bn[3], self.bn_eps)
            else:
                scale = shift = None
        self._params = ConvLIFParams(self.weight, self.conv_bias, scale, shift)
        self._params_key = key
        return self._params

    def _run(self, impl, x, **kw):
        if x.ndim == 4:
            return impl.forward(x.unsqueeze(0), self.spec, self._ensure_params(), self.state,
                                **kw).squeeze(0)
        return impl.forward(x, self.spec, self._ensure_params(), self.state, **kw)

    def extra_repr(self):
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, padding={self.padding}, tau={self.tau}, "
                f"v_th={self.v_threshold}, v_reset={self.v_reset}")


class PartialFusionConvLIF(_ConvPattern):
    """Conv -> LIF (no BN)."""

    policy_row = 1

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, tau=2.0,
                 v_threshold=1.0, v_reset=0.0, decay_input=True, bias=False):
        super().__init__()
        self._setup(in_channels, out_channels, kernel_size, stride, padding, tau, v_threshold,
                    v_reset, decay_input, has_bn=False, bn_eps=1e-5, conv_bias=bias)
        self._impl = _dense_impl()

    def forward(self, x):
        return self._run(self._impl, x)

    @classmethod
    def from_sj_modules(cls, sj_conv, sj_lif):
        k, s, p = conv_geometry(sj_conv)
        inst = cls(sj_conv.in_channels, sj_conv.out_channels, k, s, p,
                   bias=sj_conv.bias is not None, **lif_params(sj_lif))
        with torch.no_grad():
            inst.weight.copy_(sj_conv.weight)
            if sj_conv.bias is not None:
                inst.conv_bias.copy_(sj_conv.bias)
        return inst.to(sj_conv.weight.device)


class PartialFusionConvBNLIF(_ConvPattern):
    """Conv -> BN (eval, folded) -> LIF."""

    policy_row = 2

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, tau=2.0,
                 v_threshold=1.0, v_reset=0.0, bn_eps=1e-5, decay_input=True, bias=False):
        super().__init__()
        self._setup(in_channels, out_channels, kernel_size, stride, padding, tau, v_threshold,
                    v_reset, decay_input, has_bn=True, bn_eps=bn_eps, conv_bias=bias)
        self.bn_weight = nn.Parameter(torch.ones(out_channels))
        self.bn_bias = nn.Parameter(torch.zeros(out_channels))
        self.register_buffer("running_mean", torch.zeros(out_channels))
        self.register_buffer("running_var", torch.ones(out_channels))
        self._impl = _dense_impl()

    def _bn_tensors(self):
        P, B = self._parameters, self._buffers
        return (P["bn_weight"], P["bn_bias"], B["running_mean"], B["running_var"])

    def forward(self, x, sew_identity=None):
        # the hand-over slots are plain instance attributes, written through
        # __dict__ (nn.Module.__setattr__ costs a microsecond per write)
        d = self.__dict__
        pr = d["_pair_result"]
        d["_pair_result"] = None
        if pr is not None and pr[0] is x and sew_identity is None:
            return pr[1]                   # computed by the partner's paired launch
        pw = d["_pair_with"]
        d["_pair_with"] = None
        impl = self._modules["_impl"]
        if pw is not None and pw[1] is x and sew_identity is None:
            res = _paired_forward(self, pw[0], x)
            if res is not None:
                pw[0].__dict__["_pair_result"] = (x, res[1])
                return res[0]
        if sew_identity is not None:
            return self._run(impl, x, identity=sew_identity, identity_mode=ID_ADD_SPIKE)
        return self._run(impl, x)

    def supports_sew_identity(self):
        return isinstance(self._impl, StreamFuse)

    def _copy_bn(self, sj_bn):
        with torch.no_grad():
            if sj_bn.weight is not None:
                self.bn_weight.copy_(sj_bn.weight)
            if sj_bn.bias is not None:
                self.bn_bias.copy_(sj_bn.bias)
            self.running_mean.copy_(sj_bn.running_mean)
            self.running_var.copy_(sj_bn.running_var)

    @classmethod
    def from_sj_modules(cls, sj_conv, sj_bn, sj_lif):
        k, s, p = conv_geometry(sj_conv)
        inst = cls(sj_conv.in_channels, sj_conv.out_channels, k, s, p, bn_eps=sj_bn.eps,
                   bias=sj_conv.bias is not None, **lif_params(sj_lif))
        with torch.no_grad():
            inst.weight.copy_(sj_conv.weight)
            if sj_conv.bias is not None:
                inst.conv_bias.copy_(sj_conv.bias)
        inst._copy_bn(sj_bn)
        return inst.to(sj_conv.weight.device)


class PartialFusionConvBNAddLIF(PartialFusionConvBNLIF):
    """Conv -> BN -> (+ identity) -> LIF, the second half of a spiking-ResNet
    block; identity is added to z inside the conv epilogue."""

    policy_row = 9

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        self._impl = StreamFuse()

    def forward(self, x, identity):
        return self._run(self._impl, x, identity=identity.contiguous(), identity_mode=ID_ADD_Z)


class PartialFusionConvBNAvgPoolLIF(PartialFusionConvBNLIF):
    """Conv -> BN -> AvgPool2d(2, 2) -> LIF.  A spike input to a stride-1
    3x3 conv with whole 32-channel groups runs the whole chain in the conv
    kernel (cf_conv_mfma's pooled epilogue: BN, the 2x2 average of the z
    tile in registers, the pooled LIF; only the pooled spikes and state are
    written), and so does an analog input of at most 4 channels
    (cf_conv_direct_avgpool_lif, fp32 VALU: VGG's first layer).  Otherwise
    the conv writes z (BN in its epilogue) and the pooled LIF runs in one
    streaming kernel; every path gives the same bits (the
    reference's F8, catfuse/kernels/conv_pool_lif.py:94-178: the 2x2 average
    (z00 + z01 + z10 + z11) * 0.25 in that order, line 162, then the LIF
    with v in registers across the steps)."""

    policy_row = "ConvBNAvgPoolLIF"

    def _pool_in_epilogue(self, H, W) -> bool:
        k, p = self.kernel_size, self.padding
        return (k == 3 and self.stride == 1 and self.out_channels % 32 == 0
                and H + 2 * p - k + 1 >= 2 and W + 2 * p - k + 1 >= 2)

    def forward(self, x):
        squeeze = x.ndim == 4
        if squeeze:
            x = x.unsqueeze(0)
        params = self._ensure_params()
        impl = self._impl
        r = impl.runner(self.spec, params, x.device)
        T, B, _, H, W = x.shape
        analog = impl.input_is_analog(x)
        if (self._pool_in_epilogue(H, W) if not analog else r.direct_avgpool_supported(x)):
            Ho, Wo = r.out_hw(H, W)
            v_in = self.state.peek((B, self.out_channels, Ho // 2, Wo // 2), x.device)
            if analog:
                s, v = r.run_direct_avgpool(x, v_in, nz_out=r.out_counter(x.device),
                                            gen_cell=r._gen)
            else:
                s, v = r.run_mfma(x.contiguous(), v_in, epilogue=EPI_POOL, static_zero=True)
            self.state.set(v)
            return s.squeeze(0) if squeeze else s
        if analog:
            z, _ = r.run_direct(x, epilogue=EPI_Z)
        else:
            z, _ = r.run_mfma(x.contiguous(), epilogue=EPI_Z, static_zero=True)
        T, B, C, H, W = z.shape
        v_in = self.state.peek((B, C, H // 2, W // 2), z.device)
        s, v = avgpool2x2_lif(z, v_in, tau=self.tau, v_threshold=self.v_threshold,
                              v_reset=self.v_reset, decay_input=self.decay_input)
        self.state.set(v)
        return s.squeeze(0) if squeeze else s

    @classmethod
    def from_sj_modules(cls, sj_conv, sj_bn, sj_pool, sj_lif):
        inst = super().from_sj_modules(sj_conv, sj_bn, sj_lif)
        ks, st = _first(sj_pool.kernel_size), _first(sj_pool.stride or sj_pool.kernel_size)
        if ks != 2 or st != 2 or _first(getattr(sj_pool, "padding", 0)) != 0:
            raise ValueError("only AvgPool2d(2, 2) is fused")
        return inst


class PartialFusionConvBNLIFMaxPool(PartialFusionConvBNLIF):
    """Conv -> BN -> LIF -> MaxPool2d(3, 2, 1): the SEW/Spiking-ResNet stem.

    No counterpart in the reference, which fuses conv1/bn1/sn1
    (catfuse/patterns.py:237-387) and leaves SpikingJelly's MaxPool2d after
    it.  For a direct-encoded image (the same frame at every step, a stride-0
    time axis) the whole chain is one gfx950 kernel
    (cf_conv_stem_lif_maxpool): the conv runs once per image on the matrix
    cores, the LIF over T, and the max of spikes is the OR of their trains.
    Any other input takes the Conv->BN->LIF kernels followed by the pool.
    The state is the conv-resolution membrane, as SpikingJelly's sn1 keeps."""

    policy_row = "ConvBNLIFMaxPool"

    def __init__(self, *args, pool=(3, 2, 1), **kw):
        super().__init__(*args, **kw)
        self.pool = tuple(int(p) for p in pool)

    def forward(self, x):
        squeeze = x.ndim == 4
        if squeeze:
            x = x.unsqueeze(0)
        self._impl.check_input(x, self.spec)
        params = self._ensure_params()
        r = self._impl.runner(self.spec, params, x.device)
        if r.stem_supported(x, self.pool) and self._impl.input_is_analog(x):
            B = x.shape[1]
            Hc, Wc = r.out_hw(x.shape[3], x.shape[4])
            v_in = self.state.peek((B, self.out_channels, Hc, Wc), x.device)
            s, v = r.run_stem_pool(x, v_in)
            self.state.set(v)
        else:
            y = self._run(self._impl, x)
            T, B = y.shape[:2]
            k, st, pd = self.pool
            s = torch.nn.functional.max_pool2d(y.flatten(0, 1), k, st, pd)
            s = s.reshape(T, B, *s.shape[1:])
        return s.squeeze(0) if squeeze else s

    @classmethod
    def from_sj_modules(cls, sj_conv, sj_bn, sj_lif, sj_pool):
        ks = _first(sj_pool.kernel_size)
        st = _first(sj_pool.stride if sj_pool.stride is not None else sj_pool.kernel_size)
        pd = _first(getattr(sj_pool, "padding", 0))
        if (ks, st, pd) != (3, 2, 1) or _first(getattr(sj_pool, "dilation", 1)) != 1 or \
                getattr(sj_pool, "ceil_mode", False):
            raise ValueError("only MaxPool2d(3, 2, 1) is fused")
        k, s, p = conv_geometry(sj_conv)
        inst = cls(sj_conv.in_channels, sj_conv.out_channels, k, s, p, bn_eps=sj_bn.eps,
                   bias=sj_conv.bias is not None, pool=(ks, st, pd), **lif_params(sj_lif))
        with torch.no_grad():
            inst.weight.copy_(sj_conv.weight)
            if sj_conv.bias is not None:
                inst.conv_bias.copy_(sj_conv.bias)
        inst._copy_bn(sj_bn)
        return inst.to(sj_conv.weight.device)


class PartialFusionGroupedConvBNLIF(CTFPattern):
    """Grouped Conv (groups > 1; depthwise when groups == in_channels) ->
    BN (eval, folded) -> LIF in one launch over all T steps
    (cf_conv_grouped_lif).  The reference runs a grouped conv as `groups`
    independent sparse sub-convs with the LIF separate
    (catfuse/sparseflow/sparse_grouped_conv2d_kernel.py:93-364); a grouped
    conv is HBM-bound (Cin/groups * k^2 products per output), so here it is
    one streaming kernel on the fp16 NHWC copies, StaticZero on an all-zero
    input.  The membrane state is channels-last ([B, Cout, Ho, Wo] in
    torch's channels_last format).  Analog inputs are read in fp32."""

    policy_row = "GroupedConvBNLIF"

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, groups=1,
                 tau=2.0, v_threshold=1.0, v_reset=0.0, bn_eps=1e-5, decay_input=True,
                 bias=False, has_bn=True):
        super().__init__()
        if in_channels % groups or out_channels % groups:
            raise ValueError("channels must be divisible by groups")
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = int(kernel_size), int(stride), int(padding)
        self.groups = int(groups)
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.bn_eps = float(bn_eps)
        self.weight = nn.Parameter(torch.empty(out_channels, in_channels // groups, kernel_size,
                                               kernel_size))
        nn.init.kaiming_normal_(self.weight)
        self.conv_bias = nn.Parameter(torch.zeros(out_channels)) if bias else None
        if has_bn:
            self.bn_weight = nn.Parameter(torch.ones(out_channels))
            self.bn_bias = nn.Parameter(torch.zeros(out_channels))
            self.register_buffer("running_mean", torch.zeros(out_channels))
            self.register_buffer("running_var", torch.ones(out_channels))
        else:
            self.bn_weight = self.bn_bias = None
            self.register_buffer("running_mean", None)
            self.register_buffer("running_var", None)
        self.state = StateBuffer()
        self._register_state(self.state)
        self._runner = None
        self._runner_key = None
        self._exact_input = None

    def runner(self) -> GroupedConvLIFRunner:
        ts = [t for t in (self.weight, self.conv_bias, self.bn_weight, self.bn_bias,
                          self.running_mean, self.running_var) if t is not None]
        key = tuple((id(t), t._version, t.device) for t in ts)
        if key != self._runner_key:
            scale = shift = None
            if self.bn_weight is not None:
                scale, shift = fold_bn(self.bn_weight, self.bn_bias, self.running_mean,
                                       self.running_var, self.bn_eps)
            self._runner = GroupedConvLIFRunner(
                self.weight.detach(), self.groups, scale, shift,
                None if self.conv_bias is None else self.conv_bias.detach(), self.stride,
                self.padding, self.tau, self.v_threshold, self.v_reset, self.decay_input)
            self._runner_key = key
        return self._runner

    def forward(self, x):
        squeeze = x.ndim == 4
        if squeeze:
            x = x.unsqueeze(0)
        if x.dim() != 5 or not x.is_cuda or x.dtype != torch.float32:
            raise RuntimeError("catfuse_amd fused patterns take float32 GPU [T, B, C, H, W] "
                               "tensors (there is no CPU path)")
        if self._exact_input is None:   # one host check per layer: spikes or analog values
            self._exact_input = bool((x.half().float() == x).all().item())
        r = self.runner()
        B = x.shape[1]
        Ho, Wo = r.out_hw(x.shape[3], x.shape[4])
        v_in = self.state.peek((B, self.out_channels, Ho, Wo), x.device)
        s, v = r.run(x, v_in, analog=not self._exact_input)
        self.state.set(v)
        return s.squeeze(0) if squeeze else s

    @classmethod
    def from_sj_modules(cls, sj_conv, sj_bn, sj_lif):
        if not grouped_conv_supported(sj_conv):
            raise ValueError("not a grouped conv the fused grouped kernel computes")
        k, s, p = (int(_first(getattr(sj_conv, n))) for n in ("kernel_size", "stride", "padding"))
        inst = cls(sj_conv.in_channels, sj_conv.out_channels, k, s, p, sj_conv.groups,
                   bn_eps=sj_bn.eps if sj_bn is not None else 1e-5,
                   bias=sj_conv.bias is not None, has_bn=sj_bn is not None, **lif_params(sj_lif))
        with torch.no_grad():
            inst.weight.copy_(sj_conv.weight)
            if sj_conv.bias is not None:
                inst.conv_bias.copy_(sj_conv.bias)
            if sj_bn is not None:
                inst.bn_weight.copy_(sj_bn.weight)
                inst.bn_bias.copy_(sj_bn.bias)
                inst.running_mean.copy_(sj_bn.running_mean)
                inst.running_var.copy_(sj_bn.running_var)
        return inst.to(sj_conv.weight.device)

    def extra_repr(self):
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, padding={self.padding}, groups={self.groups}, "
                f"tau={self.tau}, v_th={self.v_threshold}, v_reset={self.v_reset}")


# ---------------------------------------------------------------------------
# Linear -> LIF
# ---------------------------------------------------------------------------

class FusedLinearLIF(CTFPattern):
    """Linear (+bias) -> LIF on [T, B, I] (catfuse/patterns.py:533-571: the
    linear over the T * B rows, then the LIF over T with the state
    [B, out]).  Spike inputs run on the matrix cores as a 1x1 convolution
    over the B samples of each step viewed as token images
    (ConvLIFRunner.run_tokens: 8 x 8 images of 64 samples when 64 divides
    B), the LIF in its epilogue; the output is the fp16 copy the next fused
    layer reads.  The state is kept in that launch view, [nimg, out, H * W];
    membrane() gives it as [B, out].  Analog inputs take the fp32 direct
    path, state [B, out, 1, 1]."""

    policy_row = 4

    def __init__(self, in_features, out_features, tau=2.0, v_threshold=1.0, v_reset=0.0,
                 decay_input=True, bias=True):
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.weight_io = nn.Parameter(torch.empty(in_features, out_features))
        nn.init.kaiming_normal_(self.weight_io.T)
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None
        self.state = StateBuffer()
        self._register_state(self.state)
        self.spec = ConvLIFSpec(self.in_features, self.out_features, 1, 1, 0,
                                has_conv_bias=bool(bias), has_bn=False, tau=self.tau,
                                v_threshold=self.v_threshold, v_reset=self.v_reset,
                                decay_input=self.decay_input)
        self._impl = StreamFuse()
        self._params = None
        self._params_key = None
        self._batch = None   # B of the last spike-input call (the state's view)

    def _ensure_params(self):
        key = (id(self.weight_io), self.weight_io._version,
               None if self.bias is None else (id(self.bias), self.bias._version))
        if self._params_key != key:
            w = self.weight_io.detach().t().contiguous().view(self.out_features, self.in_features, 1, 1)
            self._params = ConvLIFParams(w, self.bias, None, None)
            self._params_key = key
        return self._params

    def forward(self, x):
        squeeze = x.ndim == 2
        if squeeze:
            x = x.unsqueeze(0)
        T, B, I = x.shape
        impl = self._impl
        params = self._ensure_params()
        if not isinstance(x, runtime.NHWCSpikes) and impl.input_is_analog(x):
            y = impl.forward(x.reshape(T, B, I, 1, 1), self.spec, params, self.state)
            y = y.reshape(T, B, self.out_features)
            self._batch = None
            return y.squeeze(0) if squeeze else y
        r = impl.runner(self.spec, params, x.device)
        nimg, H, W = runtime.token_view(B, 1)
        v_in = self.state.peek((nimg, self.out_features, H * W), x.device)
        y, v = r.run_tokens(x, v_in)
        self.state.set(v)
        self.__dict__["_batch"] = B   # a plain attribute (no nn.Module hook)
        return y.squeeze(0) if squeeze else y

    def membrane(self):
        """The LIF state after the last call as [B, out_features] (None after
        a reset)."""
        v = self.state.tensor
        if v is None:
            return None
        if self.__dict__.get("_batch") is None:
            return v.reshape(v.shape[0], self.out_features)
        return runtime.token_membrane(v, self._batch, 1).reshape(self._batch, self.out_features)

    @classmethod
    def from_sj_modules(cls, sj_linear, sj_lif):
        inst = cls(sj_linear.in_features, sj_linear.out_features,
                   bias=sj_linear.bias is not None, **lif_params(sj_lif))
        with torch.no_grad():
            inst.weight_io.copy_(sj_linear.weight.t())
            if sj_linear.bias is not None:
                inst.bias.copy_(sj_linear.bias)
        return inst.to(sj_linear.weight.device)


# ---------------------------------------------------------------------------
# streaming tails: Add -> LIF, Add -> BN -> LIF, AvgPool -> LIF
# ---------------------------------------------------------------------------

class _TailPattern(CTFPattern):
    def _lif_setup(self, tau, v_threshold, v_reset, decay_input):
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.state = StateBuffer()
        self._register_state(self.state)

    def _lif(self, z, **kw):
        v_in = self.state.peek(z.shape[1:], z.device)
        s, v = lif_multistep(z, v_in, tau=self.tau, v_threshold=self.v_threshold,
                             v_reset=self.v_reset, decay_input=self.decay_input, **kw)
        self.state.set(v)
        return s


class FusedLIF(_TailPattern):
    """A multi-step LIF node that no fused pattern absorbed (e.g. the
    pre-head LIF of a spiking transformer), as one streaming kernel:
    cf_lif_multistep over x [T, ...] with v in registers across T
    (catfuse/sparseflow/lif_seq_kernel.py:51-90 `lif_sequential`, the
    kernel the reference's patterns call; bit-exact against the LIF oracle).
    The state is [...] of one step, as SpikingJelly's node keeps it."""

    policy_row = "LIF"

    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True):
        super().__init__()
        self._lif_setup(tau, v_threshold, v_reset, decay_input)
        self.step_mode = "m"

    def forward(self, x):
        return self._lif(x.contiguous())

    @classmethod
    def from_sj_modules(cls, sj_lif):
        return cls(**lif_params(sj_lif))


class FusedAddLIF(_TailPattern):
    """a + x -> LIF (catfuse/kernels/add_lif.py:63-151)."""

    policy_row = 5

    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True):
        super().__init__()
        self._lif_setup(tau, v_threshold, v_reset, decay_input)

    def forward(self, a, x):
        return self._lif(a.contiguous(), mode=3, z2=x.contiguous())

    @classmethod
    def from_sj_modules(cls, sj_lif):
        return cls(**lif_params(sj_lif))


class FusedAddBNLIF(_TailPattern):
    """(a + x) -> BN (eval) -> LIF (benchmarks/add_bn_lif_min.py:72-226)."""

    policy_row = 6

    def __init__(self, num_features, tau=2.0, v_threshold=1.0, v_reset=0.0, bn_eps=1e-5,
                 decay_input=True):
        super().__init__()
        self._lif_setup(tau, v_threshold, v_reset, decay_input)
        self.num_features = int(num_features)
        self.bn_eps = float(bn_eps)
        self.bn_weight = nn.Parameter(torch.ones(num_features))
        self.bn_bias = nn.Parameter(torch.zeros(num_features))
        self.register_buffer("running_mean", torch.zeros(num_features))
        self.register_buffer("running_var", torch.ones(num_features))

    def forward(self, a, x):
        scale, shift = fold_bn(self.bn_weight, self.bn_bias, self.running_mean, self.running_var,
                               self.bn_eps)
        T, B, C = a.shape[:3]
        hw = a[0, 0, 0].numel()
        return self._lif(a.contiguous(), mode=4, z2=x.contiguous(), scale=scale.contiguous(),
                         shift=shift.contiguous(), channels=C, hw=hw)

    @classmethod
    def from_sj_modules(cls, sj_bn, sj_lif):
        inst = cls(sj_bn.num_features, bn_eps=sj_bn.eps, **lif_params(sj_lif))
        with torch.no_grad():
            inst.bn_weight.copy_(sj_bn.weight)
            inst.bn_bias.copy_(sj_bn.bias)
            inst.running_mean.copy_(sj_bn.running_mean)
            inst.running_var.copy_(sj_bn.running_var)
        return inst.to(sj_bn.running_mean.device)


class FusedAvgPoolLIF(_TailPattern):
    """AvgPool2d(2, 2) -> LIF (catfuse/kernels/avgpool_lif.py:61-190)."""

    policy_row = 7

    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True):
        super().__init__()
        self._lif_setup(tau, v_threshold, v_reset, decay_input)

    def forward(self, x):
        T, B, C, H, W = x.shape
        v_in = self.state.peek((B, C, H // 2, W // 2), x.device)
        s, v = avgpool2x2_lif(x.contiguous(), v_in, tau=self.tau, v_threshold=self.v_threshold,
                              v_reset=self.v_reset, decay_input=self.decay_input)
        self.state.set(v)
        return s

    @classmethod
    def from_sj_modules(cls, sj_pool, sj_lif):
        if _first(sj_pool.kernel_size) != 2 or _first(sj_pool.stride or 2) != 2:
            raise ValueError("only AvgPool2d(2, 2) is fused")
        return cls(**lif_params(sj_lif))


class FusedGlobalAvgPool(nn.Module):
    """AdaptiveAvgPool2d((1, 1)) of a network head that reads the fp16 NHWC
    copy a fused conv wrote (cf_global_avgpool_nhwc) instead of first
    materialising the fp32 feature map.  No counterpart in the reference,
    whose fused layers hand the head (SpikingJelly's layer.AdaptiveAvgPool2d)
    an fp32 tensor.  Values: torch's GPU mean (fp32 sum over H x W, times
    float(1)/(H*W)); the copy's values are integers, so the sum is exact and
    the result bit-identical.  Inputs without a current copy go through
    torch's adaptive_avg_pool2d (counted in `fallback_calls`).
    step_mode 'm': x [T, B, C, H, W] -> [T, B, C, 1, 1]; 's': [N, C, H, W] ->
    [N, C, 1, 1]."""

    def __init__(self, step_mode: str = "s"):
        super().__init__()
        self.step_mode = step_mode
        self.fallback_calls = 0

    def forward(self, x):
        lead = x.shape[:-3]
        C, H, W = x.shape[-3:]
        nb = 1
        for d in lead:
            nb *= int(d)
        xp = shadow_of(x, (nb, H, W, pad32(C)), resolve=False, u8_ok=True) if x.is_cuda else None
        if xp is not None:
            return global_avgpool_nhwc(xp, C, desc=desc_of(x)).view(*lead, C, 1, 1)
        self.fallback_calls += 1
        y = nn.functional.adaptive_avg_pool2d(x.reshape(nb, C, H, W), 1)
        return y.view(*lead, C, 1, 1)

    @classmethod
    def from_sj_modules(cls, pool):
        return cls(getattr(pool, "step_mode", "s"))


class FusedLinear(nn.Module):
    """A network's last Linear (no neuron) after a fused Linear-LIF: reads
    the spikes from the fp16 copy the fused layer wrote (through its
    descriptor, cf_linear_tokens) instead of their fp32 form.  No
    counterpart in the reference (SpikingJelly's layer.Linear).  fp32
    accumulation in a fixed order: equal to F.linear within fp32 rounding.
    Inputs without a current copy go through F.linear (counted in
    `fallback_calls`)."""

    def __init__(self, in_features, out_features, bias=True):
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None
        self.fallback_calls = 0

    def forward(self, x):
        if x.is_cuda and x.shape[-1] == self.in_features:
            y = runtime.linear_tokens(x, self.weight.detach(),
                                      None if self.bias is None else self.bias.detach())
            if y is not None:
                return y
        self.fallback_calls += 1
        return nn.functional.linear(x, self.weight, self.bias)

    @classmethod
    def from_sj_modules(cls, linear):
        inst = cls(linear.in_features, linear.out_features, bias=linear.bias is not None)
        with torch.no_grad():
            inst.weight.copy_(linear.weight)
            if linear.bias is not None:
                inst.bias.copy_(linear.bias)
        return inst.to(linear.weight.device)


class FusedFlatten(nn.Module):
    """Flatten of a network head in multi-step mode ([T, B, C, H, W] ->
    [T, B, C * H * W], SpikingJelly's layer.Flatten with step_mode 'm').  A
    fused layer's one-pixel output (H = W = 1, e.g. the last VGG pool) stays
    in its fp16 copy (runtime.pixel_tokens): the fused linear layer that
    follows reads the copy instead of a packed fp32 tensor.  No counterpart
    in the reference.  Anything else is torch.flatten (counted in
    `fallback_calls`)."""

    def __init__(self):
        super().__init__()
        self.step_mode = "m"
        self.fallback_calls = 0

    def forward(self, x):
        if x.dim() == 5:
            y = runtime.pixel_tokens(x)
            if y is not None:
                return y
        self.fallback_calls += 1
        return torch.flatten(x, 2)

    @classmethod
    def from_sj_modules(cls, flat):
        if (getattr(flat, "step_mode", "s") != "m" or flat.start_dim != 1
                or flat.end_dim != -1):
            raise ValueError("only the multi-step Flatten(start_dim=1) is fused")
        return cls()


# ---------------------------------------------------------------------------
# blocks
# ---------------------------------------------------------------------------

def _conv_bn_lif_from(conv, bn, lif, K=None):
    """STFusionConvBNLIF for 3x3/s1 layers in the SparseFlow regime is chosen
    by substitute_sf; blocks built here use the dense pattern."""
    return PartialFusionConvBNLIF.from_sj_modules(conv, bn, lif)


def _paired_forward(fa, fb, x):
    """fa (3x3, stride 2) and fb (1x1, stride 2) of the same input in one
    cf_conv_halo_pair launch when both run the fused dense conv on a spike
    input the pair kernel covers: (out_a, out_b), each module's state set as
    its own call would; None otherwise."""
    ia, ib = fa._impl, fb._impl
    if type(ia) is not StreamFuse or type(ib) is not StreamFuse or x.ndim != 5:
        return None
    ia.check_input(x, fa.spec)
    ib.check_input(x, fb.spec)
    if ia.input_is_analog(x) or ib.input_is_analog(x):
        return None
    dev = x.device
    ra = ia.runner(fa.spec, fa._ensure_params(), dev)
    rb = ib.runner(fb.spec, fb._ensure_params(), dev)
    B = x.shape[1]
    Ho, Wo = fa.spec.output_hw(x.shape[3], x.shape[4])
    va = fa.state.peek((B, fa.out_channels, Ho, Wo), dev)
    vb = fb.state.peek((B, fb.out_channels, Ho, Wo), dev)
    # no initial states: the launch plan cached for x's signature, when
    # there is one (it was made by the same support checks)
    res = runtime.halo_pair_repeat(ra, rb, x) if va is None and vb is None else None
    if res is None:
        if not runtime.halo_pair_supported(ra, rb, x):
            return None
        res = runtime.run_halo_pair(ra, rb, x.contiguous(), va, vb)
    out_a, v_a, out_b, v_b = res
    fa.state.set(v_a)
    fb.state.set(v_b)
    return out_a, out_b


class CTFSEWBasicBlock(CTFPattern):
    """SEW-ResNet BasicBlock: out = sew(identity, LIF(BN(conv2(LIF(BN(conv1 x))))))
    with identity = downsample_sn(downsample(x)) or x; for cnf='ADD' the add
    is done in conv2's epilogue.  A stride-2 conv1 and its 1x1 downsample
    run as one paired launch (cf_conv_halo_pair): conv1's call computes
    both, the downsample's call returns its half (each module is still
    called, so its hooks run)."""

    def __init__(self, fused_first, fused_second, fused_downsample, cnf):
        super().__init__()
        self.fused_first = fused_first
        self.fused_second = fused_second
        self.fused_downsample = fused_downsample
        self.cnf = cnf

    def forward(self, x):
        mods = self._modules
        first, ds = mods["fused_first"], mods.get("fused_downsample")
        paired = (ds is not None and isinstance(first, PartialFusionConvBNLIF)
                  and isinstance(ds, PartialFusionConvBNLIF) and first.stride == 2)
        if paired:
            first.__dict__["_pair_with"] = (ds, x)
        out = first(x)
        if paired:
            first.__dict__["_pair_with"] = None
        identity = ds(x) if ds is not None else x
        second = mods["fused_second"]
        if (self.cnf == "ADD" and getattr(second, "supports_sew_identity", lambda: False)()
                and identity.shape[:2] == out.shape[:2]):
            return second(out, sew_identity=identity.contiguous())
        return sew_function(identity, second(out), self.cnf)

    @classmethod
    def from_sj_block(cls, sj_block):
        first = _conv_bn_lif_from(sj_block.conv1, sj_block.bn1, sj_block.sn1)
        second = _conv_bn_lif_from(sj_block.conv2, sj_block.bn2, sj_block.sn2)
        ds = None
        if sj_block.downsample is not None:
            ds = PartialFusionConvBNLIF.from_sj_modules(sj_block.downsample[0],
                                                        sj_block.downsample[1],
                                                        sj_block.downsample_sn)
        return cls(first, second, ds, sj_block.cnf)


class _DownsampleConvBN(nn.Module):
    """Conv -> BN without LIF (spiking-ResNet shortcut), z from the MFMA conv."""

    def __init__(self, weight, bn_scale, bn_bias, stride, padding):
        super().__init__()
        self.weight = nn.Parameter(weight.detach().clone())
        self.register_buffer("bn_scale", bn_scale.detach().clone())
        self.register_buffer("bn_bias", bn_bias.detach().clone())
        self.stride, self.padding = int(stride), int(padding)
        self._runner = None
        self._key = None

    def forward(self, x):
        key = (id(self.weight), self.weight._version, id(self.bn_scale), id(self.bn_bias))
        if self._key != key:
            self._runner = ConvLIFRunner(self.weight, self.bn_scale, self.bn_bias, None,
                                         self.stride, self.padding, 2.0, 1.0, 0.0, True)
            self._key = key
        z, _ = self._runner.run_mfma(x.contiguous(), epilogue=EPI_Z, static_zero=True)
        return z


class CTFSpikingBasicBlock(CTFPattern):
    """Spiking-ResNet BasicBlock: LIF(BN(conv2(LIF(BN(conv1 x)))) + identity),
    identity = BN(conv_ds(x)) or x (no LIF on the shortcut)."""

    def __init__(self, fused_first, fused_second_add, downsample_conv_weight, downsample_bn_scale,
                 downsample_bn_bias, downsample_stride, downsample_padding):
        super().__init__()
        self.fused_first = fused_first
        self.fused_second_add = fused_second_add
        self.has_downsample = downsample_conv_weight is not None
        self.downsample = (_DownsampleConvBN(downsample_conv_weight, downsample_bn_scale,
                                             downsample_bn_bias, downsample_stride,
                                             downsample_padding)
                           if self.has_downsample else None)

    def forward(self, x):
        out = self.fused_first(x)
        identity = self.downsample(x) if self.has_downsample else x
        return self.fused_second_add(out, identity)

    @classmethod
    def from_sj_block(cls, sj_block):
        first = PartialFusionConvBNLIF.from_sj_modules(sj_block.conv1, sj_block.bn1, sj_block.sn1)
        second = PartialFusionConvBNAddLIF.from_sj_modules(sj_block.conv2, sj_block.bn2,
                                                           sj_block.sn2)
        if sj_block.downsample is None:
            return cls(first, second, None, None, None, 0, 0)
        c, b = sj_block.downsample[0], sj_block.downsample[1]
        sc, sh = fold_bn(b.weight, b.bias, b.running_mean, b.running_var, b.eps)
        k, s, p = conv_geometry(c)
        return cls(first, second, c.weight.data, sc, sh, s, p)


class CTFSEWBottleneck(CTFPattern):
    """SEW-ResNet Bottleneck: three Conv-BN-LIF stages + SEW connect."""

    def __init__(self, fused_first, fused_middle, fused_last, fused_downsample, cnf):
        super().__init__()
        self.fused_first = fused_first
        self.fused_middle = fused_middle
        self.fused_last = fused_last
        self.fused_downsample = fused_downsample
        self.cnf = cnf

    def forward(self, x):
        out = self.fused_middle(self.fused_first(x))
        identity = self.fused_downsample(x) if self.fused_downsample is not None else x
        if self.cnf == "ADD" and self.fused_last.supports_sew_identity():
            return self.fused_last(out, sew_identity=identity.contiguous())
        return sew_function(identity, self.fused_last(out), self.cnf)

    @classmethod
    def from_sj_block(cls, b):
        mk = PartialFusionConvBNLIF.from_sj_modules
        ds = None
        if b.downsample is not None:
            ds = mk(b.downsample[0], b.downsample[1], b.downsample_sn)
        return cls(mk(b.conv1, b.bn1, b.sn1), mk(b.conv2, b.bn2, b.sn2), mk(b.conv3, b.bn3, b.sn3),
                   ds, b.cnf)


class CTFSpikingBottleneck(CTFPattern):
    """Spiking-ResNet Bottleneck: LIF(BN(conv3(...)) + identity) last."""

    def __init__(self, fused_first, fused_middle, fused_last_add, downsample_conv_weight,
                 downsample_bn_scale, downsample_bn_bias, downsample_stride, downsample_padding):
        super().__init__()
        self.fused_first = fused_first
        self.fused_middle = fused_middle
        self.fused_last_add = fused_last_add
        self.has_downsample = downsample_conv_weight is not None
        self.downsample = (_DownsampleConvBN(downsample_conv_weight, downsample_bn_scale,
                                             downsample_bn_bias, downsample_stride,
                                             downsample_padding)
                           if self.has_downsample else None)

    def forward(self, x):
        out = self.fused_middle(self.fused_first(x))
        identity = self.downsample(x) if self.has_downsample else x
        return self.fused_last_add(out, identity)

    @classmethod
    def from_sj_block(cls, b):
        mk = PartialFusionConvBNLIF.from_sj_modules
        last = PartialFusionConvBNAddLIF.from_sj_modules(b.conv3, b.bn3, b.sn3)
        if b.downsample is None:
            return cls(mk(b.conv1, b.bn1, b.sn1), mk(b.conv2, b.bn2, b.sn2), last,
                       None, None, None, 0, 0)
        c, bn = b.downsample[0], b.downsample[1]
        sc, sh = fold_bn(bn.weight, bn.bias, bn.running_mean, bn.running_var, bn.eps)
        k, s, p = conv_geometry(c)
        return cls(mk(b.conv1, b.bn1, b.sn1), mk(b.conv2, b.bn2, b.sn2), last, c.weight.data,
                   sc, sh, s, p)


PATTERN_REGISTRY = {
    "PartialFusionConvLIF": PartialFusionConvLIF,
    "PartialFusionConvBNLIF": PartialFusionConvBNLIF,
    "PartialFusionConvBNAddLIF": PartialFusionConvBNAddLIF,
    "PartialFusionConvBNAvgPoolLIF": PartialFusionConvBNAvgPoolLIF,
    "PartialFusionConvBNLIFMaxPool": PartialFusionConvBNLIFMaxPool,
    "PartialFusionGroupedConvBNLIF": PartialFusionGroupedConvBNLIF,
    "FusedLinearLIF": FusedLinearLIF,
    "FusedAddLIF": FusedAddLIF,
    "FusedAddBNLIF": FusedAddBNLIF,
    "FusedAvgPoolLIF": FusedAvgPoolLIF,
    "CTFSEWBasicBlock": CTFSEWBasicBlock,
    "CTFSpikingBasicBlock": CTFSpikingBasicBlock,
    "CTFSEWBottleneck": CTFSEWBottleneck,
    "CTFSpikingBottleneck": CTFSpikingBottleneck,
}

from catfuse_amd.sparseflow.ops.st_fusion_conv_bn_lif import STFusionConvBNLIF  # noqa: E402

PATTERN_REGISTRY["STFusionConvBNLIF"] = STFusionConvBNLIF

__all__ = ["CTFPattern", "PartialFusionConvLIF", "PartialFusionConvBNLIF",
           "PartialFusionConvBNAddLIF", "PartialFusionConvBNAvgPoolLIF",
           "PartialFusionConvBNLIFMaxPool", "PartialFusionGroupedConvBNLIF", "FusedLinearLIF",
           "FusedAddLIF", "FusedAddBNLIF", "FusedAvgPoolLIF", "FusedGlobalAvgPool",
           "FusedFlatten", "FusedLinear", "FusedLIF", "CTFSEWBasicBlock",
           "CTFSpikingBasicBlock", "CTFSEWBottleneck", "CTFSpikingBottleneck",
           "STFusionConvBNLIF", "PATTERN_REGISTRY", "fold_bn", "lif_params", "conv_geometry",
           "conv_unsupported_reason", "grouped_conv_supported", "is_lif_node"]
