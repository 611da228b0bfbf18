"""Minimal SpikingJelly-compatible modules and model builders.

SpikingJelly (the reference's model zoo, pinned at 0.0.0.0.14) is not
installed in this environment.  This module provides the subset of its
``activation_based`` API that CATFuse-SF consumes, with the same attribute
names, so ``catfuse_amd.optimize`` can be exercised on the same module trees
SpikingJelly builds:

* ``LIFNode`` (tau, decay_input, v_threshold, v_reset, step_mode, v, reset())
  running SpikingJelly's eval-mode multi-step recurrence in torch;
* multi-step layer wrappers ``Conv2d``, ``BatchNorm2d``, ``MaxPool2d``,
  ``AvgPool2d``, ``AdaptiveAvgPool2d``, ``Linear``, ``Flatten`` (``[T, B, ...]``
  inputs are flattened to ``[T*B, ...]`` as SpikingJelly's
  ``SeqToANNContainer`` does);
* ``functional.reset_net`` / ``functional.set_step_mode``;
* ``sew_resnet18`` (BasicBlock with conv{1,2}/bn{1,2}/sn{1,2}/downsample/
  downsample_sn/cnf, forward as catfuse/patterns.py:676-689 describes) and
  ``spiking_vgg11_bn`` with AvgPool->LIF at the pools.

These modules are the *unfused input* to the optimizer (the model the user
would have built with SpikingJelly); the fused path never calls them.  When
the real SpikingJelly is importable, ``catfuse_amd.substitute`` accepts its
modules as well (duck-typed on class name and attributes).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F


class MemoryModule(nn.Module):
    """Stateful module with ``reset()`` and a ``step_mode`` ('s' or 'm')."""

    def __init__(self):
        super().__init__()
        self.step_mode = "s"

    def reset(self):
        pass


class LIFNode(MemoryModule):
    """Leaky integrate-and-fire neuron, SpikingJelly semantics (eval path).

    Multi-step charge/fire/reset per step t (SpikingJelly 0.0.0.0.14
    ``LIFNode.jit_eval_multi_step_forward_*``):
      hard reset, decay_input : v = v + (x - (v - v_reset)) / tau
      hard reset, no decay    : v = v - (v - v_reset) / tau + x
      soft reset, decay_input : v = v + (x - v) / tau
      soft reset, no decay    : v = v * (1 - 1/tau) + x
      spike = (v >= v_threshold)
      hard: v = v_reset * spike + (1 - spike) * v ;  soft: v = v - spike * v_threshold
    """

    def __init__(self, tau: float = 2.0, decay_input: bool = True, v_threshold: float = 1.0,
                 v_reset=0.0, surrogate_function=None, detach_reset: bool = False,
                 step_mode: str = "s", backend: str = "torch", store_v_seq: bool = False):
        super().__init__()
        self.tau = float(tau)
        self.decay_input = bool(decay_input)
        self.v_threshold = float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.surrogate_function = surrogate_function
        self.detach_reset = detach_reset
        self.step_mode = step_mode
        self.backend = backend
        self.store_v_seq = store_v_seq
        self.v = 0.0 if self.v_reset is None else self.v_reset

    def reset(self):
        self.v = 0.0 if self.v_reset is None else self.v_reset

    def _charge(self, v, x):
        if self.v_reset is not None:
            if self.decay_input:
                return v + (x - (v - self.v_reset)) / self.tau
            return v - (v - self.v_reset) / self.tau + x
        if self.decay_input:
            return v + (x - v) / self.tau
        return v * (1.0 - 1.0 / self.tau) + x

    def _fire_reset(self, v):
        spike = (v >= self.v_threshold).to(v.dtype)
        if self.v_reset is not None:
            v = self.v_reset * spike + (1.0 - spike) * v
        else:
            v = v - spike * self.v_threshold
        return spike, v

    def _init_v(self, x):
        if not isinstance(self.v, torch.Tensor) or self.v.shape != x.shape or self.v.device != x.device:
            fill = float(self.v) if not isinstance(self.v, torch.Tensor) else (
                0.0 if self.v_reset is None else self.v_reset)
            self.v = torch.full_like(x, fill)

    def forward(self, x):
        if self.step_mode == "m":
            self._init_v(x[0])
            v = self.v
            out = torch.empty_like(x)
            for t in range(x.shape[0]):
                v = self._charge(v, x[t])
                out[t], v = self._fire_reset(v)
            self.v = v
            return out
        self._init_v(x)
        v = self._charge(self.v, x)
        s, self.v = self._fire_reset(v)
        return s

    def extra_repr(self):
        return (f"v_threshold={self.v_threshold}, v_reset={self.v_reset}, tau={self.tau}, "
                f"decay_input={self.decay_input}, step_mode={self.step_mode}")


class _SeqMixin:
    """Flatten [T, B, ...] -> [T*B, ...] around a per-sample module in 'm' mode."""

    def _seq(self, fn, x):
        if getattr(self, "step_mode", "s") == "m":
            T, B = x.shape[0], x.shape[1]
            y = fn(x.flatten(0, 1))
            return y.reshape(T, B, *y.shape[1:])
        return fn(x)


class Conv2d(nn.Conv2d, _SeqMixin):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode

    def forward(self, x):
        return self._seq(super().forward, x)


class BatchNorm2d(nn.BatchNorm2d, _SeqMixin):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode

    def forward(self, x):
        return self._seq(super().forward, x)


class MaxPool2d(nn.MaxPool2d, _SeqMixin):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode

    def forward(self, x):
        return self._seq(super().forward, x)


class AvgPool2d(nn.AvgPool2d, _SeqMixin):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode

    def forward(self, x):
        return self._seq(super().forward, x)


class AdaptiveAvgPool2d(nn.AdaptiveAvgPool2d, _SeqMixin):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode

    def forward(self, x):
        return self._seq(super().forward, x)


class Linear(nn.Linear):
    def __init__(self, *args, step_mode: str = "s", **kw):
        super().__init__(*args, **kw)
        self.step_mode = step_mode


class Flatten(nn.Flatten):
    """Flatten all dims after the batch dims ([T, B, ...] -> [T, B, F] in 'm')."""

    def __init__(self, start_dim: int = 1, end_dim: int = -1, step_mode: str = "s"):
        super().__init__(start_dim, end_dim)
        self.step_mode = step_mode

    def forward(self, x):
        if self.step_mode == "m":
            return torch.flatten(x, 2)
        return super().forward(x)


def _reset_net(net: nn.Module):
    # Every module of net in net.modules() order (pre-order, each once),
    # walked over the _modules dicts directly; a module's reset is found as
    # attribute lookup would find it (instance attribute, class attribute,
    # then a submodule of that name), without nn.Module.__getattr__'s
    # failing lookup for the modules that have none.
    seen = set()
    stack = [net]
    while stack:
        m = stack.pop()
        if id(m) in seen:
            continue
        seen.add(id(m))
        r = m.__dict__.get("reset")
        if r is None and getattr(type(m), "reset", None) is not None:
            r = m.reset
        if r is None:
            r = m._modules.get("reset")
        if r is not None and callable(r):
            r()
        kids = [c for c in m._modules.values() if c is not None]
        kids.reverse()
        stack.extend(kids)


def _set_step_mode(net: nn.Module, step_mode: str):
    for m in net.modules():
        if hasattr(m, "step_mode"):
            m.step_mode = step_mode


functional = SimpleNamespace(reset_net=_reset_net, set_step_mode=_set_step_mode)
neuron = SimpleNamespace(LIFNode=LIFNode)
layer = SimpleNamespace(Conv2d=Conv2d, BatchNorm2d=BatchNorm2d, MaxPool2d=MaxPool2d,
                        AvgPool2d=AvgPool2d, AdaptiveAvgPool2d=AdaptiveAvgPool2d,
                        Linear=Linear, Flatten=Flatten)


# ---------------------------------------------------------------------------
# SEW-ResNet (connect function applied after both LIFs)
# ---------------------------------------------------------------------------

def sew_function(x, y, cnf: str):
    if cnf == "ADD":
        return x + y
    if cnf == "AND":
        return x * y
    if cnf == "IAND":
        return x * (1.0 - y)
    raise NotImplementedError(cnf)


class BasicBlock(nn.Module):
    """SEW-ResNet BasicBlock (attribute names as SpikingJelly's sew_resnet)."""
    expansion = 1

    def __init__(self, inplanes, planes, stride=1, downsample=None, cnf: str = "ADD",
                 spiking_neuron=LIFNode, **kwargs):
        super().__init__()
        self.conv1 = Conv2d(inplanes, planes, 3, stride, 1, bias=False)
        self.bn1 = BatchNorm2d(planes)
        self.sn1 = spiking_neuron(**kwargs)
        self.conv2 = Conv2d(planes, planes, 3, 1, 1, bias=False)
        self.bn2 = BatchNorm2d(planes)
        self.sn2 = spiking_neuron(**kwargs)
        self.downsample = downsample
        if downsample is not None:
            self.downsample_sn = spiking_neuron(**kwargs)
        self.stride = stride
        self.cnf = cnf

    def forward(self, x):
        identity = x
        out = self.sn1(self.bn1(self.conv1(x)))
        out = self.sn2(self.bn2(self.conv2(out)))
        if self.downsample is not None:
            identity = self.downsample_sn(self.downsample(x))
        return sew_function(identity, out, self.cnf)


class SEWResNet(nn.Module):
    def __init__(self, layers=(2, 2, 2, 2), num_classes=1000, cnf="ADD", spiking_neuron=LIFNode,
                 **kwargs):
        super().__init__()
        self.inplanes = 64
        self.conv1 = Conv2d(3, 64, 7, 2, 3, bias=False)
        self.bn1 = BatchNorm2d(64)
        self.sn1 = spiking_neuron(**kwargs)
        self.maxpool = MaxPool2d(3, 2, 1)
        self.layer1 = self._make_layer(64, layers[0], 1, cnf, spiking_neuron, kwargs)
        self.layer2 = self._make_layer(128, layers[1], 2, cnf, spiking_neuron, kwargs)
        self.layer3 = self._make_layer(256, layers[2], 2, cnf, spiking_neuron, kwargs)
        self.layer4 = self._make_layer(512, layers[3], 2, cnf, spiking_neuron, kwargs)
        self.avgpool = AdaptiveAvgPool2d((1, 1))
        self.fc = Linear(512, num_classes)
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_out", nonlinearity="relu")

    def _make_layer(self, planes, blocks, stride, cnf, sn, kwargs):
        downsample = None
        if stride != 1 or self.inplanes != planes:
            downsample = nn.Sequential(Conv2d(self.inplanes, planes, 1, stride, bias=False),
                                       BatchNorm2d(planes))
        layers = [BasicBlock(self.inplanes, planes, stride, downsample, cnf, sn, **kwargs)]
        self.inplanes = planes
        for _ in range(1, blocks):
            layers.append(BasicBlock(self.inplanes, planes, 1, None, cnf, sn, **kwargs))
        return nn.Sequential(*layers)

    def forward(self, x):
        x = self.maxpool(self.sn1(self.bn1(self.conv1(x))))
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        x = self.avgpool(x)
        x = torch.flatten(x, 2) if self.avgpool.step_mode == "m" else torch.flatten(x, 1)
        return self.fc(x)


def sew_resnet18(num_classes=1000, cnf="ADD", spiking_neuron=LIFNode, **kwargs):
    return SEWResNet((2, 2, 2, 2), num_classes, cnf, spiking_neuron, **kwargs)


# ---------------------------------------------------------------------------
# Spiking VGG-11-BN with AvgPool -> LIF at the pools
# ---------------------------------------------------------------------------

VGG11_CFG = (64, "M", 128, "M", 256, 256, "M", 512, 512, "M", 512, 512, "M")


class SpikingVGG(nn.Module):
    """features: Conv-BN-LIF per conv, except that the conv before a pool is
    followed by Conv-BN-AvgPool(2)-LIF; classifier: Linear-LIF, Linear-LIF,
    Linear (CIFAR-size input, 32x32 -> 1x1 after five pools)."""

    def __init__(self, cfg=VGG11_CFG, num_classes=10, spiking_neuron=LIFNode, **kwargs):
        super().__init__()
        mods, cin = [], 3
        for i, c in enumerate(cfg):
            if c == "M":
                continue
            pool_next = i + 1 < len(cfg) and cfg[i + 1] == "M"
            mods += [Conv2d(cin, c, 3, 1, 1, bias=False), BatchNorm2d(c)]
            if pool_next:
                mods.append(AvgPool2d(2, 2))
            mods.append(spiking_neuron(**kwargs))
            cin = c
        self.features = nn.Sequential(*mods)
        self.flatten = Flatten()
        self.classifier = nn.Sequential(
            Linear(512, 4096), spiking_neuron(**kwargs),
            Linear(4096, 4096), spiking_neuron(**kwargs),
            Linear(4096, num_classes))
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_out", nonlinearity="relu")

    def forward(self, x):
        return self.classifier(self.flatten(self.features(x)))


def spiking_vgg11_bn(num_classes=10, spiking_neuron=LIFNode, **kwargs):
    return SpikingVGG(VGG11_CFG, num_classes, spiking_neuron, **kwargs)


# ---------------------------------------------------------------------------
# Spikformer (the structure and module names of the reference's
# models/spikformer_github.py:59-330, multi-step: every LIF runs over T)
# ---------------------------------------------------------------------------

def _linear_bn_lif(x, linear, bn, lif):
    """[T, B, N, C] -> Linear on the last dim -> BatchNorm1d over it -> LIF
    over T (models/spikformer_github.py:126-137)."""
    t, b, n, _ = x.shape
    y = linear(x.flatten(0, 1))
    y = bn(y.transpose(-1, -2)).transpose(-1, -2)
    return lif(y.reshape(t, b, n, -1).contiguous())


class SpikformerMLP(nn.Module):
    def __init__(self, dim, hidden_dim, v_threshold=1.0):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden_dim)
        self.fc1_bn = nn.BatchNorm1d(hidden_dim)
        self.fc1_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")
        self.fc2 = nn.Linear(hidden_dim, dim)
        self.fc2_bn = nn.BatchNorm1d(dim)
        self.fc2_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")
        self.hidden_dim, self.dim = hidden_dim, dim

    def forward(self, x):
        return _linear_bn_lif(_linear_bn_lif(x, self.fc1, self.fc1_bn, self.fc1_lif),
                              self.fc2, self.fc2_bn, self.fc2_lif)


class SpikformerSSA(nn.Module):
    """Spiking self-attention: LIF(BN(Linear)) for q, k, v; ((q k^T) * scale) v
    per head; attn_lif; LIF(BN(proj)) (models/spikformer_github.py:94-160)."""

    def __init__(self, dim, num_heads, v_threshold=1.0, scale=None):
        super().__init__()
        self.dim, self.num_heads = dim, num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5 if scale is None else float(scale)
        for name in ("q", "k", "v"):
            setattr(self, name, nn.Linear(dim, dim))
            setattr(self, name + "_bn", nn.BatchNorm1d(dim))
            setattr(self, name + "_lif", LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m"))
        self.attn_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")
        self.proj = nn.Linear(dim, dim)
        self.proj_bn = nn.BatchNorm1d(dim)
        self.proj_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")

    def forward(self, x):
        t, b, n, c = x.shape
        hd = (t, b, n, self.num_heads, self.head_dim)
        q = _linear_bn_lif(x, self.q, self.q_bn, self.q_lif).reshape(hd).permute(0, 1, 3, 2, 4)
        k = _linear_bn_lif(x, self.k, self.k_bn, self.k_lif).reshape(hd).permute(0, 1, 3, 2, 4)
        v = _linear_bn_lif(x, self.v, self.v_bn, self.v_lif).reshape(hd).permute(0, 1, 3, 2, 4)
        attn = torch.matmul(q, k.transpose(-2, -1).contiguous()) * self.scale
        y = torch.matmul(attn, v.contiguous())
        y = self.attn_lif(y.transpose(2, 3).reshape(t, b, n, c).contiguous())
        return _linear_bn_lif(y, self.proj, self.proj_bn, self.proj_lif)


class SpikformerBlock(nn.Module):
    def __init__(self, dim, num_heads, mlp_ratio=4.0, v_threshold=1.0, scale=None):
        super().__init__()
        self.attn = SpikformerSSA(dim, num_heads, v_threshold, scale)
        self.mlp = SpikformerMLP(dim, int(dim * mlp_ratio), v_threshold)

    def forward(self, x):
        x = x + self.attn(x)
        return x + self.mlp(x)


class SpikformerSPS(nn.Module):
    """Spiking patch splitting: four Conv3x3-BN-LIF stages (embed/8, /4, /2,
    embed channels) with MaxPool2d(3, 2, 1) after the stages in `pools`
    (the reference's CIFAR variant pools after stages 2 and 3; four pools
    give the 14 x 14 tokens of a 224 x 224 image), then the relative
    position Conv-BN-LIF added to its input, as tokens [T, B, N, C]
    (models/spikformer_github.py:181-254)."""

    def __init__(self, in_channels, embed_dim, v_threshold=1.0, pools=(2, 3)):
        super().__init__()
        chans = [in_channels, embed_dim // 8, embed_dim // 4, embed_dim // 2, embed_dim]
        for i in range(4):
            setattr(self, f"conv{i}", nn.Conv2d(chans[i], chans[i + 1], 3, 1, 1, bias=False))
            setattr(self, f"bn{i}", nn.BatchNorm2d(chans[i + 1]))
            setattr(self, f"lif{i}", LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m"))
            setattr(self, f"pool{i}", nn.MaxPool2d(3, 2, 1) if i in pools else None)
        self.rpe_conv = nn.Conv2d(embed_dim, embed_dim, 3, 1, 1, bias=False)
        self.rpe_bn = nn.BatchNorm2d(embed_dim)
        self.rpe_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")

    def forward(self, x):
        t, b = x.shape[:2]
        y = x
        for i in range(4):
            conv, bn, lif = getattr(self, f"conv{i}"), getattr(self, f"bn{i}"), getattr(self, f"lif{i}")
            z = bn(conv(y.flatten(0, 1)))
            y = lif(z.reshape(t, b, *z.shape[1:]).contiguous())
            pool = getattr(self, f"pool{i}")
            if pool is not None:
                p = pool(y.flatten(0, 1))
                y = p.reshape(t, b, *p.shape[1:])
        z = self.rpe_bn(self.rpe_conv(y.flatten(0, 1)))
        y = self.rpe_lif(z.reshape(t, b, *z.shape[1:]).contiguous()) + y
        return y.flatten(-2).transpose(-1, -2).contiguous()


class Spikformer(nn.Module):
    """models/spikformer_github.py:256-330: SPS, `depth` blocks, token
    average, pre-head LIF, linear head; x [T, B, C, H, W] (or [B, C, H, W],
    repeated over T) -> [T, B, num_classes]."""

    def __init__(self, img_size=224, in_channels=3, num_classes=1000, embed_dim=384,
                 num_heads=12, mlp_ratio=4.0, depth=8, T=4, v_threshold=1.0, pools=(0, 1, 2, 3),
                 scale=None):
        super().__init__()
        self.T = int(T)
        self.num_classes = int(num_classes)
        self.patch_embed = SpikformerSPS(in_channels, embed_dim, v_threshold, pools)
        self.blocks = nn.ModuleList([SpikformerBlock(embed_dim, num_heads, mlp_ratio,
                                                     v_threshold, scale) for _ in range(depth)])
        self.pre_head_lif = LIFNode(tau=2.0, v_threshold=v_threshold, step_mode="m")
        self.head = nn.Linear(embed_dim, num_classes)

    def forward_features(self, x):
        y = self.patch_embed(x)
        for blk in self.blocks:
            y = blk(y)
        return y.mean(dim=2)

    def forward(self, x):
        if x.dim() == 4:
            x = x.unsqueeze(0).expand(self.T, *x.shape)
        return self.head(self.pre_head_lif(self.forward_features(x)))


def spikformer_8_384(num_classes=1000, img_size=224, T=4, **kwargs):
    """Config C4: 8 blocks, dim 384, 12 heads (head dim 32), MLP 1536; four
    SPS pools give 14 x 14 = 196 tokens at 224 x 224; attention scale 0.125
    as the config states (the reference module uses head_dim ** -0.5)."""
    kwargs.setdefault("scale", 0.125)
    return Spikformer(img_size=img_size, num_classes=num_classes, embed_dim=384, num_heads=12,
                      mlp_ratio=4.0, depth=8, T=T, **kwargs)


def randomize_bn(model: nn.Module, generator: torch.Generator) -> None:
    """BN running statistics and affine parameters as the benchmark configs
    specify: running_mean ~ N(0, 0.1), running_var ~ U(0.5, 1.5),
    gamma ~ U(0.8, 1.2), beta ~ N(0, 0.1)."""
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.BatchNorm1d, nn.BatchNorm2d)):
                C = m.num_features
                m.running_mean.copy_(torch.randn(C, generator=generator) * 0.1)
                m.running_var.copy_(torch.rand(C, generator=generator) + 0.5)
                m.weight.copy_(torch.rand(C, generator=generator) * 0.4 + 0.8)
                m.bias.copy_(torch.randn(C, generator=generator) * 0.1)


def kaiming_init(model: nn.Module, generator: torch.Generator) -> None:
    """Seeded kaiming-normal conv/linear weights (fan_out, relu gain)."""
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Conv2d, nn.Linear)):
                fan_out = m.weight.shape[0] * (m.weight[0][0].numel() if m.weight.dim() > 2 else 1)
                std = math.sqrt(2.0 / fan_out)
                m.weight.copy_(torch.randn(m.weight.shape, generator=generator) * std)
                if m.bias is not None:
                    m.bias.zero_()
