"""CPU oracle of the CATFuse-SF fused SNN inference path — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the
timed CPU baseline).  The product path (``catfuse_amd``) never imports it.

What it restates (reference = hpcyhr/CATFuse, SpikingJelly 0.0.0.0.14):

* ``lif_multistep``  — SpikingJelly multi-step LIF (eval-mode op order) and
  the reference's fused-tail input currents; plain C (oracle.c).
  Pinned by: hand-derived closed-form sequences (z = 1.5 constant, z = 0
  decay, soft reset, decay_input=False), and an independent torch-fp32
  evaluation of the same op sequence (tests/test_oracle.py).
* ``prescan2d`` — brute-force prescan from the definition (oracle.c) and
  ``prescan2d_maxpool`` — the reference's own max-pool cascade formulation
  (catfuse/sparseflow/prescan.py:32-189) in torch CPU; each pins the other,
  plus the all-zero / all-one / single-spike closed forms.
* ``conv2d`` — torch CPU convolution in float64 (library routine), pinned on
  tiny shapes against the double-precision brute force ``conv2d_bruteforce``;
  grouped convolutions (groups > 1) pinned against ``conv2d_grouped_by_parts``
  (per-group dense convolutions) and the brute force per group.
* ``bn_fold`` / ``batch_norm`` — eval-mode BatchNorm (closed form, and
  torch's F.batch_norm, the routine SpikingJelly's BatchNorm2d calls).
* ``route`` — StaticZero/SparseFlow/DenseKeep decision
  (catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524).
* geometry helpers ``choose_group_size`` (sparse_helpers.py:39-56) and
  ``select_tile_sizes`` (sparse_conv2d_kernel.py:80-84).
* network forwards ``sew_resnet_forward`` / ``vgg_forward`` — module-by-
  module SpikingJelly semantics with the ops above.
* spiking transformer: ``linear_bn_lif`` (float64 linear, torch eval BN,
  C LIF; pinned against ``conv_bn_lif`` with a 1x1 conv over the token grid,
  an independent formulation), ``spike_attention_lif`` (float64 torch
  matmuls in the reference's order; pinned against
  ``spike_attention_bruteforce``, the definition in Python loops, and the
  integer identity (Q K^T) V = Q (K^T V)) and ``spikformer_forward``.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_int64, c_void_p

import numpy as np
import torch
import torch.nn.functional as F

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        src = os.path.join(_HERE, "oracle.c")
        if not os.path.exists(path) or os.path.getmtime(path) < os.path.getmtime(src):
            from oracle.build import build
            build()
        lib = ctypes.CDLL(path)
        P, I = c_void_p, c_int64
        lib.oracle_lif_multistep.argtypes = [P, P, P, P, c_int, P, P, P, P, I, I, I, I,
                                             c_double, c_double, c_double, c_int, c_int]
        lib.oracle_lif_multistep.restype = None
        lib.oracle_prescan2d.argtypes = [P, I, I, I, I, I, I, I, I, I, I, I, I, c_float, P, P]
        lib.oracle_prescan2d.restype = None
        lib.oracle_conv2d_f64.argtypes = [P, P, P, I, I, I, I, I, I, I, I, I]
        lib.oracle_conv2d_f64.restype = None
        _LIB = lib
    return _LIB


def _f32(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


# ---------------------------------------------------------------------------
# LIF
# ---------------------------------------------------------------------------

def lif_multistep(z, v_in=None, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True,
                  mode=0, z2=None, scale=None, shift=None, C=1, HW=1):
    """z: [T, ...] fp32.  Returns (spikes [T, ...], v_final [...], h [T, ...])
    where h is the charged potential before fire/reset at every step."""
    z = _f32(z)
    T = z.shape[0]
    N = int(np.prod(z.shape[1:])) if z.ndim > 1 else 1
    z2a = _f32(z2) if z2 is not None else None
    sca = _f32(scale) if scale is not None else None
    sha = _f32(shift) if shift is not None else None
    vin = _f32(v_in).reshape(-1) if v_in is not None else None
    spike = np.empty_like(z)
    h = np.empty_like(z)
    v_out = np.empty(N, dtype=np.float32)
    hard = v_reset is not None
    _lib().oracle_lif_multistep(_p(z), _p(z2a), _p(sca), _p(sha), int(mode), _p(vin),
                                _p(spike), _p(v_out), _p(h), T, N, int(C), int(HW),
                                float(tau), float(v_threshold),
                                float(v_reset) if hard else 0.0, int(hard), int(bool(decay_input)))
    return spike, v_out.reshape(z.shape[1:]), h


# ---------------------------------------------------------------------------
# Prescan geometry and masks
# ---------------------------------------------------------------------------

TILE_ZERO, TILE_SPARSE, TILE_DENSEISH = 0, 1, 2


def choose_group_size(k_dim: int) -> int:
    """GS = 16 if k <= 128 else 32, doubled until at most 32 groups
    (catfuse/sparseflow/sparse_helpers.py:39-56)."""
    gs = 16 if k_dim <= 128 else 32
    while (k_dim + gs - 1) // gs > 32:
        gs *= 2
    return gs


def select_tile_sizes(H: int, W: int):
    """8x16 output tiles if H*W >= 3136 else 8x8
    (catfuse/sparseflow/sparse_conv2d_kernel.py:80-84)."""
    return (8, 16) if H * W >= 3136 else (8, 8)


def prescan2d(x, H_out, W_out, kernel_size=3, stride=1, padding=1, block_h=8, block_w=16,
              group_size_c=16, threshold=1e-6):
    """Brute-force prescan (oracle.c).  x: [N, C, H, W].  Returns
    (tile_class int32 [N*GH*GW], ag_mask int32 [N*GH*GW])."""
    x = _f32(x)
    N, C, H, W = x.shape
    GH, GW = -(-H_out // block_h), -(-W_out // block_w)
    ag = np.empty(N * GH * GW, dtype=np.int32)
    tc = np.empty(N * GH * GW, dtype=np.int32)
    _lib().oracle_prescan2d(_p(x), N, C, H, W, H_out, W_out, kernel_size, stride, padding,
                            block_h, block_w, group_size_c, float(threshold), _p(ag), _p(tc))
    return tc, ag


def prescan2d_maxpool(x, H_out, W_out, kernel_size=3, stride=1, padding=1, block_h=8,
                      block_w=16, group_size_c=16, threshold=1e-6):
    """The reference's formulation (catfuse/sparseflow/prescan.py:32-189):
    channel-group amax of |x| -> max_pool2d over the receptive field ->
    ceil-mode max_pool2d over the tile -> `> threshold` -> bit packing."""
    xt = torch.as_tensor(_f32(x))
    N, C, H, W = xt.shape
    G = -(-C // group_size_c)
    xl = xt.permute(0, 2, 3, 1)
    if C < G * group_size_c:
        xl = F.pad(xl, (0, G * group_size_c - C))
    gmax = xl.abs().reshape(N, H, W, G, group_size_c).amax(-1).permute(0, 3, 1, 2).contiguous()
    if kernel_size == 1 and stride == 1 and padding == 0:
        rf = gmax
    else:
        rf = F.max_pool2d(gmax, kernel_size, stride, padding)
    assert tuple(rf.shape[-2:]) == (H_out, W_out)
    tile = F.max_pool2d(rf, (block_h, block_w), (block_h, block_w), ceil_mode=True)
    act = (tile > float(threshold)).permute(0, 2, 3, 1).to(torch.int64)  # [N, GH, GW, G]
    weights = torch.tensor([1 << g for g in range(G)], dtype=torch.int64)
    ag = (act * weights).sum(-1).reshape(-1)
    ag = ((ag + 2 ** 31) % 2 ** 32 - 2 ** 31).to(torch.int32)
    anyv = act.any(-1).reshape(-1)
    allv = act.all(-1).reshape(-1)
    tc = torch.full_like(ag, TILE_SPARSE)
    tc[~anyv] = TILE_ZERO
    tc[allv] = TILE_DENSEISH
    return tc.numpy(), ag.numpy()


def route(x, sparse_threshold=0.7):
    """0 StaticZero if nnz == 0, 1 SparseFlow if sparsity > threshold, else 2
    DenseKeep (catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524)."""
    x = _f32(x)
    nnz = int(np.count_nonzero(x))
    if nnz == 0:
        return 0
    return 1 if (1.0 - nnz / x.size) > sparse_threshold else 2


# ---------------------------------------------------------------------------
# Conv / BN
# ---------------------------------------------------------------------------

def conv2d(x, w, bias=None, stride=1, padding=0, dtype=torch.float64, groups=1):
    """torch CPU convolution in `dtype` (default float64), result as fp32;
    groups > 1 is a grouped convolution (weight [Cout, Cin/groups, k, k])."""
    xt = torch.as_tensor(_f32(x)).to(dtype)
    wt = torch.as_tensor(_f32(w)).to(dtype)
    bt = None if bias is None else torch.as_tensor(_f32(bias)).to(dtype)
    return F.conv2d(xt, wt, bt, stride=stride, padding=padding,
                    groups=groups).to(torch.float32)


def conv2d_grouped_by_parts(x, w, bias=None, stride=1, padding=0, groups=1):
    """A grouped convolution as `groups` independent dense convolutions (the
    reference's formulation, catfuse/sparseflow/sparse_grouped_conv2d_kernel.py:
    251-288), each through conv2d with groups = 1, concatenated over the
    output channels."""
    xt = torch.as_tensor(_f32(x))
    wt = torch.as_tensor(_f32(w))
    cin_g = xt.shape[1] // groups
    cout_g = wt.shape[0] // groups
    parts = []
    for g in range(groups):
        b = None if bias is None else torch.as_tensor(_f32(bias))[g * cout_g:(g + 1) * cout_g]
        parts.append(conv2d(xt[:, g * cin_g:(g + 1) * cin_g], wt[g * cout_g:(g + 1) * cout_g], b,
                            stride, padding))
    return torch.cat(parts, 1)


def conv2d_bruteforce(x, w, stride=1, padding=0):
    x = _f32(x)
    w = _f32(w)
    N, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    Ho, Wo = (H + 2 * padding - KH) // stride + 1, (W + 2 * padding - KW) // stride + 1
    y = np.empty((N, Cout, Ho, Wo), dtype=np.float32)
    _lib().oracle_conv2d_f64(_p(x), _p(w), _p(y), N, Cin, H, W, Cout, KH, KW, stride, padding)
    return y


def bn_fold(gamma, beta, mean, var, eps=1e-5):
    """scale = gamma / sqrt(var + eps); shift = beta - mean * scale (fp32)
    (catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:70-88)."""
    g, b, m, v = (torch.as_tensor(_f32(a)) for a in (gamma, beta, mean, var))
    scale = g * (1.0 / torch.sqrt(v + eps))
    return scale, b - m * scale


def batch_norm(z, bn):
    """Eval BatchNorm2d on [N, C, H, W] with torch's CPU routine."""
    return F.batch_norm(z, bn.running_mean.detach().cpu().float(),
                        bn.running_var.detach().cpu().float(),
                        None if bn.weight is None else bn.weight.detach().cpu().float(),
                        None if bn.bias is None else bn.bias.detach().cpu().float(),
                        False, 0.0, bn.eps)


# ---------------------------------------------------------------------------
# Layer-level and network-level references
# ---------------------------------------------------------------------------

def lif_params_of(lif):
    return dict(tau=float(getattr(lif, "tau", 2.0)), v_threshold=float(lif.v_threshold),
                v_reset=None if lif.v_reset is None else float(lif.v_reset),
                decay_input=bool(getattr(lif, "decay_input", True)))


def conv_bn_lif(x_seq, conv, bn, lif, v_in=None, conv_dtype=torch.float64):
    """SpikingJelly Conv2d -> BatchNorm2d -> LIFNode on [T, B, C, H, W]:
    conv (fp64 by default, rounded to fp32), torch eval BN, C LIF.
    Returns (spikes, v_final, h) as numpy fp32."""
    x_seq = torch.as_tensor(_f32(x_seq))
    T, B = x_seq.shape[:2]
    z = conv2d(x_seq.flatten(0, 1), conv.weight, conv.bias, conv.stride[0], conv.padding[0],
               dtype=conv_dtype, groups=getattr(conv, "groups", 1))
    if bn is not None:
        z = batch_norm(z, bn)
    z = z.reshape(T, B, *z.shape[1:])
    return lif_multistep(z, v_in, **lif_params_of(lif))


def _lif_t(x, lif):
    s, _, _ = lif_multistep(x, None, **lif_params_of(lif))
    return torch.from_numpy(s)


def sew_resnet_forward(model, x_seq, conv_dtype=torch.float64, record=None):
    """SEW-ResNet forward on CPU in SpikingJelly multi-step semantics.

    x_seq: [T, B, 3, H, W].  Mirrors SEWResNet/BasicBlock.forward
    (out = sew(identity, sn2(bn2(conv2(sn1(bn1(conv1(x))))))), with
    identity = downsample_sn(downsample(x)) when present;
    catfuse/patterns.py:676-689).  `record`, if a dict, receives every LIF
    layer's (input, spikes, charged potential h) keyed by the module path of
    its conv ("conv1", "layer1.0.conv1", "layer2.0.downsample", ...)."""
    T, B = x_seq.shape[:2]

    def cbl(name, x, conv, bn, lif):
        s, _, h = conv_bn_lif(x, conv, bn, lif, conv_dtype=conv_dtype)
        s = torch.from_numpy(s)
        if record is not None:
            record[name] = (x, s, h)
        return s

    x = cbl("conv1", x_seq, model.conv1, model.bn1, model.sn1)
    mp = model.maxpool
    x = F.max_pool2d(x.flatten(0, 1), mp.kernel_size, mp.stride, mp.padding)
    x = x.reshape(T, B, *x.shape[1:])
    for li in range(1, 5):
        for bi, blk in enumerate(getattr(model, f"layer{li}")):
            p = f"layer{li}.{bi}"
            out = cbl(p + ".conv1", x, blk.conv1, blk.bn1, blk.sn1)
            out = cbl(p + ".conv2", out, blk.conv2, blk.bn2, blk.sn2)
            identity = x
            if blk.downsample is not None:
                identity = cbl(p + ".downsample", x, blk.downsample[0], blk.downsample[1],
                               blk.downsample_sn)
            if blk.cnf == "ADD":
                x = identity + out
            elif blk.cnf == "AND":
                x = identity * out
            else:
                x = identity * (1.0 - out)
    x = x.mean(dim=(3, 4))  # AdaptiveAvgPool2d((1,1)) + flatten(2)
    w = model.fc.weight.detach().cpu().double()
    b = model.fc.bias.detach().cpu().double() if model.fc.bias is not None else None
    y = F.linear(x.double(), w, b)
    return y.float()


def vgg_forward(model, x_seq, conv_dtype=torch.float64, record=None):
    """Spiking VGG forward on CPU in SpikingJelly multi-step semantics.

    x_seq: [T, B, 3, H, W].  `model.features` is read as runs of Conv2d ->
    BatchNorm2d -> [AvgPool2d(2, 2)] -> LIFNode (the AvgPool -> LIF tail of
    catfuse/kernels/avgpool_lif.py:193-206 when present); then flatten and
    `model.classifier` as Linear -> LIFNode pairs and a final Linear (linears
    in float64 rounded to fp32, as linear_bn_lif).  `record`, if a dict,
    receives (input, spikes, h) per LIF layer keyed "features.<i>" (i the
    conv's index) and "classifier.<j>" (j the linear's index)."""
    T, B = x_seq.shape[:2]
    x = torch.as_tensor(_f32(x_seq))
    feats = list(model.features)
    i = 0
    while i < len(feats):
        conv, bn = feats[i], feats[i + 1]
        if not (isinstance(conv, torch.nn.Conv2d) and isinstance(bn, torch.nn.BatchNorm2d)):
            raise ValueError(f"features.{i}: expected Conv2d -> BatchNorm2d")
        j = i + 2
        z = batch_norm(conv2d(x.flatten(0, 1), conv.weight, conv.bias, conv.stride[0],
                              conv.padding[0], dtype=conv_dtype), bn)
        if isinstance(feats[j], torch.nn.AvgPool2d):
            z = F.avg_pool2d(z, feats[j].kernel_size, feats[j].stride)
            j += 1
        s, _, h = lif_multistep(z.reshape(T, B, *z.shape[1:]), None, **lif_params_of(feats[j]))
        s = torch.from_numpy(s)
        if record is not None:
            record[f"features.{i}"] = (x, s, h)
        x = s
        i = j + 1
    x = x.flatten(2)
    cls = list(model.classifier)
    j = 0
    while j < len(cls):
        lin = cls[j]
        w = lin.weight.detach().cpu().double()
        b = None if lin.bias is None else lin.bias.detach().cpu().double()
        z = F.linear(x.double(), w, b).float()
        if j + 1 < len(cls) and not isinstance(cls[j + 1], torch.nn.Linear):
            s, _, h = lif_multistep(z, None, **lif_params_of(cls[j + 1]))
            s = torch.from_numpy(s)
            if record is not None:
                record[f"classifier.{j}"] = (x, s, h)
            x = s
            j += 2
        else:
            return z
    return x


# ---------------------------------------------------------------------------
# Spiking transformer (Spikformer, config C4)
# ---------------------------------------------------------------------------

def linear_bn_lif(x_seq, linear, bn, lif, v_in=None):
    """Linear -> BatchNorm1d (eval, over the feature dim) -> LIF on token
    tensors [T, B, N, I] (models/spikformer_github.py:126-137): the linear in
    float64 rounded to fp32, torch's eval batch norm, C LIF over T.
    Returns (spikes, v_final, h) as numpy fp32, [T, B, N, O] / [B, N, O]."""
    x = torch.as_tensor(_f32(x_seq))
    O = linear.out_features
    w = linear.weight.detach().cpu().double()
    b = None if linear.bias is None else linear.bias.detach().cpu().double()
    z = F.linear(x.double(), w, b).float()
    if bn is not None:
        z = batch_norm(z.reshape(-1, O), bn).reshape(z.shape)
    return lif_multistep(z, v_in, **lif_params_of(lif))


def spike_attention_lif(q, k, v, heads, scale, lif, v_in=None):
    """Spikformer's attention core in float64: per head
    ((q k^T) * scale) v, then LIF over T (models/spikformer_github.py:150-156).
    q, k, v: [T, B, N, C] spikes.  Returns (spikes, v_final, h), numpy fp32."""
    q, k, v = (torch.as_tensor(_f32(a)).double() for a in (q, k, v))
    T, B, N, C = q.shape
    dh = C // heads

    def split(a):
        return a.reshape(T, B, N, heads, dh).permute(0, 1, 3, 2, 4)
    attn = torch.matmul(split(q), split(k).transpose(-1, -2)) * scale
    y = torch.matmul(attn, split(v)).permute(0, 1, 3, 2, 4).reshape(T, B, N, C).float()
    return lif_multistep(y, v_in, **lif_params_of(lif))


def spike_attention_bruteforce(q, k, v, heads, scale):
    """The attention product from the definition with Python loops (tiny
    inputs): y[t, b, n, h*dh + j] = sum_m (sum_i q[n, i] k[m, i]) * scale * v[m, j]."""
    q, k, v = (np.asarray(_f32(a), dtype=np.float64) for a in (q, k, v))
    T, B, N, C = q.shape
    dh = C // heads
    y = np.zeros((T, B, N, C))
    for t in range(T):
        for b in range(B):
            for h in range(heads):
                sl = slice(h * dh, (h + 1) * dh)
                for n in range(N):
                    for m in range(N):
                        a = float(np.dot(q[t, b, n, sl], k[t, b, m, sl])) * scale
                        y[t, b, n, sl] += a * v[t, b, m, sl]
    return y


def spikformer_forward(model, x_seq, conv_dtype=torch.float64, record=None):
    """Spikformer forward on CPU in SpikingJelly multi-step semantics
    (models/spikformer_github.py:162-330 with every LIF over T): SPS stages
    Conv-BN-LIF (+ MaxPool), rpe Conv-BN-LIF + its input, tokens; blocks
    x + SSA(x), x + MLP(x); token mean, pre-head LIF, head (float64).
    `record`, if a dict, receives (input, LIF spikes, charged potential h)
    per LIF layer (the rpe conv's and the residual layers' spikes before
    their add; "attn.qkv" the three concatenated)."""
    T, B = x_seq.shape[:2]
    sps = model.patch_embed

    def rec(name, x, s, h):
        """Record (input, the LIF's spikes, its charged potential h); return
        the spikes as a tensor."""
        s = torch.from_numpy(s) if isinstance(s, np.ndarray) else s
        if record is not None:
            record[name] = (x, s, h)
        return s

    y = torch.as_tensor(_f32(x_seq))
    for i in range(4):
        s, _, h = conv_bn_lif(y, getattr(sps, f"conv{i}"), getattr(sps, f"bn{i}"),
                              getattr(sps, f"lif{i}"), conv_dtype=conv_dtype)
        s = rec(f"patch_embed.conv{i}", y, s, h)
        pool = getattr(sps, f"pool{i}", None)
        if pool is not None:
            p = F.max_pool2d(s.flatten(0, 1), pool.kernel_size, pool.stride, pool.padding)
            s = p.reshape(T, B, *p.shape[1:])
        y = s
    r, _, h = conv_bn_lif(y, sps.rpe_conv, sps.rpe_bn, sps.rpe_lif, conv_dtype=conv_dtype)
    r = rec("patch_embed.rpe_conv", y, r, h) + y
    x = r.flatten(-2).transpose(-1, -2).contiguous()
    for bi, blk in enumerate(model.blocks):
        a, m = blk.attn, blk.mlp
        p = f"blocks.{bi}"
        outs = [linear_bn_lif(x, getattr(a, n), getattr(a, n + "_bn"), getattr(a, n + "_lif"))
                for n in ("q", "k", "v")]
        qkv = [torch.from_numpy(o[0]) for o in outs]
        rec(p + ".attn.qkv", x, torch.cat(qkv, -1), np.concatenate([o[2] for o in outs], -1))
        s, _, h = spike_attention_lif(*qkv, a.num_heads, a.scale, a.attn_lif)
        att = rec(p + ".attn.core", torch.cat(qkv, -1), s, h)
        s, _, h = linear_bn_lif(att, a.proj, a.proj_bn, a.proj_lif)
        x = x + rec(p + ".attn.proj", att, s, h)
        s, _, h = linear_bn_lif(x, m.fc1, m.fc1_bn, m.fc1_lif)
        hid = rec(p + ".mlp.fc1", x, s, h)
        s, _, h = linear_bn_lif(hid, m.fc2, m.fc2_bn, m.fc2_lif)
        x = x + rec(p + ".mlp.fc2", hid, s, h)
    f = x.mean(dim=2)
    s = torch.from_numpy(lif_multistep(f, None, **lif_params_of(model.pre_head_lif))[0])
    w = model.head.weight.detach().cpu().double()
    b = None if model.head.bias is None else model.head.bias.detach().cpu().double()
    return F.linear(s.double(), w, b).float()
