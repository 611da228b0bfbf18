"""Module-tree rewrite: SpikingJelly model -> fused patterns.

Mirrors catfuse/substitute.py:123-813:
  * `substitute(model)` — block-level rewrite (SEW / spiking BasicBlock and
    Bottleneck -> CTF* blocks) plus Sequential (Conv, BN, LIF), (Conv, LIF),
    (Linear, LIF) triples/pairs;
  * `substitute_sf(model, T, verbose, force_sparse)` — policy-aware rewrite
    of conv{i}/bn{i}/sn{i} attributes, downsample + downsample_sn, X/X_bn/X_lif
    and conv{i}/bn{i}/lif{i} names, and Sequential patterns, routing 3x3/s1
    layers in the SparseFlow regime to STFusionConvBNLIF;
  * `print_routing_table`, `print_coverage_report`.
Both return (deep-copied fused model, stats) with the reference's stats keys.

Additions: Sequential (Conv, BN, AvgPool2d(2), LIF) and (AvgPool2d(2), LIF)
become PartialFusionConvBNAvgPoolLIF / FusedAvgPoolLIF; with fuse_sew_add
(default) a SEW BasicBlock whose convs were all fused is wrapped into
CTFSEWBasicBlock so its ADD runs in the second conv's epilogue.  The routing
label records the backend actually built (the reference labels stride-2
layers "SparseFlow" although it builds PartialFusionConvBNLIF,
substitute.py:401-418).
"""
from __future__ import annotations

import copy
import warnings

import torch.nn as nn

from catfuse_amd.transformer import (CTFSpikformerBlock, CTFSpikformerSPS, is_spikformer_block,
                                     is_spikformer_sps)
from catfuse_amd.patterns import (CTFSEWBasicBlock, CTFSEWBottleneck, CTFSpikingBasicBlock,
                                  CTFSpikingBottleneck, FusedAvgPoolLIF, FusedFlatten,
                                  FusedGlobalAvgPool, FusedLIF, FusedLinear, FusedLinearLIF,
                                  PartialFusionConvBNAvgPoolLIF, PartialFusionConvBNLIF,
                                  PartialFusionConvBNLIFMaxPool, PartialFusionConvLIF,
                                  PartialFusionGroupedConvBNLIF, STFusionConvBNLIF, conv_geometry,
                                  conv_unsupported_reason, grouped_conv_supported, is_lif_node)
from catfuse_amd.policy import SpatialBackend, get_policy


def _is_sj_conv2d(m) -> bool:
    """An nn.Conv2d the fused kernels compute (conv_unsupported_reason:
    groups, dilation, padding mode and non-square geometry are refused)."""
    return isinstance(m, nn.Conv2d) and conv_unsupported_reason(m) is None


def _is_grouped_conv(m) -> bool:
    """A grouped / depthwise nn.Conv2d the fused grouped kernel computes."""
    return isinstance(m, nn.Conv2d) and grouped_conv_supported(m)


def _is_fusable_conv(m) -> bool:
    """The conv of a Conv -> BN -> LIF triple: dense or grouped."""
    return _is_sj_conv2d(m) or _is_grouped_conv(m)


def _record_unsupported_convs(model, stats) -> None:
    """List every nn.Conv2d left in the rewritten model that the fused
    kernels cannot compute, with the reason, in stats['unsupported_structures']."""
    lst = stats.setdefault("unsupported_structures", [])
    for name, m in model.named_modules():
        if isinstance(m, nn.Conv2d):
            why = conv_unsupported_reason(m)
            if why is not None:
                lst.append(f"{_strip_root(name)}: Conv2d with {why} (left unfused)")


def _is_sj_bn2d(m) -> bool:
    return isinstance(m, nn.BatchNorm2d)


def _is_sj_linear(m) -> bool:
    return isinstance(m, nn.Linear)


def _is_avgpool2(m) -> bool:
    if not isinstance(m, nn.AvgPool2d):
        return False
    k = m.kernel_size if isinstance(m.kernel_size, int) else m.kernel_size[0]
    s = m.stride if isinstance(m.stride, int) else (m.stride[0] if m.stride else k)
    p = m.padding if isinstance(m.padding, int) else m.padding[0]
    return k == 2 and s == 2 and p == 0


def _is_maxpool_321(m) -> bool:
    if not isinstance(m, nn.MaxPool2d):
        return False
    one = lambda v: v if isinstance(v, int) else v[0]  # noqa: E731
    st = m.stride if m.stride is not None else m.kernel_size
    return ((one(m.kernel_size), one(st), one(m.padding), one(m.dilation)) == (3, 2, 1, 1)
            and not m.ceil_mode)


def _is_resnet_stem_owner(m) -> bool:
    """SpikingJelly's SEWResNet / SpikingResNet (or the catfuse_amd.snn
    stand-ins), whose forward applies conv1 -> bn1 -> sn1 -> maxpool in that
    order and uses maxpool nowhere else."""
    return (type(m).__name__ in ("SEWResNet", "SpikingResNet")
            and _is_sj_conv2d(getattr(m, "conv1", None)) and _is_sj_bn2d(getattr(m, "bn1", None))
            and _is_lif(getattr(m, "sn1", None)) and _is_maxpool_321(getattr(m, "maxpool", None)))


def _is_lif(m) -> bool:
    """SpikingJelly LIFNode or the catfuse_amd.snn stand-in (duck-typed)."""
    return is_lif_node(m)


def _block_fusable(m, n_convs: int, sew: bool) -> bool:
    """Every conv{i} / bn{i} / sn{i} site of a ResNet block (and its
    downsample) is a conv the fused kernels compute, a BatchNorm2d and an
    LIF neuron, so the whole block can be replaced."""
    for i in range(1, n_convs + 1):
        if not (_is_sj_conv2d(getattr(m, f"conv{i}", None))
                and _is_sj_bn2d(getattr(m, f"bn{i}", None))
                and _is_lif(getattr(m, f"sn{i}", None))):
            return False
    ds = getattr(m, "downsample", None)
    if ds is not None:
        if not (isinstance(ds, nn.Sequential) and len(ds) >= 2 and _is_sj_conv2d(ds[0])
                and _is_sj_bn2d(ds[1])):
            return False
        if sew and not _is_lif(getattr(m, "downsample_sn", None)):
            return False
    return True


def _is_sew_basic_block(m) -> bool:
    return (type(m).__name__ == "BasicBlock" and getattr(m, "cnf", None) is not None
            and _block_fusable(m, 2, True))


def _is_standard_spiking_basic_block(m) -> bool:
    return (type(m).__name__ == "BasicBlock" and not hasattr(m, "cnf")
            and _block_fusable(m, 2, False))


def _is_sew_bottleneck(m) -> bool:
    return (type(m).__name__ == "Bottleneck" and getattr(m, "cnf", None) is not None
            and _block_fusable(m, 3, True))


def _is_standard_spiking_bottleneck(m) -> bool:
    return (type(m).__name__ == "Bottleneck" and not hasattr(m, "cnf")
            and _block_fusable(m, 3, False))


def _count_lif(model):
    return sum(1 for _, m in model.named_modules() if _is_lif(m))


def _bump(stats, pattern):
    stats["patterns_matched"][pattern] = stats["patterns_matched"].get(pattern, 0) + 1


# ---------------------------------------------------------------------------
# substitute (block-level)
# ---------------------------------------------------------------------------

class _SequentialRewriteResult:
    def __init__(self):
        self.new_modules = []
        self.skipped_indices = []
        self.replacements = []


def _rewrite_sequential(seq: nn.Sequential):
    result = _SequentialRewriteResult()
    ch = list(seq)
    n, i, out = len(ch), 0, []
    while i < n:
        if i + 3 < n and _is_sj_conv2d(ch[i]) and _is_sj_bn2d(ch[i + 1]) and \
                _is_avgpool2(ch[i + 2]) and _is_lif(ch[i + 3]):
            out.append(PartialFusionConvBNAvgPoolLIF.from_sj_modules(*ch[i:i + 4]))
            result.replacements.append(("PartialFusionConvBNAvgPoolLIF", tuple(range(i, i + 4))))
            i += 4
            continue
        if i + 2 < n and _is_fusable_conv(ch[i]) and _is_sj_bn2d(ch[i + 1]) and _is_lif(ch[i + 2]):
            cls = (PartialFusionGroupedConvBNLIF if _is_grouped_conv(ch[i])
                   else PartialFusionConvBNLIF)
            out.append(cls.from_sj_modules(*ch[i:i + 3]))
            result.replacements.append((cls.__name__, (i, i + 1, i + 2)))
            i += 3
            continue
        if i + 1 < n and _is_sj_conv2d(ch[i]) and _is_lif(ch[i + 1]):
            out.append(PartialFusionConvLIF.from_sj_modules(ch[i], ch[i + 1]))
            result.replacements.append(("PartialFusionConvLIF", (i, i + 1)))
            i += 2
            continue
        if i + 1 < n and _is_sj_linear(ch[i]) and _is_lif(ch[i + 1]):
            out.append(FusedLinearLIF.from_sj_modules(ch[i], ch[i + 1]))
            result.replacements.append(("FusedLinearLIF", (i, i + 1)))
            i += 2
            continue
        if i + 1 < n and _is_avgpool2(ch[i]) and _is_lif(ch[i + 1]):
            out.append(FusedAvgPoolLIF.from_sj_modules(ch[i], ch[i + 1]))
            result.replacements.append(("FusedAvgPoolLIF", (i, i + 1)))
            i += 2
            continue
        if _head_linear(ch, i, out):
            out.append(FusedLinear.from_sj_modules(ch[i]))
            result.replacements.append(("FusedLinear", (i,)))
            i += 1
            continue
        out.append(ch[i])
        result.skipped_indices.append(i)
        i += 1
    result.new_modules = out
    return nn.Sequential(*out), result


def substitute(sj_model: nn.Module, verbose: bool = False):
    holder = _Root(copy.deepcopy(sj_model))
    model = holder
    stats = {"total_lif_nodes": _count_lif(model), "fused_lif_nodes": 0, "patterns_matched": {},
             "substituted_sequentials": [], "unsupported_structures": []}

    def walk(parent, ppath=""):
        for name, child in list(parent.named_children()):
            raw = f"{ppath}.{name}" if ppath else name
            path = _strip_root(raw)
            for pred, cls, tag, nlif in (
                    (_is_sew_basic_block, CTFSEWBasicBlock, "SEWBasicBlock",
                     lambda c: 3 if c.downsample is not None else 2),
                    (_is_standard_spiking_basic_block, CTFSpikingBasicBlock, "SpikingBasicBlock",
                     lambda c: 2),
                    (_is_sew_bottleneck, CTFSEWBottleneck, "SEWBottleneck",
                     lambda c: 4 if c.downsample is not None else 3),
                    (_is_standard_spiking_bottleneck, CTFSpikingBottleneck, "SpikingBottleneck",
                     lambda c: 3)):
                if pred(child):
                    setattr(parent, name, cls.from_sj_block(child))
                    _bump(stats, cls.__name__)
                    stats["fused_lif_nodes"] += nlif(child)
                    stats["substituted_sequentials"].append(f"{path}:{tag}")
                    if verbose:
                        print(f"  [substitute] {path}: {cls.__name__}")
                    break
            else:
                if isinstance(child, nn.Sequential):
                    new_seq, res = _rewrite_sequential(child)
                    if res.replacements:
                        setattr(parent, name, new_seq)
                        stats["substituted_sequentials"].append(path)
                        for pat, idx in res.replacements:
                            _bump(stats, pat)
                            stats["fused_lif_nodes"] += 1
                            if verbose:
                                print(f"  [substitute] {path}: {pat} @ indices {idx}")
                    else:
                        walk(child, raw)
                else:
                    walk(child, raw)

    walk(model)
    _record_unsupported_convs(model, stats)
    stats["coverage_pct"] = (100.0 * stats["fused_lif_nodes"] / stats["total_lif_nodes"]
                             if stats["total_lif_nodes"] else 0.0)
    return holder.root, stats


def print_coverage_report(stats: dict, title: str = "Coverage report"):
    print(f"\n{'=' * 70}\n{title}\n{'=' * 70}")
    print(f"  total LIF nodes      : {stats['total_lif_nodes']}")
    print(f"  fused LIF nodes      : {stats['fused_lif_nodes']}")
    print(f"  coverage             : {stats['coverage_pct']:.2f}%")
    print("\n  patterns matched:")
    for p, c in sorted(stats["patterns_matched"].items()):
        print(f"    {p:<30} {c} instance(s)")
    for key, label in (("substituted_sequentials", "substituted sequentials"),
                       ("unsupported_structures", "unsupported structures")):
        if stats.get(key):
            print(f"\n  {label}:")
            for s in stats[key]:
                print(f"    {s}")


# ---------------------------------------------------------------------------
# substitute_sf (policy-aware)
# ---------------------------------------------------------------------------

def _estimate_h(cin):
    """The reference routes without the real feature-map size: H_est = 32 for
    C_in <= 64, 16 for C_in <= 128, else 8 (substitute.py:395)."""
    return 32 if cin <= 64 else (16 if cin <= 128 else 8)


def _build_conv_bn_lif(c, b, l, T, force_sparse, hwprof):
    cin, cout = c.in_channels, c.out_channels
    if _is_grouped_conv(c):
        fused = PartialFusionGroupedConvBNLIF.from_sj_modules(c, b, l)
        return fused, {"pattern": "PartialFusionGroupedConvBNLIF",
                       "shape": f"{cin}->{cout}, k={fused.kernel_size}, s={fused.stride}, "
                                f"groups={fused.groups}",
                       "backend": SpatialBackend.DENSE_KEEP, "K": T}
    k, s, _ = conv_geometry(c)
    h = _estimate_h(cin)
    row = get_policy("Conv3x3_BN_LIF", C_in=cin, C_out=cout, H=h, W=h, kernel_size=k, T=T,
                     hwprof=hwprof)
    use_sparse = force_sparse or row.spatial_backend == SpatialBackend.SPARSE_FLOW
    if use_sparse and k == 3 and s == 1:
        b.eval()
        fused = STFusionConvBNLIF.from_sj_modules(c, b, l, K=row.K)
        pattern, backend = "STFusionConvBNLIF", SpatialBackend.SPARSE_FLOW
    else:
        fused = PartialFusionConvBNLIF.from_sj_modules(c, b, l)
        pattern, backend = "PartialFusionConvBNLIF", SpatialBackend.DENSE_KEEP
    entry = {"pattern": pattern, "shape": f"{cin}->{cout}, k={k}, s={s}", "backend": backend,
             "K": row.K}
    return fused, entry


class _Root(nn.Module):
    """Holder that lets a root-level nn.Sequential be rewritten like a child."""

    def __init__(self, root):
        super().__init__()
        self.root = root


def _strip_root(name: str) -> str:
    if name == "root":
        return "<root>"
    return name[len("root."):] if name.startswith("root.") else name


def substitute_sf(sj_model, T=16, verbose=False, force_sparse=False, fuse_sew_add=True,
                  hwprof=None, fuse_stem=True, fuse_head=True):
    holder = _Root(copy.deepcopy(sj_model))
    model = holder
    stats = {"total_lif_nodes": _count_lif(model), "fused_lif_nodes": 0, "patterns_matched": {},
             "routing": []}
    done = set()

    def record(name, fused, entry, lif):
        done.add(id(lif))
        stats["fused_lif_nodes"] += 1
        _bump(stats, entry["pattern"])
        name = _strip_root(name)
        entry = dict(entry, name=name)
        stats["routing"].append(entry)
        if verbose:
            print(f"  [substitute_sf] {name}: {entry['pattern']} ({entry['shape']}, "
                  f"backend={entry['backend']}, K={entry['K']})")

    # Phase 0a: spiking transformer blocks and patch splitting (Spikformer):
    # Linear -> BN1d -> LIF layers and the attention core fused (the
    # reference leaves them unfused, substitute.py:559-567).
    for pname, pmod in list(model.named_modules()):
        for name, ch in list(pmod.named_children()):
            full = f"{pname}.{name}" if pname else name
            if is_spikformer_block(ch) and id(ch.attn.q_lif) not in done:
                fused = CTFSpikformerBlock.from_sj_block(ch)
                setattr(pmod, name, fused)
                a, m = ch.attn, ch.mlp
                d, hid = a.q.in_features, m.fc1.out_features
                record(full + ".attn.qkv", fused, {"pattern": "FusedLinearBNLIF",
                       "shape": f"{d}->3x{d} (q, k, v)", "backend": "StreamFuse", "K": T},
                       a.q_lif)
                for lif in (a.k_lif, a.v_lif):
                    done.add(id(lif))
                    stats["fused_lif_nodes"] += 1
                record(full + ".attn.core", fused, {"pattern": "SpikeAttentionLIF",
                       "shape": f"{a.num_heads} heads x 32, scale {a.scale:g}",
                       "backend": "StreamFuse", "K": T}, a.attn_lif)
                record(full + ".attn.proj", fused, {"pattern": "FusedLinearBNLIF",
                       "shape": f"{d}->{d} + residual", "backend": "StreamFuse", "K": T},
                       a.proj_lif)
                record(full + ".mlp.fc1", fused, {"pattern": "FusedLinearBNLIF",
                       "shape": f"{d}->{hid}", "backend": "StreamFuse", "K": T}, m.fc1_lif)
                record(full + ".mlp.fc2", fused, {"pattern": "FusedLinearBNLIF",
                       "shape": f"{hid}->{d} + residual", "backend": "StreamFuse", "K": T},
                       m.fc2_lif)
            elif is_spikformer_sps(ch) and id(ch.lif0) not in done:
                fused = CTFSpikformerSPS.from_sj_module(ch)
                setattr(pmod, name, fused)
                for i in range(4):
                    c = getattr(ch, f"conv{i}")
                    record(f"{full}.conv{i}", fused, {"pattern": "PartialFusionConvBNLIF",
                           "shape": f"{c.in_channels}->{c.out_channels}, k=3, s=1",
                           "backend": SpatialBackend.DENSE_KEEP, "K": T}, getattr(ch, f"lif{i}"))
                c = ch.rpe_conv
                record(f"{full}.rpe_conv", fused, {"pattern": "PartialFusionConvBNLIF",
                       "shape": f"{c.in_channels}->{c.out_channels}, k=3, s=1 + input",
                       "backend": SpatialBackend.DENSE_KEEP, "K": T}, ch.rpe_lif)

    # Phase 0: ResNet stem conv1 / bn1 / sn1 / maxpool as one fused kernel
    # (no counterpart in the reference, which leaves the maxpool unfused).
    for pname, pmod in list(model.named_modules()):
        if not (fuse_stem and _is_resnet_stem_owner(pmod)) or id(pmod.sn1) in done:
            continue
        c, b, l = pmod.conv1, pmod.bn1, pmod.sn1
        fused = PartialFusionConvBNLIFMaxPool.from_sj_modules(c, b, l, pmod.maxpool)
        pmod.conv1 = fused
        pmod.bn1, pmod.sn1, pmod.maxpool = nn.Identity(), nn.Identity(), nn.Identity()
        k, st, _ = conv_geometry(c)
        record(f"{pname}.conv1" if pname else "conv1", fused,
               {"pattern": "PartialFusionConvBNLIFMaxPool",
                "shape": f"{c.in_channels}->{c.out_channels}, k={k}, s={st}, maxpool 3/2/1",
                "backend": SpatialBackend.DENSE_KEEP, "K": T}, l)

    # Phase 1a: conv{i} / bn{i} / sn{i}
    for pname, pmod in list(model.named_modules()):
        for idx in ("1", "2", "3"):
            c = getattr(pmod, f"conv{idx}", None)
            b = getattr(pmod, f"bn{idx}", None)
            l = getattr(pmod, f"sn{idx}", None)
            if not (_is_fusable_conv(c) and _is_sj_bn2d(b) and _is_lif(l)) or id(l) in done:
                continue
            fused, entry = _build_conv_bn_lif(c, b, l, T, force_sparse, hwprof)
            setattr(pmod, f"conv{idx}", fused)
            setattr(pmod, f"bn{idx}", nn.Identity())
            setattr(pmod, f"sn{idx}", nn.Identity())
            record(f"{pname}.conv{idx}" if pname else f"conv{idx}", fused, entry, l)

    # Phase 1b: downsample = Sequential(Conv, BN) + downsample_sn
    for pname, pmod in list(model.named_modules()):
        ds, ds_sn = getattr(pmod, "downsample", None), getattr(pmod, "downsample_sn", None)
        if not isinstance(ds, nn.Sequential) or len(ds) < 2 or not _is_lif(ds_sn):
            continue
        if id(ds_sn) in done or not (_is_sj_conv2d(ds[0]) and _is_sj_bn2d(ds[1])):
            continue
        c = ds[0]
        k, s, _ = conv_geometry(c)
        fused = PartialFusionConvBNLIF.from_sj_modules(c, ds[1], ds_sn)
        pmod.downsample = nn.Sequential(fused, nn.Identity())
        pmod.downsample_sn = nn.Identity()
        record(f"{pname}.downsample" if pname else "downsample", fused,
               {"pattern": "PartialFusionConvBNLIF",
                "shape": f"{c.in_channels}->{c.out_channels}, k={k}, s={s}",
                "backend": SpatialBackend.DENSE_KEEP, "K": T}, ds_sn)

    # Phase 1c: X / X_bn / X_lif (or X_sn); Phase 1d: conv{i}/bn{i}/lif{i}, rpe_*
    for pname, pmod in list(model.named_modules()):
        names = {n for n, _ in pmod.named_children()}
        triples = []
        for cname in sorted(names):
            for suf in ("_bn", "_lif", "_sn"):
                if cname.endswith(suf):
                    base = cname[:-len(suf)]
                    lif_attr = base + "_lif" if hasattr(pmod, base + "_lif") else base + "_sn"
                    triples.append((base, base + "_bn", lif_attr))
        for i in range(10):
            triples.append((f"conv{i}", f"bn{i}", f"lif{i}"))
        triples.append(("rpe_conv", "rpe_bn", "rpe_lif"))
        seen = set()
        for ca, ba, la in triples:
            if (ca, ba, la) in seen:
                continue
            seen.add((ca, ba, la))
            c, b, l = getattr(pmod, ca, None), getattr(pmod, ba, None), getattr(pmod, la, None)
            if c is None or b is None or not _is_lif(l) or id(l) in done:
                continue
            full = f"{pname}.{ca}" if pname else ca
            if _is_fusable_conv(c) and _is_sj_bn2d(b):
                fused, entry = _build_conv_bn_lif(c, b, l, T, force_sparse, hwprof)
                setattr(pmod, ca, fused)
                setattr(pmod, ba, nn.Identity())
                setattr(pmod, la, nn.Identity())
                record(full, fused, entry, l)
            elif _is_sj_linear(c) and isinstance(b, nn.BatchNorm1d):
                warnings.warn(f"catfuse_amd: Linear+BN1d+LIF at {full} is not fused (BN1d is "
                              f"kept as a separate module)", RuntimeWarning, stacklevel=2)

    # Phase 2: Sequential patterns
    for pname, pmod in list(model.named_modules()):
        for name, child in list(pmod.named_children()):
            if not isinstance(child, nn.Sequential):
                continue
            ch = list(child)
            n, i, out, changed = len(ch), 0, [], False
            while i < n:
                base = f"{pname}.{name}.{i}" if pname else f"{name}.{i}"
                if (i + 3 < n and _is_sj_conv2d(ch[i]) and _is_sj_bn2d(ch[i + 1])
                        and _is_avgpool2(ch[i + 2]) and _is_lif(ch[i + 3])
                        and id(ch[i + 3]) not in done):
                    c = ch[i]
                    k, s, _ = conv_geometry(c)
                    fused = PartialFusionConvBNAvgPoolLIF.from_sj_modules(*ch[i:i + 4])
                    out.append(fused)
                    record(base, fused, {"pattern": "PartialFusionConvBNAvgPoolLIF",
                                         "shape": f"{c.in_channels}->{c.out_channels}, k={k}, s={s}",
                                         "backend": SpatialBackend.DENSE_KEEP, "K": T}, ch[i + 3])
                    i += 4
                    changed = True
                    continue
                if (i + 2 < n and _is_fusable_conv(ch[i]) and _is_sj_bn2d(ch[i + 1])
                        and _is_lif(ch[i + 2]) and id(ch[i + 2]) not in done):
                    fused, entry = _build_conv_bn_lif(ch[i], ch[i + 1], ch[i + 2], T,
                                                      force_sparse, hwprof)
                    out.append(fused)
                    record(base, fused, entry, ch[i + 2])
                    i += 3
                    changed = True
                    continue
                if (i + 1 < n and _is_sj_linear(ch[i]) and _is_lif(ch[i + 1])
                        and id(ch[i + 1]) not in done):
                    c = ch[i]
                    fused = FusedLinearLIF.from_sj_modules(c, ch[i + 1])
                    out.append(fused)
                    record(base, fused, {"pattern": "FusedLinearLIF",
                                         "shape": f"{c.in_features}->{c.out_features}",
                                         "backend": SpatialBackend.DENSE_KEEP, "K": T}, ch[i + 1])
                    i += 2
                    changed = True
                    continue
                if (i + 1 < n and _is_avgpool2(ch[i]) and _is_lif(ch[i + 1])
                        and id(ch[i + 1]) not in done):
                    fused = FusedAvgPoolLIF.from_sj_modules(ch[i], ch[i + 1])
                    out.append(fused)
                    record(base, fused, {"pattern": "FusedAvgPoolLIF", "shape": "pool 2x2",
                                         "backend": SpatialBackend.DENSE_KEEP, "K": T}, ch[i + 1])
                    i += 2
                    changed = True
                    continue
                if _head_linear(ch, i, out):
                    out.append(FusedLinear.from_sj_modules(ch[i]))
                    _bump(stats, "FusedLinear")
                    i += 1
                    changed = True
                    continue
                out.append(ch[i])
                i += 1
            if changed:
                setattr(pmod, name, nn.Sequential(*out))

    if fuse_sew_add:
        _wrap_sew_blocks(model)

    # Phase 3: a global average pool in the head reads the last fused conv's
    # fp16 NHWC copy, a multi-step flatten passes a one-pixel fused output on
    # as tokens over that copy, and a multi-step LIF no pattern absorbed runs
    # as the streaming LIF kernel (no counterpart in the reference, which
    # leaves the head to SpikingJelly).
    if fuse_head:
        for pname, pmod in list(model.named_modules()):
            for name, ch in list(pmod.named_children()):
                if _is_global_avgpool(ch):
                    setattr(pmod, name, FusedGlobalAvgPool.from_sj_modules(ch))
                    _bump(stats, "FusedGlobalAvgPool")
                elif _is_multistep_flatten(ch):
                    setattr(pmod, name, FusedFlatten.from_sj_modules(ch))
                    _bump(stats, "FusedFlatten")
                elif (_is_lif(ch) and id(ch) not in done
                      and getattr(ch, "step_mode", "s") == "m"):
                    # a multi-step LIF no pattern absorbed: the streaming kernel
                    fused = FusedLIF.from_sj_modules(ch)
                    setattr(pmod, name, fused)
                    full = f"{pname}.{name}" if pname else name
                    record(full, fused, {"pattern": "FusedLIF", "shape": "standalone",
                                         "backend": SpatialBackend.DENSE_KEEP, "K": T}, ch)

    _record_unsupported_convs(model, stats)
    stats["coverage_pct"] = 100.0 * stats["fused_lif_nodes"] / max(stats["total_lif_nodes"], 1)
    return holder.root, stats


def _head_linear(ch, i, out) -> bool:
    """ch[i] is a plain Linear (no neuron after it) whose input is the
    output of the fused Linear-LIF just rewritten (out[-1]): it can read that
    layer's fp16 copy (FusedLinear)."""
    return (_is_sj_linear(ch[i]) and not (i + 1 < len(ch) and _is_lif(ch[i + 1]))
            and bool(out) and isinstance(out[-1], FusedLinearLIF)
            and ch[i].out_features <= 4096)


def _is_multistep_flatten(m) -> bool:
    return (isinstance(m, nn.Flatten) and getattr(m, "step_mode", "s") == "m"
            and m.start_dim == 1 and m.end_dim == -1)


def _is_global_avgpool(m) -> bool:
    if not isinstance(m, nn.AdaptiveAvgPool2d):
        return False
    o = m.output_size
    return o == 1 or tuple(o if isinstance(o, (tuple, list)) else (o, o)) == (1, 1)


def _fused_conv(m):
    return isinstance(m, (PartialFusionConvBNLIF, STFusionConvBNLIF))


def _wrap_sew_blocks(model):
    """SEW BasicBlocks whose three Conv-BN-LIF sites were all fused become
    CTFSEWBasicBlock (ADD in conv2's epilogue)."""
    for pname, pmod in list(model.named_modules()):
        for name, child in list(pmod.named_children()):
            if not (type(child).__name__ == "BasicBlock" and getattr(child, "cnf", None)):
                continue
            if not (_fused_conv(child.conv1) and _fused_conv(child.conv2)):
                continue
            ok_id = all(isinstance(getattr(child, a), nn.Identity)
                        for a in ("bn1", "sn1", "bn2", "sn2"))
            ds = child.downsample
            fused_ds = None
            if ds is not None:
                if not (isinstance(ds, nn.Sequential) and _fused_conv(ds[0])
                        and isinstance(getattr(child, "downsample_sn", None), nn.Identity)):
                    continue
                fused_ds = ds[0]
            if ok_id:
                setattr(pmod, name, CTFSEWBasicBlock(child.conv1, child.conv2, fused_ds,
                                                     child.cnf))


def print_routing_table(stats):
    routing = stats.get("routing", [])
    if not routing:
        print("  No routing decisions recorded.")
        return
    print(f"  {'Layer':<42s} {'Pattern':<30s} {'Shape':<20s} {'Backend':<12s} {'K':>3s}")
    print("  " + "-" * 109)
    for r in routing:
        print(f"  {r['name']:<42s} {r['pattern']:<30s} {r['shape']:<20s} {r['backend']:<12s} "
              f"{r['K']:>3d}")
    backends = {}
    for r in routing:
        backends[r["backend"]] = backends.get(r["backend"], 0) + 1
    print(f"\n  Backend summary: {backends}")
    print(f"  Total fused: {stats['fused_lif_nodes']}/{stats['total_lif_nodes']} "
          f"({stats['coverage_pct']:.1f}%)")
