"""Host-side logic of the drop-in API (no GPU): policy table KATs, hardware
profiles, IOCost known answers (tests/stage4_verify.py:120-124,181,247 and
the analytic columns of experiments/results/k_sweep.csv, kept as a fixture),
the schedule verifier cases (tests/stage5_verify.py:155-231), StateBuffer,
and the substitution structure/routing stats on the model builders."""
import csv
import math
import os

import pytest
import torch

from catfuse_amd import hardware, policy, snn
from catfuse_amd.implementations import (ConvLIFSpec, DenseKeep, ScheduleDecomposition,
                                         ScheduleTransform, SparseFlow, StreamFuse)
from catfuse_amd.state import StateBuffer

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_policy_kats():
    row = policy.get_policy("Conv3x3_BN_LIF", C_in=64, C_out=64, H=56, W=56)
    assert row.spatial_backend == policy.SpatialBackend.DENSE_KEEP
    row2 = policy.get_policy("Conv3x3_BN_LIF", C_in=512, C_out=512, H=7, W=7)
    assert row2.spatial_backend == policy.SpatialBackend.SPARSE_FLOW
    assert row2.K == 8
    assert policy.get_policy("Linear_LIF", T=4).K == 4
    assert policy.classify_shape_regime(64, 64, 56, 56, 1) == "memory_bound"
    assert policy.classify_shape_regime(192, 192, 40, 40) == "compute_bound"
    assert policy.classify_shape_regime(192, 192, 20, 20) == "memory_bound"
    assert policy.optimal_K(16, "compute_bound") == 4
    assert policy.optimal_K(4, "memory_bound") == 4
    assert abs(policy.io_ratio_partial_fusion(4) - 3.5 / 7) < 1e-12
    assert abs(policy.io_ratio_full_fusion(8) - 1.25 / 5) < 1e-12
    # unknown pattern -> conservative partial fusion with K = min(4, T)
    r = policy.get_policy("Conv5x5_BN_LIF", C_in=64, H=8, W=8, T=2)
    assert (r.K, r.spatial_backend) == (2, policy.SpatialBackend.DENSE_KEEP)


def test_hardware_profiles():
    assert hardware.DEFAULT is hardware.V100_PCIE_32GB
    assert hardware.MI355X.gcn_arch == "gfx950"
    assert hardware.MI355X.hbm_bandwidth_gbps == 8000.0
    assert hardware.A100_40GB.sm_capability == 80
    p = hardware.detect_hardware()
    assert isinstance(p, hardware.HardwareProfile)


SPEC = ConvLIFSpec(256, 256, 3, 1, 1, has_conv_bias=False, has_bn=True, tau=2.0,
                   v_threshold=1.0, v_reset=0.0)


def test_iocost_dense_keep_kat():
    c = DenseKeep().analytic_io_cost(SPEC, T=4, B=2, H_in=8, W_in=8, dtype_bytes=4)
    assert (c.x_load, c.w_load, c.z_io, c.v_io, c.spike_write) == \
        (524_288, 2_359_296, 1_048_576, 262_144, 524_288)
    assert c.total == 524_288 + 2_359_296 + 1_048_576 + 262_144 + 524_288
    assert c.num_blocks == 1


@pytest.mark.parametrize("impl_cls", [SparseFlow, StreamFuse])
def test_iocost_fused_kat(impl_cls):
    impl = impl_cls()
    hwc = 8 * 8 * 256
    for K in (1, 2, 4):
        c = impl.analytic_io_cost(SPEC, T=4, B=2, H_in=8, W_in=8, K=K)
        nb = math.ceil(4 / K)
        assert c.z_io == 0 and c.v_io == 2 * nb * 2 * hwc * 4 and c.num_blocks == nb
    dk = DenseKeep().analytic_io_cost(SPEC, 4, 2, 8, 8)
    sf = impl.analytic_io_cost(SPEC, 4, 2, 8, 8, K=4)
    assert abs(sf.intermediate_io / dk.intermediate_io - 1.0 / 5) < 1e-12   # 1/(T+1)


def test_iocost_matches_k_sweep_fixture():
    rows = list(csv.DictReader(open(os.path.join(GOLDEN, "k_sweep_analytic.csv"))))
    assert len(rows) >= 16
    for r in rows:
        T, B, Cin, Cout, H, W, K = (int(r[k]) for k in ("T", "B", "Cin", "Cout", "H", "W", "K"))
        spec = ConvLIFSpec(Cin, Cout, 3, 1, 1, False, True, 2.0, 1.0, 0.0)
        impl = DenseKeep() if r["impl"] == "DenseKeep" else SparseFlow()
        c = impl.analytic_io_cost(spec, T=T, B=B, H_in=H, W_in=W, K=K)
        got = (c.num_blocks, c.x_load, c.w_load, c.z_io, c.v_io, c.spike_write,
               c.intermediate_io, c.total)
        want = tuple(int(r[k]) for k in ("num_blocks", "analytic_x_load", "analytic_w_load",
                                         "analytic_z_io", "analytic_v_io",
                                         "analytic_spike_write", "analytic_intermediate_io",
                                         "analytic_total"))
        assert got == want, (r["config"], r["impl"], K)


def test_schedule_decompositions_verify():
    for impl in (DenseKeep(), SparseFlow(), StreamFuse()):
        for K in (1, 2, 4):
            ok, errs = impl.schedule_decomposition(SPEC, T=4, K=K).verify()
            assert ok, errs
    assert DenseKeep().schedule_decomposition(SPEC, 4).form == "form_1"
    assert str(SparseFlow().schedule_decomposition(SPEC, 4, 2)) == \
        "TimeBlock(K=2) ∘ StreamFuse(Conv, LIF) ∘ StateCarry(LIF)"


@pytest.mark.parametrize("transforms,marker", [
    ((ScheduleTransform.BatchFold("LIF"), ScheduleTransform.TimeBlock(4)), "BatchFold(LIF) ILLEGAL"),
    ((ScheduleTransform.StreamFuse("LIF", "Conv"), ScheduleTransform.TimeBlock(4)),
     "StreamFuse(LIF, Conv) ILLEGAL"),
    ((ScheduleTransform.StateCarry("Conv"), ScheduleTransform.TimeBlock(4)), "StateCarry(Conv) ILLEGAL"),
    ((ScheduleTransform.BatchFold("Conv"),), "Missing TimeBlock"),
    ((ScheduleTransform.StreamFuse("Conv", "LIF"), ScheduleTransform.TimeBlock(4)),
     "without StateCarry(LIF)"),
    ((ScheduleTransform.TimeBlock(0),), "K >= 1"),
    ((ScheduleTransform.BatchFold("Attention"), ScheduleTransform.TimeBlock(4)),
     "BatchFold(Attention) ILLEGAL"),
])
def test_schedule_verifier_rejects(transforms, marker):
    ok, errs = ScheduleDecomposition(transforms=transforms, form="custom").verify()
    assert not ok and any(marker in e for e in errs), errs


def test_state_buffer_lifecycle():
    s = StateBuffer()
    assert not s.is_initialized and s.peek((2, 3), "cpu") is None
    v = s.get((2, 3), "cpu")
    assert v.shape == (2, 3) and (v == 0).all()
    assert s.get((2, 3), "cpu") is v
    assert s.get((3, 3), "cpu") is not v
    s.set(torch.ones(3, 3, requires_grad=True))
    assert not s.tensor.requires_grad and s.peek((3, 3), "cpu") is not None
    s.reset()
    assert s.tensor is None


def _sew18():
    g = torch.Generator().manual_seed(0)
    m = snn.sew_resnet18(num_classes=10, cnf="ADD")
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    return m.eval()


def test_substitute_sf_sew_resnet18_routing():
    import catfuse_amd
    from catfuse_amd.patterns import CTFSEWBasicBlock, PartialFusionConvBNLIF, STFusionConvBNLIF
    m = _sew18()
    fused, stats = catfuse_amd.optimize(m, device=None, T=4)
    assert stats["total_lif_nodes"] == 20 and stats["fused_lif_nodes"] == 20
    assert stats["coverage_pct"] == 100.0
    sf = sorted(r["name"] for r in stats["routing"] if r["pattern"] == "STFusionConvBNLIF")
    assert sf == ["layer3.0.conv2", "layer3.1.conv1", "layer3.1.conv2", "layer4.0.conv2",
                  "layer4.1.conv1", "layer4.1.conv2"]
    labels = {r["name"]: r["backend"] for r in stats["routing"]}
    assert labels["layer4.0.conv1"] == "DenseKeep"   # stride 2: built and labelled dense
    assert sum(1 for b in labels.values() if b == "SparseFlow") == 6
    assert isinstance(fused.conv1, PartialFusionConvBNLIF)
    assert isinstance(fused.layer3[1].fused_second, STFusionConvBNLIF)
    assert all(isinstance(b, CTFSEWBasicBlock) for l in (fused.layer1, fused.layer2, fused.layer3,
                                                         fused.layer4) for b in l)
    # the head's global average pool reads the fused output's NHWC copy
    from catfuse_amd.patterns import FusedGlobalAvgPool
    assert isinstance(fused.avgpool, FusedGlobalAvgPool) and fused.avgpool.step_mode == "m"
    assert stats["patterns_matched"]["FusedGlobalAvgPool"] == 1
    # the original model is untouched
    assert type(m.layer1[0].sn1).__name__ == "LIFNode"


def test_substitute_block_level():
    import catfuse_amd
    fused, stats = catfuse_amd.optimize(_sew18(), device=None, use_sparseflow=False)
    assert stats["patterns_matched"]["CTFSEWBasicBlock"] == 8
    assert stats["fused_lif_nodes"] == 19   # stem LIF is not inside a block/Sequential


def test_root_sequential_is_rewritten():
    import catfuse_amd
    from catfuse_amd.patterns import CTFPattern
    m = torch.nn.Sequential(snn.Conv2d(8, 8, 3, 1, 1, bias=False), snn.BatchNorm2d(8),
                            snn.LIFNode(), snn.Linear(8, 4), snn.LIFNode())
    for use_sf in (True, False):
        fused, stats = catfuse_amd.optimize(m, device=None, T=4, use_sparseflow=use_sf)
        assert stats["fused_lif_nodes"] == 2, stats
        assert isinstance(fused, torch.nn.Sequential) and len(fused) == 2
        assert all(isinstance(c, CTFPattern) for c in fused)


def test_substitute_sf_vgg11():
    import catfuse_amd
    g = torch.Generator().manual_seed(0)
    m = snn.spiking_vgg11_bn(num_classes=10)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, stats = catfuse_amd.optimize(m.eval(), device=None, T=4)
    pm = stats["patterns_matched"]
    assert pm["PartialFusionConvBNAvgPoolLIF"] == 5
    assert pm["FusedLinearLIF"] == 2
    assert pm.get("PartialFusionConvBNLIF", 0) + pm.get("STFusionConvBNLIF", 0) == 3
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"] == 10
    # the head's multi-step flatten passes the last pool's copy on as tokens
    from catfuse_amd.patterns import FusedFlatten
    assert pm["FusedFlatten"] == 1 and isinstance(fused.flatten, FusedFlatten)
    x = torch.arange(2 * 3 * 4 * 2 * 2, dtype=torch.float32).view(2, 3, 4, 2, 2)
    assert torch.equal(fused.flatten(x), torch.flatten(x, 2))   # not a fused output
    assert fused.flatten.fallback_calls == 1
    # the last Linear reads the second Linear-LIF's copy
    from catfuse_amd.patterns import FusedLinear
    assert pm["FusedLinear"] == 1 and isinstance(fused.classifier[-1], FusedLinear)
    y = torch.randn(2, 3, 4096)
    assert torch.allclose(fused.classifier[-1](y), m.classifier[-1](y))   # fallback on CPU


def test_crossover_inputs_and_decision():
    """The crossover sweep's input patterns and its decision rule (bench.py
    --workload sf_crossover; CPU parts)."""
    import bench
    shape = (2, 3, 16, 14, 14)
    x = bench.xo_input(0.5, "iid", shape, seed=1)
    assert x.shape == shape and set(x.unique().tolist()) <= {0.0, 1.0}
    # spatial: a zeroed 8x8 block is zero in every channel
    xs = bench.xo_input(1.0, "spatial", shape, seed=2)
    blocks = xs[..., :8, :8].amax(dim=(3, 4))           # [T, B, C]
    assert torch.equal(blocks.amax(dim=2, keepdim=True).expand_as(blocks), blocks)
    # block: zeroed per channel, about 30% of the blocks survive
    xb = bench.xo_input(1.0, "block", (4, 8, 64, 16, 16), seed=3)
    frac = float(xb.mean())
    assert 0.2 < frac < 0.4
    # chgroup: a 16-channel group of an image is silent everywhere or active
    xg = bench.xo_input(1.0, "chgroup", (3, 8, 64, 6, 6), seed=4)
    per_group = xg.reshape(3, 8, 4, 16 * 36).amax(-1)     # [T, B, group]
    assert torch.equal(xg.reshape(3, 8, 4, 16 * 36).amin(-1), per_group)
    assert torch.equal(per_group, per_group[:1].expand_as(per_group))
    assert 0.1 < float(per_group.mean()) < 0.5
    # region: activity of an image only inside one H/2 x W/2 window
    xr = bench.xo_input(1.0, "region", (2, 5, 4, 12, 10), seed=5)
    for b in range(5):
        m = xr[:, b].amax(dim=(0, 1))
        rows_on, cols_on = m.amax(1).nonzero().flatten(), m.amax(0).nonzero().flatten()
        assert len(rows_on) == 6 and len(cols_on) == 5 and int(m.sum()) == 30
    with pytest.raises(ValueError):
        bench.xo_input(0.1, "checker", shape)
    rows = [dict(pattern="iid", rate=r, density=r, SparseFlow=sf, StreamFuse=10.0,
                 DenseKeep=12.0, auto=10.0, **{"SparseFlow-linear": 20.0, "SF+EGD": 10.0})
            for r, sf in ((0.0, 1.0), (0.01, 9.0), (0.1, 11.0), (0.5, 13.0))]
    # rate 0 (StaticZero) never counts as a SparseFlow win
    assert bench.xo_crossover(rows) == {"iid": pytest.approx(0.99)}
    rows[1]["SparseFlow"] = 10.5
    assert bench.xo_crossover(rows) == {"iid": None}
    assert "| iid | 0.01 |" in bench.xo_table(rows)
    # dispatch-score fit: SparseFlow wins above S = 5, loses below
    fit = [dict(density=0.1, S=s, SparseFlow=9.0 if s > 5 else 11.0, StreamFuse=10.0,
                DenseKeep=12.0) for s in (1.0, 2.0, 4.0, 6.0, 8.0)]
    assert bench.xo_egd_fit(fit) == (5.0, 0)
    fit[0]["SparseFlow"] = 9.0            # one win below the others: one misclassified
    assert bench.xo_egd_fit(fit) == (5.0, 1)
    # R_min fit: wins at R 0.6 and 0.8, losses at 0.1 and 0.3 -> midpoint 0.45
    rfit = [dict(density=0.1, R=R, SparseFlow=9.0 if R > 0.5 else 11.0, StreamFuse=10.0,
                 DenseKeep=12.0) for R in (0.1, 0.3, 0.6, 0.8)]
    assert bench.xo_rmin_fit(rfit) == (pytest.approx(0.45), 0)


def test_fused_global_avgpool_fallback_cpu():
    """Without an NHWC copy (here: a CPU tensor) the pattern is torch's
    adaptive_avg_pool2d, in both step modes."""
    from catfuse_amd.patterns import FusedGlobalAvgPool
    x = torch.randn(3, 2, 5, 7, 6, generator=torch.Generator().manual_seed(4))
    pm = FusedGlobalAvgPool("m")
    y = pm(x)
    ref = torch.nn.functional.adaptive_avg_pool2d(x.flatten(0, 1), 1).view(3, 2, 5, 1, 1)
    assert torch.equal(y, ref) and pm.fallback_calls == 1
    ps = FusedGlobalAvgPool.from_sj_modules(snn.AdaptiveAvgPool2d((1, 1)))
    assert ps.step_mode == "s"
    assert torch.equal(ps(x[0]), torch.nn.functional.adaptive_avg_pool2d(x[0], 1))


def test_token_view_and_membrane_layout():
    """A token linear views the B*N tokens of a step as 8x8 images of 64
    consecutive tokens when 64 divides B*N, else per image; its state is per
    view image [nimg, C, H*W], and token_membrane returns it as [B, N, C]."""
    import torch
    from catfuse_amd.runtime import token_membrane, token_view
    assert token_view(32, 196) == (98, 8, 8)
    assert token_view(2, 64) == (2, 8, 8)
    assert token_view(2, 196) == (2, 14, 14)
    assert token_view(3, 10) == (3, 10, 1)
    assert token_view(3, 1) == (3, 1, 1)
    for B, N, C in ((32, 196, 5), (2, 196, 3), (3, 10, 4)):
        nimg, H, W = token_view(B, N)
        # natural state [B, N, C] -> the kernel's per-view-image layout
        nat = torch.arange(B * N * C, dtype=torch.float32).view(B, N, C)
        rows = nat.reshape(B * N, C)                       # token-major rows of one step
        view = rows.view(nimg, H * W, C).transpose(1, 2)   # [nimg, C, H*W] (NCHW per image)
        assert torch.equal(token_membrane(view.contiguous(), B, N), nat)


# ---------------------------------------------------------------------------
# structures the fused kernels do not compute stay unfused
# ---------------------------------------------------------------------------

def _seq(*mods):
    m = torch.nn.Sequential(*mods)
    snn.functional.set_step_mode(m, "m")
    return m.eval()


@pytest.mark.parametrize("conv_kw, reason", [
    (dict(groups=8, dilation=2, padding=2), "groups=8"),
    (dict(groups=4, padding_mode="reflect"), "groups=4"),
    (dict(dilation=2, padding=2), "dilation"),
    (dict(padding_mode="reflect"), "padding_mode"),
    (dict(kernel_size=(1, 3), padding=(0, 1)), "non-square kernel_size"),
    (dict(stride=(1, 2)), "non-square stride"),
    (dict(padding="same"), "padding='same'"),
])
def test_unsupported_conv_left_unfused(conv_kw, reason):
    """Depthwise/grouped, dilated, reflect-padded and non-square convs are
    not substituted (a dense fused kernel would compute something else);
    optimize succeeds, the original module stays, and the reason is listed."""
    import catfuse_amd
    from catfuse_amd.patterns import conv_geometry, CTFPattern, PartialFusionConvBNLIF
    kw = dict(kernel_size=3, stride=1, padding=1, bias=False)
    kw.update(conv_kw)
    ks = kw.pop("kernel_size")
    conv = snn.Conv2d(8, 8, ks, **kw)
    m = _seq(conv, snn.BatchNorm2d(8), snn.LIFNode(),
             snn.Conv2d(8, 16, 3, 1, 1, bias=False), snn.BatchNorm2d(16), snn.LIFNode())
    from catfuse_amd.patterns import FusedLIF
    from catfuse_amd.substitute import substitute
    # optimize runs the unfused conv's LIF as the standalone LIF kernel;
    # the block-level substitute leaves it to SpikingJelly
    for fn, nfused in ((lambda mm: catfuse_amd.optimize(mm, T=4), 2), (substitute, 1)):
        fused, stats = fn(m)
        assert type(fused[0]).__name__ == "Conv2d" and not isinstance(fused[0], CTFPattern)
        assert torch.equal(fused[0].weight, conv.weight)
        assert stats["fused_lif_nodes"] == nfused and stats["total_lif_nodes"] == 2
        assert any(reason in s and s.startswith("0:") for s in stats["unsupported_structures"]), \
            stats["unsupported_structures"]
        assert sum(isinstance(x, CTFPattern) for x in fused.modules()) == nfused
        assert isinstance(fused[2], FusedLIF) == (nfused == 2)
    with pytest.raises(ValueError):
        conv_geometry(conv)
    with pytest.raises(ValueError):
        PartialFusionConvBNLIF.from_sj_modules(conv, snn.BatchNorm2d(8), snn.LIFNode())


@pytest.mark.parametrize("groups, cin, cout, k, s, p", [
    (8, 8, 8, 3, 1, 1), (8, 8, 16, 3, 2, 1), (2, 8, 16, 1, 1, 0), (4, 8, 8, 5, 1, 2)])
def test_grouped_conv_fused(groups, cin, cout, k, s, p):
    """Grouped and depthwise Conv -> BN -> LIF triples become the fused
    grouped pattern (Sequential, conv{i}/bn{i}/sn{i} attributes), with the
    weights, BN statistics and geometry of the original modules."""
    import catfuse_amd
    from catfuse_amd.patterns import PartialFusionGroupedConvBNLIF
    from catfuse_amd.substitute import substitute
    conv = snn.Conv2d(cin, cout, k, s, p, groups=groups, bias=True)
    bn = snn.BatchNorm2d(cout)
    m = _seq(conv, bn, snn.LIFNode(v_threshold=0.5))
    for fn in (lambda mm: catfuse_amd.optimize(mm, T=4), substitute):
        fused, stats = fn(m)
        f = fused[0]
        assert isinstance(f, PartialFusionGroupedConvBNLIF)
        assert (f.groups, f.kernel_size, f.stride, f.padding) == (groups, k, s, p)
        assert torch.equal(f.weight, conv.weight) and torch.equal(f.conv_bias, conv.bias)
        assert torch.equal(f.running_var, bn.running_var) and f.v_threshold == 0.5
        assert stats["fused_lif_nodes"] == 1 and not stats.get("unsupported_structures")


def test_sew_block_with_depthwise_conv():
    """A SEW BasicBlock whose conv2 is depthwise is not replaced by the
    fused block (its ADD stays the block's own): optimize fuses its convs
    one by one, the depthwise one as the grouped pattern; the block-level
    substitute leaves that block unfused and lists the conv."""
    import catfuse_amd
    from catfuse_amd.patterns import CTFSEWBasicBlock, PartialFusionGroupedConvBNLIF
    from catfuse_amd.substitute import substitute
    net = snn.sew_resnet18(num_classes=10)
    blk = net.layer1[1]
    blk.conv2 = snn.Conv2d(64, 64, 3, 1, 1, groups=64, bias=False)
    snn.functional.set_step_mode(net, "m")
    fused, stats = catfuse_amd.optimize(net.eval(), T=4)
    assert not isinstance(fused.layer1[1], CTFSEWBasicBlock)
    assert isinstance(fused.layer1[1].conv2, PartialFusionGroupedConvBNLIF)
    assert isinstance(fused.layer1[0], CTFSEWBasicBlock)
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"]
    fused, stats = substitute(net.eval())
    assert not isinstance(fused.layer1[1], CTFSEWBasicBlock)
    assert type(fused.layer1[1].conv2).__name__ == "Conv2d"
    assert any(s.startswith("layer1.1.conv2:") and "groups=64" in s
               for s in stats["unsupported_structures"])
    assert isinstance(fused.layer1[0], CTFSEWBasicBlock)


class IFNode(torch.nn.Module):
    """An integrate-and-fire neuron (SpikingJelly's IFNode has v_threshold,
    v_reset but no leak): not an LIF neuron."""

    def __init__(self, **kw):
        super().__init__()
        self.v_threshold, self.v_reset, self.step_mode = 1.0, 0.0, "m"

    def forward(self, x):
        return (x.cumsum(0) >= 1.0).float()


def test_spikformer_block_with_if_neurons_left_unfused():
    import catfuse_amd
    from catfuse_amd.transformer import CTFSpikformerBlock, is_spikformer_block
    net = snn.Spikformer(img_size=32, num_classes=10, embed_dim=64, num_heads=2, depth=2,
                         pools=(0, 1))
    net.blocks[1].attn.k_lif = IFNode()
    assert not is_spikformer_block(net.blocks[1]) and is_spikformer_block(net.blocks[0])
    fused, stats = catfuse_amd.optimize(net.eval(), T=4)
    assert isinstance(fused.blocks[0], CTFSpikformerBlock)
    assert not isinstance(fused.blocks[1], CTFSpikformerBlock)
    assert stats["fused_lif_nodes"] <= stats["total_lif_nodes"]


def test_spikformer_attention_kernel_coverage():
    """head dim 64 (the reference's spikformer_cifar_tiny: dim 192, 3 heads)
    is substituted and its attention core is covered by the hand-written
    kernels, as are long token rows (56 x 56 = 3,136 tokens, the two-pool
    patch splitter at 224 x 224); a head dim the kernels do not take (48)
    runs the exact library-GEMM core."""
    import catfuse_amd
    from catfuse_amd.transformer import CTFSpikformerBlock
    net = snn.Spikformer(img_size=32, num_classes=10, embed_dim=192, num_heads=3, depth=1,
                         pools=(0, 1))
    fused, stats = catfuse_amd.optimize(net.eval(), T=4)
    blk = fused.blocks[0]
    assert isinstance(blk, CTFSpikformerBlock)
    assert blk.attn.head_dim == 64 and blk.attn.kernel_covers(64) and blk.attn.kernel_covers(3136)
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"]   # pre-head LIF: FusedLIF
    from catfuse_amd.patterns import FusedLIF
    assert isinstance(fused.pre_head_lif, FusedLIF) and stats["patterns_matched"]["FusedLIF"] == 1
    small = snn.spikformer_8_384(img_size=224)
    f2, _ = catfuse_amd.optimize(small.eval(), T=4)
    a = f2.blocks[0].attn
    assert a.head_dim == 32 and a.kernel_covers(196) and a.kernel_covers(3136)
    odd = snn.Spikformer(img_size=32, num_classes=10, embed_dim=96, num_heads=2, depth=1,
                         pools=(0, 1))
    f3, _ = catfuse_amd.optimize(odd.eval(), T=4)
    assert f3.blocks[0].attn.head_dim == 48 and not f3.blocks[0].attn.kernel_covers(64)


def test_lazy_head_helpers_decline_plain_tensors():
    """The copy-reading head helpers take only pending fused outputs: a plain
    tensor, a wrong axis or extra arguments go through torch (None)."""
    from catfuse_amd import runtime
    x = torch.randn(2, 3, 5, 4)
    assert runtime._token_mean((x, 2), {}) is None
    assert runtime._token_mean((x,), {"dim": 2, "keepdim": True}) is None
    assert torch.equal(x.mean(dim=2), x.mean(2))
    assert runtime.pixel_tokens(torch.randn(2, 3, 4, 1, 1)) is None
    assert runtime.linear_tokens(torch.randn(2, 3, 8), torch.randn(4, 8)) is None


@pytest.mark.parametrize("downsample", [False, True])
def test_substitute_bottlenecks(downsample):
    """SEW and spiking-ResNet Bottlenecks become CTFSEWBottleneck /
    CTFSpikingBottleneck (catfuse/substitute.py matches "Bottleneck" blocks,
    with and without `cnf`), every LIF of the block counted as fused."""
    from catfuse_amd.substitute import substitute
    from catfuse_amd.patterns import (CTFSEWBottleneck, CTFSpikingBottleneck,
                                      PartialFusionConvBNAddLIF, PartialFusionConvBNLIF)
    from blocks import SEWBottleneck, SpikingBottleneck
    stride = 2 if downsample else 1
    inp = 64 if downsample else 128
    sew = torch.nn.Sequential(SEWBottleneck(inp, 32, stride, "ADD", downsample))
    snn.functional.set_step_mode(sew, "m")
    fused, stats = substitute(sew)
    blk = fused[0]
    assert isinstance(blk, CTFSEWBottleneck) and blk.cnf == "ADD"
    assert stats["patterns_matched"].get("CTFSEWBottleneck") == 1
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"] == (4 if downsample else 3)
    for part in (blk.fused_first, blk.fused_middle, blk.fused_last):
        assert isinstance(part, PartialFusionConvBNLIF)
    assert (blk.fused_downsample is not None) == downsample
    assert blk.fused_middle.stride == stride
    spk = torch.nn.Sequential(SpikingBottleneck(inp, 32, stride, downsample))
    snn.functional.set_step_mode(spk, "m")
    fused, stats = substitute(spk)
    blk = fused[0]
    assert isinstance(blk, CTFSpikingBottleneck)
    assert isinstance(blk.fused_last_add, PartialFusionConvBNAddLIF)
    assert stats["patterns_matched"].get("CTFSpikingBottleneck") == 1
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"] == 3
    assert blk.has_downsample == downsample


def test_mi355x_profile_refuses_sparseflow_for_1x1(monkeypatch):
    """The measured gfx950 crossover (SparseFlow 1.42-2.11x slower than the
    dense route on every 1x1 row) makes the MI355X profile refuse
    SparseFlow for 1x1 convs: no scan/prescan geometry even with the
    sparsity threshold lowered; 3x3 layers keep their gate (tau 0, R_min 0.4)."""
    monkeypatch.setenv("CATFUSE_SF_SPARSITY_THRESHOLD", "0.7")
    sf = SparseFlow()
    assert math.isinf(hardware.MI355X.sf_egd_tau_1x1)
    kw = dict(has_conv_bias=False, has_bn=True, tau=2.0, v_threshold=1.0, v_reset=0.0,
              decay_input=True)
    assert sf.route_geometry(ConvLIFSpec(64, 128, 1, 2, 0, **kw), 56, 56) is None
    assert sf.route_geometry(ConvLIFSpec(256, 256, 1, 1, 0, **kw), 14, 14) is None
    g = sf.route_geometry(ConvLIFSpec(64, 64, 3, 1, 1, **kw), 56, 56)
    assert g is not None and g["egd"] == (0.0, 0.4) and (g["block_h"], g["block_w"]) == (8, 8)


def test_lazy_output_metadata_without_materialising():
    """A fused layer's pending output answers metadata queries (shape,
    dtype, device, dim, numel, contiguity, contiguous()) from the record
    made at creation, without materialising (on the CPU any
    materialisation would call the HIP library and fail)."""
    from catfuse_amd import runtime
    base = torch.empty(4, 2, 8, 5, 5)
    nhwc = torch.zeros(8, 5, 5, 32, dtype=torch.float16)
    x = runtime.NHWCSpikes(base, nhwc)
    assert x.shape == (4, 2, 8, 5, 5) and x.dtype == torch.float32
    assert x.device == torch.device("cpu") and not x.is_cuda
    assert x.ndim == x.dim() == 5 and x.numel() == 1600 and x.size(2) == 8
    assert x.is_contiguous() and x.contiguous() is x
    assert x.__dict__["_cf_pending"]
    x._cf_pending = False          # materialised: the ordinary path
    assert x.shape == (4, 2, 8, 5, 5) and x.dim() == 5 and x.is_contiguous()
