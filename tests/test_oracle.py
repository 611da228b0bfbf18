"""Pins the CPU oracle (oracle/) with checks that do not restate its code:
hand-derived closed-form LIF sequences, an independent torch evaluation of
SpikingJelly's op sequence, two independent prescan formulations plus their
closed-form special cases, and a brute-force convolution."""
import numpy as np
import pytest
import torch

import oracle


# ---------------------------------------------------------------------------
# LIF: closed forms (derived by hand, SpikingJelly semantics)
# ---------------------------------------------------------------------------

def test_lif_constant_input_closed_form():
    # tau=2, v_th=1, hard reset 0, decay_input: v1 = 1.5/2 = 0.75;
    # v2 = 0.75 + (1.5 - 0.75)/2 = 1.125 -> spike, reset to 0; period 2.
    z = np.full((6, 1), 1.5, np.float32)
    s, v, h = oracle.lif_multistep(z)
    assert s[:, 0].tolist() == [0, 1, 0, 1, 0, 1]
    assert h[:, 0].tolist() == [0.75, 1.125, 0.75, 1.125, 0.75, 1.125]
    assert v[0] == 0.0


def test_lif_zero_input_decays_by_half():
    v0 = np.array([0.8, -0.4, 0.0], np.float32)
    s, v, h = oracle.lif_multistep(np.zeros((3, 3), np.float32), v_in=v0)
    assert not s.any()
    np.testing.assert_array_equal(h[0], v0 / 2)
    np.testing.assert_array_equal(v, v0 / 8)


def test_lif_threshold_is_inclusive():
    # v = 0 + (2 - 0)/2 = 1.0 exactly -> fires (v >= v_th)
    s, v, _ = oracle.lif_multistep(np.array([[2.0]], np.float32))
    assert s[0, 0] == 1.0 and v[0] == 0.0


def test_lif_soft_reset_subtracts_threshold():
    # soft reset: v1 = 3/2 = 1.5 -> spike, v = 0.5; v2 = 0.5 + (0 - 0.5)/2 = 0.25
    z = np.array([[3.0], [0.0]], np.float32)
    s, v, h = oracle.lif_multistep(z, v_reset=None)
    assert s[:, 0].tolist() == [1.0, 0.0]
    assert h[:, 0].tolist() == [1.5, 0.25]
    assert v[0] == 0.25


def test_lif_no_decay_input():
    # decay_input=False, hard reset: v = v - (v - 0)/2 + x; x=0.6: 0.6, 0.9, 1.05 -> spike
    z = np.full((3, 1), 0.6, np.float32)
    s, v, h = oracle.lif_multistep(z, decay_input=False)
    np.testing.assert_allclose(h[:, 0], [0.6, 0.9, 1.05], rtol=1e-6)
    assert s[:, 0].tolist() == [0.0, 0.0, 1.0]


def test_lif_nonzero_reset_value():
    # hard reset to -0.5: v1 = -0.5 + (4 - (-0.5 + 0.5))/2 = 1.5 -> spike -> v = -0.5
    s, v, h = oracle.lif_multistep(np.array([[4.0]], np.float32), v_reset=-0.5)
    assert h[0, 0] == 1.5 and s[0, 0] == 1.0 and v[0] == -0.5


def _torch_sj_reference(z, v, tau, vth, vreset, decay):
    """SpikingJelly's eval recurrence evaluated with torch fp32 CPU ops."""
    out = []
    for t in range(z.shape[0]):
        x = z[t]
        if vreset is not None:
            v = v + (x - (v - vreset)) / tau if decay else v - (v - vreset) / tau + x
        else:
            v = v + (x - v) / tau if decay else v * (1.0 - 1.0 / tau) + x
        s = (v >= vth).to(torch.float32)
        v = vreset * s + (1.0 - s) * v if vreset is not None else v - s * vth
        out.append(s)
    return torch.stack(out), v


@pytest.mark.parametrize("tau,vreset,decay", [(2.0, 0.0, True), (3.0, 0.0, True),
                                              (2.0, None, True), (1.7, 0.0, False),
                                              (2.5, None, False), (2.0, -0.2, True)])
def test_lif_matches_torch_fp32_evaluation(tau, vreset, decay):
    g = torch.Generator().manual_seed(7)
    z = torch.randn(6, 4000, generator=g) * 0.9
    v0 = torch.randn(4000, generator=g) * 0.3
    s_ref, v_ref = _torch_sj_reference(z, v0.clone(), tau, 1.0, vreset, decay)
    s, v, _ = oracle.lif_multistep(z, v_in=v0, tau=tau, v_reset=vreset, decay_input=decay)
    np.testing.assert_array_equal(s, s_ref.numpy())
    np.testing.assert_array_equal(v, v_ref.numpy())


def test_lif_modes_input_current():
    g = torch.Generator().manual_seed(1)
    T, C, HW = 3, 4, 5
    z = torch.randn(T, 2 * C * HW, generator=g)
    z2 = torch.randn(T, 2 * C * HW, generator=g)
    sc = torch.rand(C, generator=g) + 0.5
    sh = torch.randn(C, generator=g)
    c = (torch.arange(2 * C * HW) // HW) % C
    expect = {
        1: z * sc[c] + sh[c],
        2: (z * sc[c] + sh[c]) + z2,
        3: z + z2,
        4: (z + z2) * sc[c] + sh[c],
    }
    for mode, x in expect.items():
        s, v, h = oracle.lif_multistep(z, mode=mode, z2=z2, scale=sc, shift=sh, C=C, HW=HW)
        s0, v0, h0 = oracle.lif_multistep(x)
        np.testing.assert_array_equal(h, h0)
        np.testing.assert_array_equal(s, s0)


# ---------------------------------------------------------------------------
# Prescan: two independent formulations + closed forms
# ---------------------------------------------------------------------------

PRESCAN_CASES = [
    # N, C, H, W, k, s, p
    (2, 64, 32, 32, 3, 1, 1),
    (1, 256, 14, 14, 3, 1, 1),
    (2, 32, 56, 56, 3, 1, 1),
    (1, 40, 9, 11, 3, 1, 1),
    (1, 64, 16, 16, 3, 2, 1),
    (2, 48, 12, 12, 1, 2, 0),
    (1, 128, 8, 8, 1, 1, 0),
]


@pytest.mark.parametrize("case", PRESCAN_CASES)
@pytest.mark.parametrize("rate", [0.0, 0.002, 0.05, 0.5])
def test_prescan_bruteforce_equals_maxpool_cascade(case, rate):
    N, C, H, W, k, s, p = case
    g = torch.Generator().manual_seed(hash((case, rate)) % 1000)
    x = (torch.rand(N, C, H, W, generator=g) < rate).float()
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    bh, bw = oracle.select_tile_sizes(Ho, Wo)
    gs = oracle.choose_group_size(C)
    a = oracle.prescan2d(x, Ho, Wo, k, s, p, bh, bw, gs)
    b = oracle.prescan2d_maxpool(x, Ho, Wo, k, s, p, bh, bw, gs)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_prescan_closed_forms():
    N, C, H, W = 1, 64, 16, 16
    gs = oracle.choose_group_size(C)          # 16 -> 4 groups
    assert gs == 16
    zero = np.zeros((N, C, H, W), np.float32)
    tc, ag = oracle.prescan2d(zero, H, W, 3, 1, 1, 8, 8, gs)
    assert (tc == 0).all() and (ag == 0).all()
    ones = np.ones((N, C, H, W), np.float32)
    tc, ag = oracle.prescan2d(ones, H, W, 3, 1, 1, 8, 8, gs)
    assert (tc == 2).all() and (ag == 0b1111).all()
    # one spike at channel 37 (group 2), pixel (7, 8): the 3x3 RF of output
    # pixels (6..8, 7..9) touches tiles (0,0)? no: oh in 6..8 -> gh 0 (6,7) and
    # gh 1 (8); ow in 7..9 -> gw 0 (7) and gw 1 (8, 9) -> all four tiles.
    one = np.zeros((N, C, H, W), np.float32)
    one[0, 37, 7, 8] = 1.0
    tc, ag = oracle.prescan2d(one, H, W, 3, 1, 1, 8, 8, gs)
    assert ag.tolist() == [4, 4, 4, 4] and tc.tolist() == [1, 1, 1, 1]
    # at pixel (3, 3) only tile (0, 0) sees it
    one[:] = 0
    one[0, 5, 3, 3] = 1.0
    tc, ag = oracle.prescan2d(one, H, W, 3, 1, 1, 8, 8, gs)
    assert ag.tolist() == [1, 0, 0, 0]
    # threshold: |x| must exceed 1e-6 strictly; negative values count
    one[0, 5, 3, 3] = -2e-6
    assert oracle.prescan2d(one, H, W, 3, 1, 1, 8, 8, gs)[1][0] == 1
    one[0, 5, 3, 3] = 1e-6
    assert oracle.prescan2d(one, H, W, 3, 1, 1, 8, 8, gs)[1][0] == 0


def test_prescan_32_groups_sign_bit():
    C = 1024  # gs 32 -> 32 groups -> bit 31 is the int32 sign bit
    assert oracle.choose_group_size(C) == 32
    x = np.zeros((1, C, 8, 8), np.float32)
    x[0, C - 1, 0, 0] = 1
    tc, ag = oracle.prescan2d(x, 8, 8, 1, 1, 0, 8, 8, 32)
    assert ag[0] == np.int32(-2 ** 31)
    tc2, ag2 = oracle.prescan2d_maxpool(x, 8, 8, 1, 1, 0, 8, 8, 32)
    assert ag2[0] == ag[0]


def test_geometry_helpers():
    assert [oracle.choose_group_size(c) for c in (3, 64, 128, 129, 256, 512, 1024, 2048)] == \
        [16, 16, 16, 32, 32, 32, 32, 64]
    assert oracle.select_tile_sizes(56, 56) == (8, 16)
    assert oracle.select_tile_sizes(55, 57) == (8, 8)    # 3135 pixels < 3136
    assert oracle.select_tile_sizes(14, 14) == (8, 8)


def test_route_decision():
    assert oracle.route(np.zeros(100, np.float32)) == 0
    x = np.zeros(1000, np.float32)
    x[:300] = 1   # sparsity 0.7 -> not > 0.7 -> dense
    assert oracle.route(x) == 2
    x[299] = 0    # sparsity 0.701 -> sparse
    assert oracle.route(x) == 1


# ---------------------------------------------------------------------------
# Conv / BN
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(2, 3, 9, 9, 5, 3, 1, 1), (1, 4, 8, 10, 6, 1, 2, 0),
                                   (1, 3, 15, 15, 4, 7, 2, 3)])
def test_conv_library_equals_bruteforce(shape):
    N, Cin, H, W, Cout, k, s, p = shape
    g = torch.Generator().manual_seed(3)
    x = torch.randn(N, Cin, H, W, generator=g)
    w = torch.randn(Cout, Cin, k, k, generator=g)
    a = oracle.conv2d(x, w, stride=s, padding=p).numpy()
    b = oracle.conv2d_bruteforce(x, w, stride=s, padding=p)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-6)


def test_bn_fold_matches_torch_batch_norm():
    g = torch.Generator().manual_seed(4)
    C = 16
    bn = torch.nn.BatchNorm2d(C).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(C, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(C, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(C, generator=g) * 0.4 + 0.8)
        bn.bias.copy_(torch.randn(C, generator=g) * 0.1)
    z = torch.randn(2, C, 5, 5, generator=g)
    sc, sh = oracle.bn_fold(bn.weight, bn.bias, bn.running_mean, bn.running_var, bn.eps)
    folded = z * sc.view(1, -1, 1, 1) + sh.view(1, -1, 1, 1)
    np.testing.assert_allclose(folded.numpy(), oracle.batch_norm(z, bn).numpy(), rtol=1e-5,
                               atol=1e-6)


# ---------------------------------------------------------------------------
# spiking transformer restatements
# ---------------------------------------------------------------------------

def _lin_bn(I, O, seed):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(I, O)
    bn = torch.nn.BatchNorm1d(O).eval()
    with torch.no_grad():
        lin.weight.copy_(torch.randn(O, I, generator=g) * (2.0 / I) ** 0.5)
        lin.bias.copy_(torch.randn(O, generator=g) * 0.1)
        bn.running_mean.copy_(torch.randn(O, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(O, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(O, generator=g) * 0.4 + 0.8)
        bn.bias.copy_(torch.randn(O, generator=g) * 0.1)
    return lin, bn


def test_linear_bn_lif_equals_1x1_conv_formulation():
    """Linear -> BN1d -> LIF over tokens equals Conv1x1 -> BN2d -> LIF over
    the token grid (an independent formulation through conv_bn_lif), bit for
    bit: both take the float64 product rounded to fp32 and torch's eval BN."""
    from catfuse_amd import snn
    T, B, Hg, Wg, I, O = 3, 2, 3, 4, 24, 40
    lin, bn1 = _lin_bn(I, O, seed=1)
    lif = snn.LIFNode(step_mode="m")
    x = (torch.rand(T, B, Hg * Wg, I, generator=torch.Generator().manual_seed(2)) < 0.3).float()
    s1, v1, h1 = oracle.linear_bn_lif(x, lin, bn1, lif)
    conv = torch.nn.Conv2d(I, O, 1, bias=True)
    bn2 = torch.nn.BatchNorm2d(O).eval()
    with torch.no_grad():
        conv.weight.copy_(lin.weight.view(O, I, 1, 1))
        conv.bias.copy_(lin.bias)
        for n in ("weight", "bias", "running_mean", "running_var"):
            getattr(bn2, n).copy_(getattr(bn1, n))
    xc = x.reshape(T, B, Hg, Wg, I).permute(0, 1, 4, 2, 3)
    s2, v2, h2 = oracle.conv_bn_lif(xc, conv, bn2, lif)
    to_tok = lambda a: np.moveaxis(a, -3, -1).reshape(*a.shape[:-3], Hg * Wg, O)
    np.testing.assert_array_equal(s1, to_tok(s2))
    np.testing.assert_array_equal(h1, to_tok(h2))
    np.testing.assert_array_equal(v1, to_tok(v2))


def test_spike_attention_oracle_pins():
    """The float64 attention equals the definition in loops, and the integer
    identity (Q K^T) V = Q (K^T V) holds (the reordering the kernel uses)."""
    from catfuse_amd import snn
    g = torch.Generator().manual_seed(3)
    T, B, N, heads = 2, 2, 7, 2
    q, k, v = ((torch.rand(T, B, N, 64, generator=g) < 0.4).float() for _ in range(3))
    for scale in (0.125, 32 ** -0.5):
        y = oracle.spike_attention_bruteforce(q, k, v, heads, scale)
        lif = snn.LIFNode(step_mode="m", v_threshold=2.0)
        s, vf, h = oracle.spike_attention_lif(q, k, v, heads, scale, lif)
        # the charge of the first step from v = 0 with tau = 2 is z / 2
        np.testing.assert_allclose(h[0], (y[0] * 0.5).astype(np.float32), rtol=1e-6)
        s_ref, _, _ = oracle.lif_multistep(torch.from_numpy(y).float(), None, v_threshold=2.0)
        np.testing.assert_array_equal(s, s_ref)
    qi, ki, vi = (a.reshape(T, B, N, heads, 32).permute(0, 1, 3, 2, 4).long() for a in (q, k, v))
    assert torch.equal((qi @ ki.transpose(-1, -2)) @ vi, qi @ (ki.transpose(-1, -2) @ vi))


# ---------------------------------------------------------------------------
# network-level forwards, pinned against the eager SpikingJelly-style models
# (catfuse_amd.snn: the module formulation, nn.Conv2d / BatchNorm2d /
# LIFNode.forward in torch fp32) layer by layer, with conv_dtype fp32 so the
# conv is the same library routine on the same values
# ---------------------------------------------------------------------------

def _lif_outputs(model, names_of):
    """Forward hooks on every LIFNode: {key: output spikes}."""
    from catfuse_amd import snn
    outs, hs = {}, []
    for name, mod in model.named_modules():
        if isinstance(mod, snn.LIFNode):
            key = names_of(name)
            hs.append(mod.register_forward_hook(
                lambda m, a, o, key=key: outs.__setitem__(key, o.detach().clone())))
    return outs, hs


def _assert_spikes(got, ref, h, what):
    from parity import lif_parity
    lif_parity(got.numpy(), None, np.asarray(ref), None, h, what=what)


def _sew_key(name):
    if name == "sn1":
        return "conv1"
    base, leaf = name.rsplit(".", 1)
    return {"sn1": base + ".conv1", "sn2": base + ".conv2",
            "downsample_sn": base + ".downsample"}[leaf]


@pytest.mark.parametrize("v_th", [1.0, 0.1])
def test_sew_resnet_forward_pinned_by_eager_model(v_th):
    """oracle.sew_resnet_forward (block order, downsample + its LIF, the
    SEW ADD, the stem pool, the head) equals the eager SEW-ResNet18 built
    from modules: every LIF layer's spikes and the logits.  v_th = 0.1 keeps
    every layer active (checked), so no layer compares all-zero tensors."""
    from catfuse_amd import snn
    m = snn.sew_resnet18(num_classes=10, cnf="ADD", v_threshold=v_th)
    snn.functional.set_step_mode(m, "m")
    g = torch.Generator().manual_seed(5)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    m.eval()
    T, B = 2, 2
    x = torch.randn(B, 3, 48, 48, generator=g).unsqueeze(0).expand(T, B, 3, 48, 48)
    outs, hs = _lif_outputs(m, _sew_key)
    with torch.no_grad():
        y = m(x.contiguous())
    for h in hs:
        h.remove()
    rec = {}
    y_ref = oracle.sew_resnet_forward(m, x, conv_dtype=torch.float32, record=rec)
    assert set(rec) == set(outs) and len(rec) == 20
    for k, (xin, s, h) in rec.items():
        # the stem's spikes before the pool, every other layer's before the add
        _assert_spikes(outs[k], s, h, k)
        if v_th < 1.0:
            assert float(s.sum()) > 0, f"{k}: no spikes (the live variant must be active)"
    np.testing.assert_allclose(y.numpy(), y_ref.numpy(), rtol=1e-5, atol=1e-5)
    if v_th < 1.0:
        # a plausible composition mistake fails on the live network: the
        # wrong connect function in one block changes the logits
        blk = m.layer1[0]
        blk.cnf = "AND"
        y_bad = oracle.sew_resnet_forward(m, x, conv_dtype=torch.float32)
        blk.cnf = "ADD"
        assert not torch.allclose(y_bad, y_ref)


def test_vgg_forward_pinned_by_eager_model():
    """oracle.vgg_forward (Conv-BN-[AvgPool]-LIF runs, flatten, Linear-LIF
    head) equals the eager spiking VGG-11-BN layer by layer and in its
    logits; v_th = 0.25 keeps every layer active (checked)."""
    from catfuse_amd import snn
    m = snn.spiking_vgg11_bn(num_classes=10, v_threshold=0.25)
    snn.functional.set_step_mode(m, "m")
    g = torch.Generator().manual_seed(6)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    with torch.no_grad():   # fan-out init leaves the 4096-wide head silent
        for mod in m.classifier:
            if isinstance(mod, torch.nn.Linear):
                mod.weight.mul_(8.0)
    m.eval()
    T, B = 2, 2
    x = torch.randn(T, B, 3, 32, 32, generator=g)
    keys = {}
    feats = list(m.features)
    conv_idx = [i for i, mod in enumerate(feats) if isinstance(mod, torch.nn.Conv2d)]
    lif_idx = [i for i, mod in enumerate(feats) if isinstance(mod, snn.LIFNode)]
    for ci, li in zip(conv_idx, lif_idx):
        keys[f"features.{li}"] = f"features.{ci}"
    keys["classifier.1"] = "classifier.0"
    keys["classifier.3"] = "classifier.2"
    outs, hs = _lif_outputs(m, lambda n: keys[n])
    with torch.no_grad():
        y = m(x)
    for h in hs:
        h.remove()
    rec = {}
    y_ref = oracle.vgg_forward(m, x, conv_dtype=torch.float32, record=rec)
    assert set(rec) == set(outs) and len(rec) == 10
    for k, (xin, s, h) in rec.items():
        _assert_spikes(outs[k], s, h, k)
        assert float(s.sum()) > 0, f"{k}: no spikes"
    np.testing.assert_allclose(y.numpy(), y_ref.numpy(), rtol=1e-5, atol=1e-5)


def test_spikformer_forward_pinned_by_eager_model():
    """oracle.spikformer_forward (SPS stages and pools, rpe + its input,
    token layout, q/k/v/attention/proj and MLP with their residuals, token
    mean, pre-head LIF, head) equals the eager Spikformer layer by layer and
    in its logits; weights scaled so every layer is active (checked)."""
    from catfuse_amd import snn
    m = snn.Spikformer(img_size=32, num_classes=10, embed_dim=64, num_heads=2, depth=2, T=2,
                       pools=(2, 3), scale=0.125)
    g = torch.Generator().manual_seed(7)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, (torch.nn.Linear, torch.nn.Conv2d)) and mod is not m.head:
                mod.weight.mul_(3.0)
    m.eval()
    T, B = 2, 2
    x = torch.randn(B, 3, 32, 32, generator=g).unsqueeze(0).expand(T, B, 3, 32, 32)

    def key(n):
        if n.startswith("patch_embed."):
            leaf = n.split(".", 1)[1]
            return "patch_embed." + ("rpe_conv" if leaf == "rpe_lif" else "conv" + leaf[3:])
        if n == "pre_head_lif":
            return n
        blk, rest = n.split(".attn.") if ".attn." in n else n.split(".mlp.")
        leaf = rest[:-4]
        if ".attn." in n:
            return f"{blk}.attn." + {"q": "q", "k": "k", "v": "v", "attn": "core",
                                     "proj": "proj"}[leaf]
        return f"{blk}.mlp.{leaf}"
    outs, hs = _lif_outputs(m, key)
    with torch.no_grad():
        y = m(x)
    for h in hs:
        h.remove()
    rec = {}
    y_ref = oracle.spikformer_forward(m, x, conv_dtype=torch.float32, record=rec)
    for k, (xin, s, h) in rec.items():
        if k.endswith(".attn.qkv"):
            b = k[:-len(".qkv")]
            got = torch.cat([outs[b + ".q"], outs[b + ".k"], outs[b + ".v"]], -1)
        else:
            got = outs[k]
        got = got.reshape(s.shape) if got.numel() == s.numel() else got
        _assert_spikes(got, s, h, k)
        assert float(s.sum()) > 0, f"{k}: no spikes"
    assert len(rec) == 5 + 2 * 5
    np.testing.assert_allclose(y.numpy(), y_ref.numpy(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("groups, cin, cout, k, s, p", [
    (4, 8, 8, 3, 1, 1), (8, 8, 16, 3, 2, 1), (2, 6, 4, 1, 1, 0), (3, 6, 9, 5, 1, 2)])
def test_grouped_conv_oracle_pins(groups, cin, cout, k, s, p):
    """The oracle's grouped conv equals the per-group dense convolutions
    concatenated, and each group equals the C brute force; a plausible
    mistake (groups taken in the wrong order) fails."""
    g = torch.Generator().manual_seed(groups * 10 + k)
    x = (torch.rand(3, cin, 9, 7, generator=g) < 0.4).float()
    w = torch.randn(cout, cin // groups, k, k, generator=g)
    y = oracle.conv2d(x, w, None, s, p, groups=groups)
    np.testing.assert_array_equal(y.numpy(),
                                  oracle.conv2d_grouped_by_parts(x, w, None, s, p, groups).numpy())
    cg, og = cin // groups, cout // groups
    for gi in range(groups):
        bf = oracle.conv2d_bruteforce(x[:, gi * cg:(gi + 1) * cg], w[gi * og:(gi + 1) * og], s, p)
        np.testing.assert_allclose(y[:, gi * og:(gi + 1) * og].numpy(), bf, rtol=1e-6, atol=1e-6)
    w_swapped = torch.cat([w[og:], w[:og]]) if groups > 1 else w
    assert not torch.equal(oracle.conv2d(x, w_swapped, None, s, p, groups=groups), y)
