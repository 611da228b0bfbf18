"""Fused grouped / depthwise Conv -> BN -> LIF (cf_conv_grouped_lif) against
the CPU oracle: spikes under the north-star flip rule, the membrane within
1e-4 relative; the analog-input form, the StaticZero route and the state
carried between calls bit for bit; a MobileNet-style network through
optimize layer by layer."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from parity import lif_parity

pytestmark = pytest.mark.gpu


def _gen(s):
    return torch.Generator().manual_seed(s)


def _layer(cin, cout, k, s, p, groups, seed, v_th=1.0, bias=True):
    from catfuse_amd import snn
    g = _gen(seed)
    conv = snn.Conv2d(cin, cout, k, s, p, groups=groups, bias=bias)
    bn = snn.BatchNorm2d(cout)
    lif = snn.LIFNode(tau=2.0, v_threshold=v_th, v_reset=0.0, step_mode="m")
    with torch.no_grad():
        fan = (cin // groups) * k * k
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * (4.0 / fan) ** 0.5)
        if bias:
            conv.bias.copy_(torch.randn(cout, generator=g) * 0.1)
        bn.running_mean.copy_(torch.randn(cout, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(cout, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(cout, generator=g) * 0.4 + 0.8)
        bn.bias.copy_(torch.randn(cout, generator=g) * 0.1 + 0.3)
    return conv, bn.eval(), lif


CASES = [
    # name, T, B, Cin, Cout, groups, H, k, s, p
    ("dw3", 4, 2, 64, 64, 64, 20, 3, 1, 1),
    ("dw3s2", 4, 2, 48, 48, 48, 17, 3, 2, 1),
    ("dw3x2", 3, 2, 32, 64, 32, 14, 3, 1, 1),      # depthwise with channel multiplier 2
    ("g4", 4, 2, 64, 128, 4, 12, 3, 1, 1),
    ("g2_1x1", 4, 3, 40, 24, 2, 9, 1, 1, 0),
    ("g3_5x5", 2, 2, 12, 18, 3, 11, 5, 2, 2),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_grouped_conv_bn_lif_parity(cuda, case):
    from catfuse_amd.patterns import PartialFusionGroupedConvBNLIF
    name, T, B, cin, cout, groups, H, k, s, p = case
    conv, bn, lif = _layer(cin, cout, k, s, p, groups, seed=len(name) * 7 + H)
    x = (torch.rand(T, B, cin, H, H, generator=_gen(H)) < 0.3).float()
    pat = PartialFusionGroupedConvBNLIF.from_sj_modules(conv, bn, lif).to(cuda)
    out = pat(x.to(cuda))
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif)
    assert s_ref.any() and not s_ref.all()
    v = pat.state.tensor.cpu().contiguous()            # [B, Cout, Ho, Wo] (channels-last storage)
    lif_parity(out.cpu().numpy(), v.numpy(), s_ref, v_ref, h_ref, what=name)
    # state carried into a second call equals one call over all the steps
    pat.reset()
    h = T // 2
    if h >= 1:
        o1 = pat(x[:h].to(cuda)).clone()
        o2 = pat(x[h:].to(cuda))
        assert torch.equal(torch.cat([o1, o2]), out)
        assert torch.equal(pat.state.tensor, v.to(cuda))


def test_grouped_conv_analog_input(cuda):
    """An analog input is read in fp32 (stride-0 time axis: one image for
    every step) and matches the oracle."""
    from catfuse_amd.patterns import PartialFusionGroupedConvBNLIF
    conv, bn, lif = _layer(12, 24, 3, 1, 1, 3, seed=5)
    img = torch.randn(2, 12, 15, 15, generator=_gen(6))
    for x in (img.unsqueeze(0).expand(4, 2, 12, 15, 15),
              torch.randn(3, 2, 12, 15, 15, generator=_gen(7))):
        pat = PartialFusionGroupedConvBNLIF.from_sj_modules(conv, bn, lif).to(cuda)
        out = pat(x.to(cuda) if x.stride(0) else img.to(cuda).unsqueeze(0).expand(x.shape))
        s_ref, v_ref, h_ref = oracle.conv_bn_lif(x.contiguous(), conv, bn, lif)
        lif_parity(out.cpu().numpy(), pat.state.tensor.cpu().contiguous().numpy(), s_ref, v_ref,
                   h_ref, what="analog")


def test_grouped_conv_static_zero_route(cuda):
    """An all-zero input that carries a zero count block (a fused layer's
    silent output) takes StaticZero; it equals the dense evaluation of the
    same zero input bit for bit, and publishes the output's count block."""
    from catfuse_amd import runtime
    from catfuse_amd.patterns import PartialFusionGroupedConvBNLIF
    conv, bn, lif = _layer(32, 32, 3, 1, 1, 32, seed=9, v_th=0.25)
    T, B, H = 4, 2, 10
    pat = PartialFusionGroupedConvBNLIF.from_sj_modules(conv, bn, lif).to(cuda)
    nhwc = torch.zeros(T * B, H, H, 32, dtype=torch.float16, device=cuda)
    xz = runtime.lazy_output((T, B, 32, H, H), nhwc, cuda)
    blk = runtime.count_block(cuda)
    runtime.attach_count(xz, blk, [0])                  # published count 0: all zero
    y_zero = pat(xz).clone()
    v_zero = pat.state.tensor.clone()
    pat.reset()
    y_dense = pat(torch.zeros(T, B, 32, H, H, device=cuda))
    assert torch.equal(y_zero, y_dense) and torch.equal(v_zero, pat.state.tensor)
    assert bool(y_dense.any())                          # biased channels spike
    cnt = runtime.count_of(y_dense)
    assert cnt is not None and int(cnt[1].item()) > 0


def _mobilenet_like():
    from catfuse_amd import snn
    mods = []
    cfg = [(3, 16, 3, 1, 1, 1), (16, 16, 3, 1, 1, 16), (16, 32, 1, 1, 0, 1),
           (32, 32, 3, 2, 1, 32), (32, 64, 1, 1, 0, 1), (64, 64, 3, 1, 1, 64)]
    for i, (ci, co, k, s, p, g) in enumerate(cfg):
        conv, bn, lif = _layer(ci, co, k, s, p, g, seed=40 + i, v_th=0.5, bias=False)
        mods += [conv, bn, lif]
    m = nn.Sequential(*mods)
    snn.functional.set_step_mode(m, "m")
    return m.eval()


def test_mobilenet_like_network_per_layer(cuda):
    """Dense and depthwise layers interleaved (a MobileNet-style SNN): every
    fused layer against the oracle on the input it received; the depthwise
    layers read the previous fused layer's fp16 NHWC copy."""
    import catfuse_amd
    from catfuse_amd.patterns import PartialFusionGroupedConvBNLIF
    m = _mobilenet_like()
    fused, stats = catfuse_amd.optimize(m, T=4)
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"] == 6
    assert sum(isinstance(f, PartialFusionGroupedConvBNLIF) for f in fused) == 3
    recs, hs = [], []
    orig = [tuple(m[3 * i:3 * i + 3]) for i in range(6)]
    for f, o in zip(fused, orig):
        hs.append(f.register_forward_hook(
            lambda mod, a, out, o=o: recs.append((o, a[0].detach().cpu(), out.detach().cpu()))))
    img = torch.randn(2, 3, 24, 24, generator=_gen(50))
    with torch.no_grad():
        fused(img.to(cuda).unsqueeze(0).expand(4, 2, 3, 24, 24))
    torch.cuda.synchronize()
    for h in hs:
        h.remove()
    catfuse_amd.check_status()
    assert len(recs) == 6
    for (conv, bn, lif), xin, out in recs:
        s_ref, _, h_ref = oracle.conv_bn_lif(xin.contiguous(), conv, bn, lif)
        lif_parity(out.numpy(), None, s_ref, None, h_ref, v_th=lif.v_threshold,
                   what=f"groups={conv.groups}")
        assert bool(xin.any()) and bool(out.any())
