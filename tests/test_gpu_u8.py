"""One-byte spike copies between fused layers (the halo convolutions,
paired stride-2 launch, stem, head pool and materialisation read and write
NHWC copies of one byte per channel; catfuse_amd.set_spike_copy("u8")).

The motivation is the reference's fp32 -> uint8 spike exchange
(tests/test_32_spike_uint8.py:16-104).  The byte path widens each staged
byte to fp16 in LDS, so its K loop is the fp16 path's: every test here
compares the two formats bit for bit (spikes, membrane potentials, count
blocks, logits), layer by layer and over whole networks, and checks that
the byte copies were actually used (copy dtypes, no widening on the SEW
chain).  The fp16 path itself is checked against the oracle elsewhere."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from parity import lif_parity

pytestmark = pytest.mark.gpu


def _gen(s):
    return torch.Generator().manual_seed(s)


@pytest.fixture
def u8_off():
    from catfuse_amd import runtime
    yield
    runtime.set_spike_copy("f16")


def test_widened_byte_copy_reaches_fp16_readers(cuda, u8_off):
    """A byte copy read by a reader that takes fp16 copies only (here the
    NHWC max pool) is widened first (counted), with the same result as the
    fp16 copy."""
    from catfuse_amd import runtime
    g = _gen(9)
    vals = ((torch.rand(4, 2, 64, 12, 12, generator=g) < 0.3).float()
            * torch.randint(1, 4, (4, 2, 64, 12, 12), generator=g).float())
    ys = []
    for dt in (torch.float16, torch.uint8):
        x = _copy(vals, 64, dt, cuda)
        runtime.U8_WIDENED[0] = 0
        ys.append(runtime.maxpool_nhwc(x, 3, 2, 1).cpu())
        assert runtime.U8_WIDENED[0] == (1 if dt == torch.uint8 else 0)
    assert torch.equal(ys[0], ys[1])
    ref = torch.nn.functional.max_pool2d(vals.flatten(0, 1), 3, 2, 1).view_as(ys[0])
    assert torch.equal(ys[0], ref)


def test_copy_u8_to_f16_every_byte(cuda):
    from catfuse_amd import _hip
    src = torch.arange(256, dtype=torch.uint8).repeat(5).to(cuda)     # 1280 = 8 * 160
    dst = torch.full((1280,), -1.0, dtype=torch.float16, device=cuda)
    assert _hip.lib().cf_copy_u8_to_f16(src.data_ptr(), dst.data_ptr(), 1280,
                                        _hip.stream(cuda)) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), torch.arange(256, dtype=torch.float16).repeat(5))
    assert dst.view(torch.int16).min().item() >= 0          # +0, never -0


def _copy(vals, cp, dtype, dev):
    """A fused layer's output standing for vals [T, B, C, H, W] (small
    integers) as an NHWC copy of the given element type."""
    from catfuse_amd import runtime
    T, B, C, H, W = vals.shape
    nhwc = torch.zeros(T * B, H, W, cp, dtype=dtype)
    nhwc[..., :C] = vals.reshape(T * B, C, H, W).permute(0, 2, 3, 1).to(dtype)
    return runtime.lazy_output((T, B, C, H, W), nhwc.to(dev), dev)


def _layer(Cin, Cout, k, s, p, seed, v_th=0.5):
    from catfuse_amd import runtime
    g = _gen(seed)
    w = torch.randn(Cout, Cin, k, k, generator=g) * (2.0 / (Cin * k * k)) ** 0.5
    sc = torch.rand(Cout, generator=g) * 0.4 + 0.8
    sh = torch.randn(Cout, generator=g) * 0.1
    sh[::7] += 1.2                     # channels that fire on their bias alone
    return runtime.ConvLIFRunner(w.cuda(), sc.cuda(), sh.cuda(), None, s, p, 2.0, v_th, 0.0, True)


U8_CASES = [
    # name, T, B, Cin, Cout, H, W, k, s, p, rate, identity
    ("s1", 4, 3, 64, 64, 20, 20, 3, 1, 1, 0.2, True),
    ("s1_odd", 3, 2, 96, 96, 9, 11, 3, 1, 1, 0.3, True),
    ("c96", 4, 2, 64, 96, 16, 16, 3, 1, 1, 0.2, False),
    ("t6", 6, 2, 64, 64, 12, 12, 3, 1, 1, 0.3, True),
    ("s2", 4, 2, 64, 128, 28, 28, 3, 2, 1, 0.3, False),
    ("s2_t5", 5, 1, 32, 64, 15, 15, 3, 2, 1, 0.3, False),
    ("k1", 4, 2, 128, 64, 14, 14, 1, 1, 0, 0.3, False),
    ("k1s2", 4, 2, 128, 256, 28, 28, 1, 2, 0, 0.3, False),
    ("l4", 4, 2, 512, 512, 7, 7, 3, 1, 1, 0.2, True),
]


@pytest.mark.parametrize("case", U8_CASES, ids=[c[0] for c in U8_CASES])
def test_conv_u8_copies_equal_f16(cuda, case, u8_off):
    """cf_conv_halo_u8 (byte input, identity and output copies) against
    cf_conv_mfma on fp16 copies of the same values: spikes and membrane
    potentials bit for bit, and against the oracle."""
    from catfuse_amd import runtime
    name, T, B, Cin, Cout, H, W, k, s, p, rate, with_id = case
    r = _layer(Cin, Cout, k, s, p, seed=len(name) + 7 * T)
    g = _gen(100 + Cin)
    vals = ((torch.rand(T, B, Cin, H, W, generator=g) < rate).float()
            * torch.randint(1, 4, (T, B, Cin, H, W), generator=g).float())
    Ho, Wo = r.out_hw(H, W)
    idv = None
    if with_id:
        idv = ((torch.rand(T, B, Cout, Ho, Wo, generator=g) < 0.3).float()
               * torch.randint(1, 3, (T, B, Cout, Ho, Wo), generator=g).float())
    outs = {}
    for fmt, dt in (("f16", torch.float16), ("u8", torch.uint8)):
        runtime.set_spike_copy(fmt)
        x = _copy(vals, r.Cp, dt, cuda)
        ident = _copy(idv, runtime.pad32(Cout), dt, cuda) if with_id else None
        y, v = r.run_mfma(x, identity=ident)
        copy = runtime.shadow_of(y, (T * B, Ho, Wo, runtime.pad32(Cout)), resolve=False,
                                 u8_ok=True)
        assert copy is not None and copy.dtype == dt, (name, fmt)
        outs[fmt] = (y.clone().cpu(), v.clone().cpu(), int(runtime.count_of(y)[1].item()) != 0)
    (yf, vf, nzf), (yb, vb, nzb) = outs["f16"], outs["u8"]
    assert torch.equal(yf, yb), f"{name}: spikes differ"
    assert torch.equal(vf, vb), f"{name}: membrane differs"
    assert nzf == nzb
    spikes = yf - (idv if with_id else 0)
    conv = nn.Conv2d(Cin, Cout, k, s, p, bias=False)
    with torch.no_grad():
        conv.weight.copy_(r.weight.cpu())
    z = oracle.conv2d(vals.flatten(0, 1), conv.weight, None, s, p).float()
    z = z * r.bn_scale.cpu().view(1, -1, 1, 1) + r.bn_shift.cpu().view(1, -1, 1, 1)
    s_ref, v_ref, h_ref = oracle.lif_multistep(z.reshape(T, B, Cout, Ho, Wo), None,
                                               tau=2.0, v_threshold=0.5, v_reset=0.0)
    lif_parity(spikes.numpy(), vf.numpy(), s_ref, v_ref, h_ref, v_th=0.5, what=name)


def test_pair_u8_equals_f16(cuda, u8_off):
    """cf_conv_halo_pair_u8 (a block's stride-2 conv1 and 1x1 downsample on
    one byte copy) against cf_conv_halo_pair on the fp16 copy."""
    from catfuse_amd import runtime
    T, B, C, H = 4, 2, 64, 28
    ra, rb = _layer(C, 128, 3, 2, 1, seed=3), _layer(C, 128, 1, 2, 0, seed=4)
    g = _gen(5)
    vals = (torch.rand(T, B, C, H, H, generator=g) < 0.3).float()
    res = {}
    for fmt, dt in (("f16", torch.float16), ("u8", torch.uint8)):
        runtime.set_spike_copy(fmt)
        x = _copy(vals, ra.Cp, dt, cuda)
        assert runtime.halo_pair_supported(ra, rb, x)
        oa, va, ob, vb = runtime.run_halo_pair(ra, rb, x)
        ca = runtime.shadow_of(oa, (T * B, 14, 14, 128), resolve=False, u8_ok=True)
        assert ca.dtype == dt
        res[fmt] = [t.clone().cpu() for t in (oa, va, ob, vb)]
    for a, b in zip(res["f16"], res["u8"]):
        assert torch.equal(a, b)


def _sew(v_th, seed=11):
    from catfuse_amd import snn
    m = snn.sew_resnet18(num_classes=100, cnf="ADD", v_threshold=v_th)
    g = _gen(seed)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    return m.eval()


@pytest.mark.parametrize("v_th", [1.0, 0.1], ids=["kaiming", "live"])
def test_sew_resnet18_u8_chain_equals_f16(cuda, v_th, u8_off):
    """SEW-ResNet18 (T=4, B=2, 128x128: layer 4 at 4x4, where its 1x1
    downsample still runs the halo kernel) with byte copies between all fused
    layers against the fp16 copies: every layer's output and the logits bit
    for bit; the chain's copies are bytes end to end (no widening), from the
    stem (given the direct-encoded image as a stride-0 view over T) to the
    head's average pool.  The silent net takes StaticZero from
    layer 2 on (output elision and identity aliases on byte copies); the
    live one runs every conv on the matrix cores."""
    import catfuse_amd
    from catfuse_amd import runtime, snn
    m = _sew(v_th)
    T, B, hw = 4, 2, 128
    img = torch.randn(B, 3, hw, hw, generator=_gen(12))
    # direct encoding as a stride-0 view over T: the fused stem kernel (the
    # chain's first byte-copy producer) takes it
    x = img.to(cuda).unsqueeze(0).expand(T, B, 3, hw, hw)
    res = {}
    for fmt in ("f16", "u8"):
        runtime.set_spike_copy(fmt)
        fused, _ = catfuse_amd.optimize(m, T=T)
        outs, dts = [], []

        def record(mod, a, o):
            dts.append(getattr(o, "_cf_nhwc", (None,))[0])
            outs.append(o.detach().float().cpu())

        hooks = [mod.register_forward_hook(record)
                 for mod in fused.modules() if type(mod).__name__ == "CTFSEWBasicBlock"]
        runtime.U8_WIDENED[0] = 0
        with torch.no_grad():
            snn.functional.reset_net(fused)
            y = fused(x)
        torch.cuda.synchronize()
        for h in hooks:
            h.remove()
        assert len(outs) == 8
        want = torch.uint8 if fmt == "u8" else torch.float16
        assert all(d is not None and d.dtype == want for d in dts), fmt
        if fmt == "u8":
            assert runtime.U8_WIDENED[0] == 0
        res[fmt] = (y.cpu(), outs)
    assert torch.equal(res["f16"][0], res["u8"][0])
    for a, b in zip(res["f16"][1], res["u8"][1]):
        assert torch.equal(a, b)


def test_sew_resnet18_u8_graph_replay(cuda, u8_off):
    """The byte-copy forward captured as a HIP graph: every replay (with
    eager work and synchronisation between them) equals the eager forward."""
    import catfuse_amd
    from catfuse_amd import runtime, snn
    runtime.set_spike_copy("u8")
    m = _sew(0.1)
    T, B, hw = 4, 2, 64
    img = torch.randn(B, 3, hw, hw, generator=_gen(13)).to(cuda)
    x = img.unsqueeze(0).expand(T, B, 3, hw, hw)
    fused, _ = catfuse_amd.optimize(m, T=T)
    with torch.no_grad():
        snn.functional.reset_net(fused)
        y_ref = fused(x).clone()
        graphed = catfuse_amd.capture(fused, x)
        for i in range(3):
            y = graphed(img)
            torch.cuda.synchronize()
            assert torch.equal(y, y_ref), f"replay {i}"
            _ = (img * 2).sum().item()     # eager work between replays


def test_vgg_with_u8_selected_equals_f16(cuda, u8_off):
    """A network whose fused layers produce and read fp16 copies only
    (VGG's analog first layer, pooled epilogues, token-view linears) with
    byte copies selected: the layers that could take byte copies receive
    fp16 ones and keep that format, the logits equal the fp16 run's bit for
    bit."""
    import catfuse_amd
    from catfuse_amd import runtime, snn
    g = _gen(21)
    m = snn.spiking_vgg11_bn(num_classes=10, v_threshold=0.1)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    m.eval()
    T, B = 4, 4
    x = torch.randn(B, 3, 32, 32, generator=_gen(22)).unsqueeze(0).expand(T, B, 3, 32, 32)
    ys = {}
    for fmt in ("f16", "u8"):
        runtime.set_spike_copy(fmt)
        fused, _ = catfuse_amd.optimize(m, T=T)
        with torch.no_grad():
            snn.functional.reset_net(fused)
            ys[fmt] = fused(x.to(cuda)).cpu()
    assert torch.equal(ys["f16"], ys["u8"])
