"""The eager forward's repeat path: launch plans cached per input signature
(ConvLIFRunner._dense_repeat, runtime.halo_pair_repeat) give the same
outputs, membrane states, copies and routes as the general path, launch
for launch, and are dropped when a layer's parameters change in place."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _sew(dev, v_th, T):
    import catfuse_amd
    from catfuse_amd import snn
    g = torch.Generator().manual_seed(11)
    m = snn.sew_resnet18(num_classes=10, cnf="ADD", tau=2.0, v_threshold=v_th, v_reset=0.0)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, _ = catfuse_amd.optimize(m.eval(), device=dev, T=T)
    return fused.eval()


def _states(fused):
    from catfuse_amd.state import StateBuffer
    out = []
    for mod in fused.modules():
        st = getattr(mod, "state", None)
        if isinstance(st, StateBuffer) and st.tensor is not None:
            out.append(st.tensor.clone())
    return out


def _run(fused, xs):
    from catfuse_amd import snn
    res = []
    for x in xs:
        snn.functional.reset_net(fused)
        y = fused(x).clone()
        res.append((y, _states(fused)))
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("fmt", ["f16", "u8"])
@pytest.mark.parametrize("v_th", [1.0, 0.3])
def test_repeat_path_matches_general_path(cuda, monkeypatch, fmt, v_th):
    """SEW-ResNet-18 at T=4 on silent, live and all-zero inputs (StaticZero
    with elided copies and per-channel states, dense launches, the paired
    stride-2 launches): every logit and every fused layer's state equal the
    general path's, bit for bit, with the repeat path taken on most
    launches."""
    from catfuse_amd import runtime
    T, B, HW = 4, 2, 64
    fused = _sew(cuda, v_th, T)
    gen = torch.Generator(device=cuda).manual_seed(1)
    xs = [torch.randn(B, 3, HW, HW, device=cuda, generator=gen).unsqueeze(0).expand(T, B, 3, HW, HW)
          for _ in range(2)]
    xs = [xs[0], torch.zeros_like(xs[0]), xs[1], xs[0]]
    taken = {"dense": 0, "pair": 0}
    dense, pair = runtime.ConvLIFRunner._dense_repeat, runtime.halo_pair_repeat

    def count_dense(self, *a, **k):
        r = dense(self, *a, **k)
        taken["dense"] += r is not None
        return r

    def count_pair(*a, **k):
        r = pair(*a, **k)
        taken["pair"] += r is not None
        return r

    monkeypatch.setattr(runtime.ConvLIFRunner, "_dense_repeat", count_dense)
    monkeypatch.setattr(runtime, "halo_pair_repeat", count_pair)
    runtime.set_spike_copy(fmt)
    try:
        with torch.no_grad():
            fast = _run(fused, xs)
            runtime.REPEAT_PLANS = False
            try:
                general = _run(fused, xs)
            finally:
                runtime.REPEAT_PLANS = True
    finally:
        runtime.set_spike_copy("f16")
    # single convs and stride-2 pairs (layer2, layer3; layer4's 2x2 output is
    # below the pair kernel's 4x4) of every forward
    assert taken["dense"] >= 8 * len(xs) and taken["pair"] >= 2 * len(xs), taken
    for i, ((yf, sf), (yg, sg)) in enumerate(zip(fast, general)):
        assert torch.equal(yf, yg), f"input {i}: logits"
        assert len(sf) == len(sg)
        for k, (a, b) in enumerate(zip(sf, sg)):
            assert torch.equal(a, b), f"input {i}: state of layer {k}"
    if v_th < 1.0:
        assert not torch.equal(fast[0][0], fast[1][0])


def test_repeat_plans_follow_in_place_parameter_changes(cuda):
    """A plan holds the packed weights of its layer: changing conv weights
    in place between two forwards repacks the layers, and the forward after
    it equals the general path's on the new parameters."""
    from catfuse_amd import runtime
    T, B, HW = 4, 2, 64
    fused = _sew(cuda, 0.3, T)
    gen = torch.Generator(device=cuda).manual_seed(2)
    x = torch.randn(B, 3, HW, HW, device=cuda, generator=gen).unsqueeze(0).expand(T, B, 3, HW, HW)
    with torch.no_grad():
        before = _run(fused, [x, x])
        blk = fused.layer2[0]
        blk.fused_first.weight.mul_(1.25)          # the paired stride-2 conv
        blk.fused_second.weight.mul_(0.8)          # a single conv
        fast = _run(fused, [x])
        runtime.REPEAT_PLANS = False
        try:
            general = _run(fused, [x])
        finally:
            runtime.REPEAT_PLANS = True
    assert not torch.equal(before[1][0], fast[0][0])
    assert torch.equal(fast[0][0], general[0][0])
    for a, b in zip(fast[0][1], general[0][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("v_th", [1.0, 0.1])
def test_repeat_path_matches_general_path_vgg(cuda, monkeypatch, v_th):
    """Spiking VGG-11-BN (the pooled epilogue's Conv-BN-AvgPool-LIF layers,
    Conv-BN-LIF layers, the Linear-LIF classifier) at T=4 on live and
    all-zero inputs: logits and every fused layer's state equal the general
    path's bit for bit, with the repeat path taken by the pooled layers."""
    import catfuse_amd
    from catfuse_amd import runtime, snn
    g = torch.Generator().manual_seed(12)
    m = snn.spiking_vgg11_bn(num_classes=10, v_threshold=v_th)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, _ = catfuse_amd.optimize(m.eval(), device=cuda, T=4)
    fused.eval()
    T, B = 4, 8
    gen = torch.Generator(device=cuda).manual_seed(3)
    x0 = torch.randn(B, 3, 32, 32, device=cuda, generator=gen).unsqueeze(0).expand(T, B, 3, 32, 32)
    xs = [x0, torch.zeros_like(x0), x0]
    pooled = {"n": 0}
    dense = runtime.ConvLIFRunner._dense_repeat

    def count(self, *a, **k):
        r = dense(self, *a, **k)
        if r is not None and len(a) > 4 and a[4] == runtime.EPI_POOL:
            pooled["n"] += 1
        return r

    monkeypatch.setattr(runtime.ConvLIFRunner, "_dense_repeat", count)
    with torch.no_grad():
        fast = _run(fused, xs)
        runtime.REPEAT_PLANS = False
        try:
            general = _run(fused, xs)
        finally:
            runtime.REPEAT_PLANS = True
    assert pooled["n"] >= len(xs), pooled
    for i, ((yf, sf), (yg, sg)) in enumerate(zip(fast, general)):
        assert torch.equal(yf, yg), f"input {i}: logits"
        assert len(sf) == len(sg)
        for k, (a, b) in enumerate(zip(sf, sg)):
            assert torch.equal(a, b), f"input {i}: state of layer {k}"


@pytest.mark.parametrize("v_th", [1.0, 0.2])
def test_repeat_path_matches_general_path_spikformer(cuda, monkeypatch, v_th):
    """A small Spikformer (token Linear-BN-LIF layers with and without the
    residual identity, attention between them): logits and every fused
    layer's state equal the general path's bit for bit on live and
    all-zero inputs, with the token layers' repeat path taken."""
    import catfuse_amd
    from catfuse_amd import runtime, snn
    T, B = 4, 2
    g = torch.Generator().manual_seed(5)
    net = snn.Spikformer(img_size=32, num_classes=10, embed_dim=64, num_heads=2, depth=2,
                         pools=(0, 1), v_threshold=v_th)
    snn.kaiming_init(net, g)
    snn.randomize_bn(net, g)
    fused, _ = catfuse_amd.optimize(net.eval(), device=cuda, T=T)
    fused = fused.eval()
    gen = torch.Generator(device=cuda).manual_seed(2)
    x0 = torch.randn(B, 3, 32, 32, device=cuda, generator=gen).unsqueeze(0).expand(T, B, 3, 32, 32)
    x1 = torch.randn(B, 3, 32, 32, device=cuda, generator=gen).unsqueeze(0).expand(T, B, 3, 32, 32)
    xs = [x0, torch.zeros_like(x0), x1, x0]
    taken = {"n": 0}
    tokens = runtime.ConvLIFRunner._tokens_repeat

    def count(self, *a, **k):
        r = tokens(self, *a, **k)
        taken["n"] += r is not None
        return r

    monkeypatch.setattr(runtime.ConvLIFRunner, "_tokens_repeat", count)
    with torch.no_grad():
        fast = _run(fused, xs)
        runtime.REPEAT_PLANS = False
        try:
            general = _run(fused, xs)
        finally:
            runtime.REPEAT_PLANS = True
    assert taken["n"] >= 4 * len(xs), taken
    for i, ((yf, sf), (yg, sg)) in enumerate(zip(fast, general)):
        assert torch.equal(yf, yg), f"input {i}: logits"
        assert len(sf) == len(sg)
        for k, (a, b) in enumerate(zip(sf, sg)):
            assert torch.equal(a, b), f"input {i}: state of layer {k}"
