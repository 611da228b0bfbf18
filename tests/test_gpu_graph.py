"""HIP-graph replay of a fused network equals its eager forward, replay
after replay, with eager work between the replays."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _net(dev, T):
    import catfuse_amd
    from catfuse_amd import snn
    g = torch.Generator().manual_seed(3)
    m = snn.sew_resnet18(num_classes=10, cnf="ADD", tau=2.0, v_threshold=1.0, v_reset=0.0)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, _ = catfuse_amd.optimize(m.eval(), device=dev, T=T)
    return fused.eval()


@pytest.mark.parametrize("expanded", [True, False])
def test_graph_replays_match_eager(cuda, expanded):
    from catfuse_amd import graph, snn
    T, B, HW = 2, 2, 64
    fused = _net(cuda, T)
    gen = torch.Generator(device=cuda).manual_seed(0)
    imgs = [torch.randn(B, 3, HW, HW, device=cuda, generator=gen) for _ in range(3)]

    def as_input(img):
        x = img.unsqueeze(0).expand(T, B, 3, HW, HW)
        return x if expanded else x.contiguous()

    with torch.no_grad():
        eager = []
        for img in imgs:
            snn.functional.reset_net(fused)
            eager.append(fused(as_input(img)).clone())
        graphed = graph.capture(fused, as_input(imgs[0]))
        for rep in range(2):
            for i, img in enumerate(imgs):
                y = graphed(as_input(img)).clone()
                torch.cuda.synchronize()
                assert torch.equal(y, eager[i]), f"replay {rep}, input {i}"
                # eager work between replays (same model, other input)
                snn.functional.reset_net(fused)
                z = fused(as_input(imgs[(i + 1) % 3]))
                assert torch.equal(z, eager[(i + 1) % 3])
        with pytest.raises(ValueError):
            graphed(torch.zeros(T, B + 1, 3, HW, HW, device=cuda))


def test_graph_replays_of_a_model_ending_in_a_fused_conv(cuda):
    """A captured forward whose output is a fused layer's NHWC-backed tensor
    (a feature extractor): every replay's fp32 output holds that replay's
    values (the fp16 -> fp32 fill is part of the graph)."""
    import catfuse_amd
    from catfuse_amd import graph, snn
    g = torch.Generator().manual_seed(4)
    m = torch.nn.Sequential(
        snn.Conv2d(16, 32, 3, 1, 1, bias=False), snn.BatchNorm2d(32), snn.LIFNode(v_threshold=0.3),
        snn.Conv2d(32, 32, 3, 1, 1, bias=False), snn.BatchNorm2d(32), snn.LIFNode(v_threshold=0.3))
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, _ = catfuse_amd.optimize(m.eval(), device=cuda, T=4)
    T, B = 4, 2
    xs = [(torch.rand(T, B, 16, 24, 24, generator=g) < 0.3).float().to(cuda) for _ in range(3)]
    with torch.no_grad():
        eager = []
        for x in xs:
            snn.functional.reset_net(fused)
            eager.append(fused(x).clone())
        assert not torch.equal(eager[0], eager[1])
        graphed = graph.capture(fused, xs[0])
        for rep in range(2):
            for i, x in enumerate(xs):
                y = graphed(x).clone()
                torch.cuda.synchronize()
                assert torch.equal(y, eager[i]), f"replay {rep}, input {i}"
                snn.functional.reset_net(fused)
                fused(xs[(i + 2) % 3])     # eager work between replays


def test_graph_replays_keep_elided_outputs_and_states_current(cuda):
    """Replays alternating between an all-zero input (every fused conv takes
    StaticZero: its output recorded in a descriptor, its state kept per
    channel) and live ones: after every replay the output and every fused
    layer's membrane state equal the eager forward's, bit for bit."""
    import catfuse_amd
    from catfuse_amd import graph, snn
    from catfuse_amd.state import StateBuffer
    g = torch.Generator().manual_seed(5)
    m = torch.nn.Sequential(
        snn.Conv2d(16, 32, 3, 1, 1, bias=False), snn.BatchNorm2d(32), snn.LIFNode(v_threshold=0.3),
        snn.Conv2d(32, 32, 3, 1, 1, bias=False), snn.BatchNorm2d(32), snn.LIFNode(v_threshold=0.3),
        snn.Conv2d(32, 32, 3, 1, 1, bias=False), snn.BatchNorm2d(32), snn.LIFNode(v_threshold=0.3))
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.BatchNorm2d):
                mod.bias.fill_(-0.2)     # no channel fires on its bias alone
    fused, _ = catfuse_amd.optimize(m.eval(), device=cuda, T=4)
    bufs = [mod.state for mod in fused.modules() if isinstance(getattr(mod, "state", None), StateBuffer)]
    assert len(bufs) == 3
    T, B = 4, 2
    live = [(torch.rand(T, B, 16, 24, 24, generator=g) < 0.3).float().to(cuda) for _ in range(2)]
    xs = [torch.zeros_like(live[0]), live[0], torch.zeros_like(live[0]), live[1]]

    def states():
        return [b.tensor.clone() for b in bufs]

    with torch.no_grad():
        eager = []
        for x in xs:
            snn.functional.reset_net(fused)
            y = fused(x).clone()
            eager.append((y, states()))
        assert bool(eager[1][0].any()) and not bool(eager[0][0].any())
        graphed = graph.capture(fused, xs[1])
        for rep in range(2):
            for i, x in enumerate(xs):
                y = graphed(x).clone()
                got = states()
                torch.cuda.synchronize()
                assert torch.equal(y, eager[i][0]), f"replay {rep}, input {i}: output"
                for k, (a, b) in enumerate(zip(got, eager[i][1])):
                    assert torch.equal(a, b), f"replay {rep}, input {i}: state of layer {k}"


@pytest.mark.parametrize("live", [False, True])
def test_graph_replays_of_vgg(cuda, live):
    """Spiking VGG-11-BN: pooled conv epilogues, the analog conv + avg pool,
    the token-view Linear-LIFs, the lazy flatten and the head Linear over
    the copy, with (live) and without (silent: elided outputs, per-channel
    states) activity past the first layers; every replay equals the eager
    forward with eager work between replays."""
    import catfuse_amd
    from catfuse_amd import graph, snn
    from catfuse_amd.patterns import FusedFlatten, FusedLinear
    T, B = 4, 64
    g = torch.Generator().manual_seed(11)
    m = snn.spiking_vgg11_bn(num_classes=10, v_threshold=0.1 if live else 1.0)
    snn.functional.set_step_mode(m, "m")
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    fused, _ = catfuse_amd.optimize(m.eval(), device=cuda, T=T)
    fused = fused.eval()
    assert isinstance(fused.flatten, FusedFlatten) and isinstance(fused.classifier[-1], FusedLinear)
    gen = torch.Generator(device=cuda).manual_seed(1)
    imgs = [torch.randn(B, 3, 32, 32, device=cuda, generator=gen) for _ in range(3)]

    def as_input(img):
        return img.unsqueeze(0).expand(T, B, 3, 32, 32)

    with torch.no_grad():
        eager = []
        for img in imgs:
            snn.functional.reset_net(fused)
            eager.append(fused(as_input(img)).clone())
        graphed = graph.capture(fused, as_input(imgs[0]))
        for rep in range(2):
            for i, img in enumerate(imgs):
                y = graphed(as_input(img)).clone()
                torch.cuda.synchronize()
                assert torch.equal(y, eager[i]), f"replay {rep}, input {i}"
                snn.functional.reset_net(fused)
                z = fused(as_input(imgs[(i + 1) % 3]))
                assert torch.equal(z, eager[(i + 1) % 3])
    assert fused.flatten.fallback_calls == 0 and fused.classifier[-1].fallback_calls == 0


@pytest.mark.parametrize("v_th", [1.0, 0.2])
def test_graph_replays_of_spikformer(cuda, v_th):
    """A small Spikformer (patch splitter, two blocks, the pre-head LIF as
    FusedLIF, the token mean read from the last copy): every replay equals
    the eager forward, with eager work between replays."""
    import catfuse_amd
    from catfuse_amd import graph, snn
    from catfuse_amd.patterns import FusedLIF
    T, B = 4, 2
    g = torch.Generator().manual_seed(5)
    net = snn.Spikformer(img_size=32, num_classes=10, embed_dim=64, num_heads=2, depth=2,
                         pools=(0, 1), v_threshold=v_th)
    snn.kaiming_init(net, g)
    snn.randomize_bn(net, g)
    fused, stats = catfuse_amd.optimize(net.eval(), device=cuda, T=T)
    fused = fused.eval()
    assert isinstance(fused.pre_head_lif, FusedLIF)
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"]
    gen = torch.Generator(device=cuda).manual_seed(2)
    imgs = [torch.randn(B, 3, 32, 32, device=cuda, generator=gen) for _ in range(3)]

    def as_input(img):
        return img.unsqueeze(0).expand(T, B, 3, 32, 32)

    with torch.no_grad():
        eager = []
        for img in imgs:
            snn.functional.reset_net(fused)
            eager.append(fused(as_input(img)).clone())
        graphed = graph.capture(fused, as_input(imgs[0]))
        for rep in range(2):
            for i, img in enumerate(imgs):
                y = graphed(as_input(img)).clone()
                torch.cuda.synchronize()
                assert torch.equal(y, eager[i]), f"replay {rep}, input {i}"
                snn.functional.reset_net(fused)
                z = fused(as_input(imgs[(i + 1) % 3]))
                assert torch.equal(z, eager[(i + 1) % 3])


def test_launch_stream_is_torch_current_stream(cuda):
    """The handle the launches use is torch's current stream: the default
    stream, a side stream selected with torch.cuda.stream, and the capture
    stream of a graph being recorded."""
    from catfuse_amd import _hip
    assert _hip.stream(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    side = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(side):
        assert _hip.stream(cuda) == side.cuda_stream
    g = torch.cuda.CUDAGraph()
    x = torch.zeros(8, device=cuda)
    seen = []
    with torch.cuda.graph(g):
        seen.append((_hip.stream(cuda), torch.cuda.current_stream(cuda).cuda_stream))
        x.add_(1.0)
    assert seen[0][0] == seen[0][1]
