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
