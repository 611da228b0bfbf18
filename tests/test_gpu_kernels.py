"""Kernel-level parity of the gfx950 HIP path against the CPU oracle.

Element-wise LIF tails, prescan masks/classes, route words and nonzero
counts are compared bit-exactly; fused Conv->BN->LIF layers use the LIF
tolerance in tests/parity.py.  SparseFlow and DenseKeep routes of the same
conv are compared bit-exactly with each other.
"""
import numpy as np
import pytest
import torch

import oracle
from parity import lif_parity, membrane_parity, pooled_parity

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# matrix-core layout
# ---------------------------------------------------------------------------

def test_mfma_layout_probe(cuda):
    from catfuse_amd import _hip
    g = _gen(0)
    A = torch.randint(-8, 9, (32, 16), generator=g).to(torch.float16)
    B = torch.randint(-8, 9, (16, 32), generator=g).to(torch.float16)
    Ad, Bd = A.to(cuda), B.to(cuda)
    D = torch.zeros(32, 32, dtype=torch.float32, device=cuda)
    _hip.check(_hip.lib().cf_probe_mfma_layout(Ad.data_ptr(), Bd.data_ptr(), D.data_ptr(),
                                               _hip.stream(cuda)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(D.cpu().numpy(), (A.float() @ B.float()).numpy())


# ---------------------------------------------------------------------------
# LIF family: bit-exact
# ---------------------------------------------------------------------------

LIF_VARIANTS = [
    dict(tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True),
    dict(tau=3.0, v_threshold=1.0, v_reset=0.0, decay_input=True),
    dict(tau=2.0, v_threshold=0.5, v_reset=None, decay_input=True),
    dict(tau=1.7, v_threshold=1.0, v_reset=0.0, decay_input=False),
    dict(tau=2.5, v_threshold=1.0, v_reset=None, decay_input=False),
    dict(tau=2.0, v_threshold=1.0, v_reset=-0.2, decay_input=True),
]


@pytest.mark.parametrize("variant", range(len(LIF_VARIANTS)))
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("shape", [(4, 2, 16, 7, 9), (4, 3, 8, 8, 8), (7, 2, 4, 5, 8)])
def test_lif_multistep_bit_exact(cuda, variant, mode, shape):
    from catfuse_amd import runtime
    p = LIF_VARIANTS[variant]
    T, B, C, H, W = shape
    g = _gen(100 * variant + mode)
    z = torch.randn(shape, generator=g) * 1.2
    z2 = torch.randn(shape, generator=g) * 0.5
    sc = torch.rand(C, generator=g) + 0.5
    sh = torch.randn(C, generator=g) * 0.2
    v0 = torch.randn(B, C, H, W, generator=g) * 0.4
    s_ref, v_ref, _ = oracle.lif_multistep(z, v0, mode=mode, z2=z2, scale=sc, shift=sh, C=C,
                                           HW=H * W, **p)
    s, v = runtime.lif_multistep(z.to(cuda), v0.to(cuda), mode=mode, z2=z2.to(cuda),
                                 scale=sc.to(cuda), shift=sh.to(cuda), channels=C, hw=H * W, **p)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(v.cpu().numpy(), v_ref)


def test_lif_uint8_spikes_and_default_v(cuda):
    from catfuse_amd import runtime
    z = torch.randn(5, 1000, generator=_gen(5)) * 2
    s_ref, v_ref, _ = oracle.lif_multistep(z)
    s, v = runtime.lif_multistep(z.to(cuda), None, spike_dtype=torch.uint8)
    assert s.dtype == torch.uint8
    np.testing.assert_array_equal(s.cpu().numpy().astype(np.float32), s_ref)
    np.testing.assert_array_equal(v.cpu().numpy(), v_ref)


def test_lif_sequential_api(cuda):
    from catfuse_amd.sparseflow.lif_seq_kernel import lif_sequential
    z = torch.randn(4, 2, 3, 5, 5, generator=_gen(9))
    v0 = torch.zeros(2, 3, 5, 5)
    s, v = lif_sequential(z.to(cuda), v0.to(cuda), tau=2.0, v_threshold=1.0, v_reset=0.0)
    s_ref, v_ref, _ = oracle.lif_multistep(z, v0)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(v.cpu().numpy(), v_ref)


@pytest.mark.parametrize("shape", [(4, 2, 8, 16, 16), (3, 1, 5, 7, 9), (5, 2, 3, 9, 12),
                                   (9, 1, 4, 8, 20)])
@pytest.mark.parametrize("variant", [0, 2, 5])
def test_avgpool2x2_lif_bit_exact(cuda, shape, variant):
    """Both kernels (two outputs per thread when W is a multiple of 4, else
    one), steps beyond a 4-step load chunk, odd heights, every LIF
    specialisation, a carried membrane and uint8 spikes."""
    from catfuse_amd import runtime
    p = LIF_VARIANTS[variant]
    g = _gen(11 + variant)
    x = torch.rand(shape, generator=g) * 3
    T, B, C, H, W = shape
    z = torch.nn.functional.avg_pool2d(x.flatten(0, 1), 2, 2)
    z = z.reshape(T, B, C, H // 2, W // 2)
    v0 = torch.rand(B, C, H // 2, W // 2, generator=g) * 0.5
    s_ref, v_ref, _ = oracle.lif_multistep(z, v0, **p)
    s, v = runtime.avgpool2x2_lif(x.to(cuda), v0.to(cuda), **p)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(v.cpu().numpy(), v_ref)
    s8, v8 = runtime.avgpool2x2_lif(x.to(cuda), v0.to(cuda), spike_dtype=torch.uint8, **p)
    assert torch.equal(s8.float(), s) and torch.equal(v8, v)


# ---------------------------------------------------------------------------
# pack + prescan + route: bit-exact
# ---------------------------------------------------------------------------

PRESCAN_SHAPES = [
    # N, C, H, W, k, s, p
    (8, 64, 32, 32, 3, 1, 1),
    (4, 256, 14, 14, 3, 1, 1),
    (2, 64, 56, 56, 3, 1, 1),
    (2, 40, 9, 11, 3, 1, 1),
    (2, 128, 28, 28, 3, 2, 1),
    (3, 64, 14, 14, 1, 2, 0),
    (2, 1024, 8, 8, 1, 1, 0),
]


@pytest.mark.parametrize("shape", PRESCAN_SHAPES)
@pytest.mark.parametrize("rate", [0.0, 0.001, 0.05, 0.5])
def test_pack_prescan_bit_exact(cuda, shape, rate):
    from catfuse_amd import runtime
    N, C, H, W, k, s, p = shape
    x = (torch.rand(N, C, H, W, generator=_gen(int(rate * 1000) + C)) < rate).float()
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    bh, bw = oracle.select_tile_sizes(Ho, Wo)
    gs = oracle.choose_group_size(C)
    G = -(-C // gs)
    xd = x.to(cuda)
    nnz = runtime.count_block(cuda)
    st = torch.zeros(1, dtype=torch.int32, device=cuda)
    xp, act = runtime.pack_input(xd, group_size=gs, nnz=nnz, status=st)
    tc, ag = runtime.prescan_tiles(act, H, W, Ho, Wo, k, s, p, bh, bw, G)
    tc_ref, ag_ref = oracle.prescan2d(x, Ho, Wo, k, s, p, bh, bw, gs)
    np.testing.assert_array_equal(ag.cpu().numpy(), ag_ref)
    np.testing.assert_array_equal(tc.cpu().numpy(), tc_ref)
    assert int(nnz[1].item()) == int(np.count_nonzero(x.numpy()))
    assert int(nnz[0].item()) == 0  # the pass left its accumulator cleared
    assert int(st.item()) == 0
    cp = runtime.pad32(C)
    ref_xp = torch.zeros(N, H, W, cp, dtype=torch.float16)
    ref_xp[..., :C] = x.permute(0, 2, 3, 1).half()
    assert torch.equal(xp.cpu(), ref_xp)
    route = runtime.route_from_nnz(nnz, x.numel(), 0.7)
    assert int(route.item()) == oracle.route(x)


def test_pack_flags_inexact_inputs(cuda):
    from catfuse_amd import runtime
    st = torch.zeros(1, dtype=torch.int32, device=cuda)
    x = torch.full((1, 32, 4, 4), 0.5, device=cuda)
    runtime.pack_input(x, status=st)
    assert int(st.item()) == 0
    x[0, 3, 1, 1] = 0.1  # not representable in fp16
    runtime.pack_input(x, status=st)
    assert int(st.item()) == runtime.STATUS_INEXACT_FP16


def test_fast_spike_prescan_api(cuda):
    from catfuse_amd.sparseflow.prescan import fast_spike_prescan_2d_v2
    x = (torch.rand(4, 256, 14, 14, generator=_gen(3)) < 0.02).float()
    tc, ag = fast_spike_prescan_2d_v2(x.to(cuda), 14, 14, kernel_size=3, stride=1, padding=1,
                                      block_h=8, block_w=8, group_size_c=32)
    tc_ref, ag_ref = oracle.prescan2d(x, 14, 14, 3, 1, 1, 8, 8, 32)
    np.testing.assert_array_equal(tc.cpu().numpy(), tc_ref)
    np.testing.assert_array_equal(ag.cpu().numpy(), ag_ref)


# ---------------------------------------------------------------------------
# fused conv -> BN -> LIF
# ---------------------------------------------------------------------------

def _bn(C, g):
    bn = torch.nn.BatchNorm2d(C).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(C, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(C, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(C, generator=g) * 0.4 + 0.8)
        bn.bias.copy_(torch.randn(C, generator=g) * 0.1)
    return bn


def _layer(Cin, Cout, k, s, p, seed, bias=False, lif=None):
    from catfuse_amd import snn
    g = _gen(seed)
    conv = torch.nn.Conv2d(Cin, Cout, k, s, p, bias=bias)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) *
                          (2.0 / (Cin * k * k)) ** 0.5)
        if bias:
            conv.bias.copy_(torch.randn(Cout, generator=g) * 0.1)
    bn = _bn(Cout, g)
    return conv, bn, (lif or snn.LIFNode(tau=2.0, v_threshold=1.0, v_reset=0.0))


def _runner(conv, bn, lif, dev):
    from catfuse_amd import runtime
    sc, sh = oracle.bn_fold(bn.weight, bn.bias, bn.running_mean, bn.running_var, bn.eps)
    return runtime.ConvLIFRunner(conv.weight.detach().to(dev), sc.to(dev), sh.to(dev),
                                 None if conv.bias is None else conv.bias.detach().to(dev),
                                 conv.stride[0], conv.padding[0], lif.tau, lif.v_threshold,
                                 lif.v_reset, lif.decay_input)


CONV_CASES = [
    # name, T, B, Cin, Cout, H, W, k, s, p, rate
    ("C0", 4, 8, 64, 64, 32, 32, 3, 1, 1, 0.15),
    ("C1", 4, 4, 256, 256, 14, 14, 3, 1, 1, 0.05),
    ("l4", 4, 4, 512, 512, 7, 7, 3, 1, 1, 0.2),
    ("s2", 2, 2, 64, 128, 28, 28, 3, 2, 1, 0.3),
    ("ds", 2, 2, 128, 256, 28, 28, 1, 2, 0, 0.3),
    ("odd", 3, 2, 40, 96, 9, 11, 3, 1, 1, 0.4),
    ("t1", 1, 2, 64, 64, 16, 16, 3, 1, 1, 0.5),
    ("t6", 6, 2, 64, 128, 12, 12, 3, 1, 1, 0.3),
    ("t9s2", 9, 1, 32, 64, 15, 15, 3, 2, 1, 0.3),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv_bn_lif_mfma_parity(cuda, case):
    name, T, B, Cin, Cout, H, W, k, s, p, rate = case
    conv, bn, lif = _layer(Cin, Cout, k, s, p, seed=hash(name) % 997)
    x = (torch.rand(T, B, Cin, H, W, generator=_gen(1)) < rate).float()
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif)
    r = _runner(conv, bn, lif, cuda)
    spk, v = r.run_mfma(x.to(cuda))
    lif_parity(spk.cpu().numpy(), v.cpu().numpy(), s_ref, v_ref, h_ref, what=name)
    # z itself against the oracle's fp64 conv + fp32 BN
    z, _ = r.run_mfma(x.to(cuda), epilogue=1)
    zr = oracle.batch_norm(oracle.conv2d(x.flatten(0, 1), conv.weight, None, s, p), bn)
    np.testing.assert_allclose(z.cpu().numpy().reshape(zr.shape), zr.numpy(), rtol=2e-5,
                               atol=2e-5)


POOL_EPI_CASES = [
    # name, T, B, Cin, Cout, H, W, padding, LIF variant, rate, v_in, SparseFlow
    ("vgg", 4, 2, 64, 128, 16, 16, 1, 0, 0.2, False, False),
    ("odd", 3, 2, 40, 96, 15, 13, 1, 0, 0.4, True, False),
    ("t9", 9, 1, 32, 64, 12, 12, 1, 2, 0.3, True, False),
    ("t6_generic", 6, 2, 64, 64, 10, 18, 1, 3, 0.3, False, False),
    ("pad0", 2, 3, 64, 32, 6, 7, 0, 5, 0.5, True, False),
    ("sparse", 4, 2, 64, 64, 16, 16, 1, 1, 0.05, False, True),
]


@pytest.mark.parametrize("case", POOL_EPI_CASES, ids=[c[0] for c in POOL_EPI_CASES])
def test_conv_bn_avgpool_lif_epilogue_bitwise(cuda, case):
    """The pooled epilogue (BN -> AvgPool2d(2, 2) -> LIF inside the conv)
    equals the conv's z (EPI_Z) followed by cf_avgpool2x2_lif bit for bit:
    same accumulation, the same four-term sum, the same LIF.  Covers odd
    sizes (the floor of AvgPool2d, partial tiles), Cout not a multiple of 64,
    time blocks carried through v_out (T > 4), an initial state, generic LIF
    forms and the SparseFlow route."""
    from catfuse_amd import runtime, snn
    name, T, B, Cin, Cout, H, W, p, variant, rate, with_v, sparse = case
    lif = snn.LIFNode(**LIF_VARIANTS[variant])
    conv, bn, lif = _layer(Cin, Cout, 3, 1, p, seed=len(name) * 31 + T, lif=lif)
    r = _runner(conv, bn, lif, cuda)
    g = _gen(T * 7 + Cout)
    x = (torch.rand(T, B, Cin, H, W, generator=g) < rate).float()
    Ho, Wo = H + 2 * p - 2, W + 2 * p - 2
    v0 = (torch.randn(B, Cout, Ho // 2, Wo // 2, generator=g) * 0.4).to(cuda) if with_v else None
    sp = dict(block_h=8, block_w=8, group_size=16) if sparse else None
    s, v = r.run_mfma(x.to(cuda), v0, epilogue=runtime.EPI_POOL, sparse=sp)
    z, _ = r.run_mfma(x.to(cuda), epilogue=runtime.EPI_Z, sparse=sp)
    s_ref, v_ref = runtime.avgpool2x2_lif(z, v0, **LIF_VARIANTS[variant])
    torch.cuda.synchronize()
    # the output count block: zero iff every pooled spike is zero
    nz = runtime.count_of(s)
    assert nz is not None and (int(nz[1].item()) != 0) == bool(s_ref.any()), name
    assert s.shape == (T, B, Cout, Ho // 2, Wo // 2) and v.shape == (B, Cout, Ho // 2, Wo // 2)
    assert torch.equal(s.cpu(), s_ref.cpu()), name
    assert torch.equal(v.cpu(), v_ref.cpu()), name
    # the pooled spikes feed the next fused conv through their fp16 copy
    conv2, bn2, lif2 = _layer(Cout, 32, 3, 1, 1, seed=5)
    r2 = _runner(conv2, bn2, lif2, cuda)
    s2, _ = r2.run_mfma(s)
    s2_ref, _ = r2.run_mfma(s_ref.clone())
    assert torch.equal(s2.cpu(), s2_ref.cpu()), name


def test_pooled_epilogue_all_zero_input(cuda):
    """An all-zero input (StaticZero route, no K loop): z is the BN bias at
    every pixel, the pooled LIF as the two-kernel path computes it."""
    from catfuse_amd import runtime
    conv, bn, lif = _layer(64, 64, 3, 1, 1, seed=77)
    r = _runner(conv, bn, lif, cuda)
    x = torch.zeros(4, 2, 64, 8, 8, device=cuda)
    s, v = r.run_mfma(x, epilogue=runtime.EPI_POOL)
    z, _ = r.run_mfma(x, epilogue=runtime.EPI_Z)
    s_ref, v_ref = runtime.avgpool2x2_lif(z, None)
    assert torch.equal(s.cpu(), s_ref.cpu()) and torch.equal(v.cpu(), v_ref.cpu())


@pytest.mark.parametrize("bias", ["quiet", "fires"])
def test_pooled_static_zero_elision(cuda, bias):
    """The pooled epilogue on an all-zero input (a fused layer's silent
    output): with a silent pooled bias response (cf_bias_response, pool = 1)
    the copy is left unwritten (descriptor: all zero) and the state kept
    per channel; with a channel that fires on its bias the launch writes.
    Outputs, states, the count-block verdict and a next conv reading the
    output through its descriptor equal the always-writing path's."""
    from catfuse_amd import runtime, snn
    T, B, C, H = 4, 2, 64, 16
    lif = snn.LIFNode(tau=2.0, v_threshold=0.5, v_reset=0.0)

    def run(elide):
        runtime.COPY_ELISION = elide
        try:
            conv0, bn0, _ = _layer(C, C, 3, 1, 1, seed=51)
            conv1, bn1, _ = _layer(C, C, 3, 1, 1, seed=52)
            conv2, bn2, _ = _layer(C, C, 3, 1, 1, seed=53)
            with torch.no_grad():
                bn0.bias.fill_(-8.0)          # silences every output
                bn1.bias.fill_(-0.2)
                if bias == "fires":
                    bn1.bias[7] = 4.0         # channel 7 fires on its bias alone
            r0, r1, r2 = (_runner(c, b, lif, cuda) for c, b in ((conv0, bn0), (conv1, bn1),
                                                                  (conv2, bn2)))
            x = (torch.rand(T, B, C, H, H, generator=_gen(54)) < 0.3).float().to(cuda)
            z, _ = r0.run_mfma(x)                              # all zero, counted
            s, v = r1.run_mfma(z, epilogue=runtime.EPI_POOL)   # StaticZero, pooled
            d = runtime.desc_of(s)
            d = None if d is None else d.clone()
            nz = int(runtime.count_of(s)[1].item())
            s2, v2 = r2.run_mfma(s)                            # reads s through d
            res = (s.clone(), v.clone(), s2.clone(), v2.clone(), nz, d)
            torch.cuda.synchronize()
            return res
        finally:
            runtime.COPY_ELISION = True

    se, ve, s2e, v2e, nze, de = run(True)
    sw, vw, s2w, v2w, nzw, dw = run(False)
    assert dw is None
    for a, b, n in ((se, sw, "s"), (ve, vw, "v"), (s2e, s2w, "s2"), (v2e, v2w, "v2")):
        assert torch.equal(a, b), n
    assert (nze != 0) == (nzw != 0) == bool(sw.any())
    if bias == "quiet":
        assert not bool(sw.any())
        assert de is not None and int(de[0].item() & 0xffffffff) == 1    # all zero
        assert int(de[0].item() >> 32) == 1                               # per-channel state
    else:
        assert bool(sw.any()) and de is None    # written; no descriptor attached


OUTPUT_COUNT_CASES = [
    # name, Cin, Cmid, Cout, k1, k2, s2, p2, H, producer SparseFlow tile width
    ("halo", 64, 64, 64, 3, 3, 1, 1, 16, 0),
    ("halo_s2", 32, 64, 128, 3, 3, 2, 1, 16, 0),
    ("ds", 32, 64, 128, 3, 1, 2, 0, 16, 0),
    ("flat", 32, 64, 64, 5, 5, 1, 2, 12, 0),
    ("tile8x16", 32, 64, 64, 3, 3, 1, 1, 56, 16),
    ("c96", 32, 96, 96, 3, 3, 1, 1, 16, 0),
]


@pytest.mark.parametrize("case", OUTPUT_COUNT_CASES, ids=[c[0] for c in OUTPUT_COUNT_CASES])
def test_output_count_routes_next_layer(cuda, case):
    """A fused conv publishes a count block for its output (zero iff every
    output value is zero); the next fused conv reads it from its input and
    takes the StaticZero route on an all-zero input, bit-identical to the
    dense route.  A later call of the producer invalidates the block for the
    earlier output."""
    from catfuse_amd import runtime
    name, Cin, Cmid, Cout, k1, k2, s2, p2, H, tw1 = case
    T, B = 4, 2
    conv1, bn1, lif1 = _layer(Cin, Cmid, k1, 1, k1 // 2, seed=61)
    conv2, bn2, lif2 = _layer(Cmid, Cout, k2, s2, p2, seed=62)
    r1 = _runner(conv1, bn1, lif1, cuda)
    r2 = _runner(conv2, bn2, lif2, cuda)
    sp1 = dict(block_h=8, block_w=tw1, group_size=16) if tw1 else None
    g = _gen(63)
    seen_zero = seen_nonzero = False
    for rate in (0.0, 0.4, 0.0, 0.02):
        x = (torch.rand(T, B, Cin, H, H, generator=g) < rate).float().to(cuda)
        y1, _ = r1.run_mfma(x, sparse=sp1)
        blk = runtime.count_of(y1)
        assert blk is not None
        n1 = int(blk[1].item())
        assert int(blk[0].item()) == 0 and not bool(blk[16::16].any())  # accumulators cleared
        dense_y1 = y1.clone()  # the fp32 values, as a plain tensor
        all_zero = int(torch.count_nonzero(dense_y1)) == 0
        assert (n1 == 0) == all_zero, f"{name} rate {rate}: count {n1}"
        seen_zero |= all_zero
        seen_nonzero |= not all_zero
        y2, v2 = r2.run_mfma(y1)
        assert r2.last_nnz is blk
        y2d, v2d = r2.run_mfma(y1, static_zero=False)
        assert r2.last_nnz is None
        assert torch.equal(y2, y2d) and torch.equal(v2, v2d), f"{name} rate {rate}"
        y2p, v2p = r2.run_mfma(dense_y1)  # plain fp32 input: counted by the pack pass
        assert torch.equal(y2p, y2d) and torch.equal(v2p, v2d)
    assert seen_zero and seen_nonzero
    ya, _ = r1.run_mfma(x, sparse=sp1)
    yb, _ = r1.run_mfma(x, sparse=sp1)
    assert runtime.count_of(ya) is None and runtime.count_of(yb) is not None


STATICZERO_CASES = [
    # name, Cin, Cout, k, s, p, H, T, SparseFlow tile width (0: dense tiles)
    ("s1", 64, 64, 3, 1, 1, 12, 4, 0),
    ("s1_T6", 64, 64, 3, 1, 1, 12, 6, 0),
    ("s2", 64, 128, 3, 2, 1, 16, 4, 0),
    # stride-2 3x3 tiles hold one halo buffer: the lean epilogue's T spike
    # rows + final potentials fit it up to T = 582, longer runs take the
    # per-element epilogue
    ("s2_T580", 64, 64, 3, 2, 1, 16, 580, 0),
    ("s2_T600", 64, 64, 3, 2, 1, 16, 600, 0),
    ("ds", 64, 128, 1, 2, 0, 16, 4, 0),
    ("tile8x16", 32, 64, 3, 1, 1, 56, 4, 16),
    ("c96", 64, 96, 3, 1, 1, 12, 4, 0),
]


@pytest.mark.parametrize("case", STATICZERO_CASES, ids=[c[0] for c in STATICZERO_CASES])
def test_staticzero_epilogues_bitwise(cuda, case):
    """An all-zero input takes StaticZero; from the initial state (no v_in)
    the lean kernel runs the LIF once per channel and writes the tile from
    per-step spike rows.  It equals the per-element StaticZero epilogue (v_in
    given) and the dense route bit for bit, with and without a SEW identity
    (read from its fp16 NHWC copy), including the final membrane potential."""
    from catfuse_amd import runtime
    name, Cin, Cout, k, s, p, H, T, tw = case
    B = 2
    conv, bn, lif = _layer(Cin, Cout, k, s, p, seed=71)
    with torch.no_grad():
        bn.bias[::3] += 1.5      # channels whose constant drive spikes
        bn.bias[1::5] -= 0.7
    r = _runner(conv, bn, lif, cuda)
    Ho = (H + 2 * p - k) // s + 1
    x = torch.zeros(T, B, Cin, H, H, device=cuda)
    g = _gen(72)
    idv = ((torch.rand(T, B, Cout, Ho, Ho, generator=g) < 0.3).float()
           * torch.randint(1, 3, (T, B, Cout, Ho, Ho), generator=g).float())
    id_nhwc = torch.zeros(T * B, Ho, Ho, runtime.pad32(Cout), dtype=torch.float16)
    id_nhwc[..., :Cout] = idv.reshape(T * B, Cout, Ho, Ho).permute(0, 2, 3, 1).half()
    identity = runtime.lazy_output((T, B, Cout, Ho, Ho), id_nhwc.to(cuda), cuda)
    sp = dict(block_h=8, block_w=tw, group_size=16) if tw else None
    v0 = torch.zeros(B, Cout, Ho, Ho, device=cuda)  # the initial state, given explicitly
    for ident in (None, identity):
        runs = [r.run_mfma(x, sparse=sp, identity=ident),             # uniform StaticZero
                r.run_mfma(x, v0, sparse=sp, identity=ident),         # per-element StaticZero
                r.run_mfma(x, identity=ident, static_zero=False)]     # dense route
        outs = [(y.clone(), v.clone()) for y, v in runs]
        for y, v in outs[1:]:
            assert torch.equal(y, outs[0][0]), f"{name}: spikes"
            assert torch.equal(v, outs[0][1]), f"{name}: membrane"
        y0 = outs[0][0].cpu()
        assert bool((y0 - (0 if ident is None else idv)).abs().max() <= 1.0)
        assert bool(y0.any())    # the biased channels spike
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x.cpu(), conv, bn, lif)
    lif_parity(outs[0][0].cpu().numpy() - idv.numpy(), outs[0][1].cpu().numpy(), s_ref, v_ref,
               h_ref, what=name)


@pytest.mark.parametrize("rate", [0.0, 0.01, 0.05, 0.2, 0.5])
@pytest.mark.parametrize("pattern", ["iid", "block"])
def test_sparse_route_bitwise_equals_dense(cuda, rate, pattern):
    T, B, C, H, W = 4, 4, 256, 14, 14
    conv, bn, lif = _layer(C, C, 3, 1, 1, seed=5)
    g = _gen(int(rate * 100) + (7 if pattern == "block" else 0))
    x = (torch.rand(T, B, C, H, W, generator=g) < rate).float()
    if pattern == "block":
        keep = (torch.rand(T, B, C, 2, 2, generator=g) >= 0.7).float()
        keep = keep.repeat_interleave(8, 3).repeat_interleave(8, 4)[..., :H, :W]
        x = x * keep
    r = _runner(conv, bn, lif, cuda)
    xd = x.to(cuda)
    v0 = (torch.rand(B, C, H, W, generator=g) * 0.5).to(cuda)
    s_dense, v_dense = r.run_mfma(xd, v0, static_zero=False)
    s_sparse, v_sparse = r.run_mfma(xd, v0, sparse=dict(block_h=8, block_w=8, group_size=32))
    s_sz, v_sz = r.run_mfma(xd, v0, static_zero=True)
    for s2, v2 in ((s_sparse, v_sparse), (s_sz, v_sz)):
        assert torch.equal(s2, s_dense)
        assert torch.equal(v2, v_dense)
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif, v_in=v0.cpu())
    lif_parity(s_dense.cpu().numpy(), v_dense.cpu().numpy(), s_ref, v_ref, h_ref,
               what=f"C1 {pattern} {rate}")


@pytest.mark.parametrize("rate", [0.0, 0.02, 0.3])
def test_sparse_8x16_tiles_bitwise_equals_dense(cuda, rate):
    T, B, C, H, W = 4, 2, 64, 56, 56      # 3136 px -> 8x16 prescan tiles
    conv, bn, lif = _layer(C, 64, 3, 1, 1, seed=6)
    x = (torch.rand(T, B, C, H, W, generator=_gen(int(rate * 100) + 1)) < rate).float()
    r = _runner(conv, bn, lif, cuda)
    xd = x.to(cuda)
    s_dense, v_dense = r.run_mfma(xd, static_zero=False)
    s_sparse, v_sparse = r.run_mfma(xd, sparse=dict(block_h=8, block_w=16, group_size=16))
    assert torch.equal(s_sparse, s_dense) and torch.equal(v_sparse, v_dense)
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif)
    lif_parity(s_dense.cpu().numpy(), v_dense.cpu().numpy(), s_ref, v_ref, h_ref, what="56x56")


@pytest.mark.parametrize("stride,T", [(1, 7), (2, 5)])
def test_sparse_route_multiblock_bitwise(cuda, stride, T):
    # several time blocks per tile (4 steps, 2 for stride 2): the state
    # passes between blocks through v_out, the staging of the next block's
    # first chunk overlaps the current block's taps
    B, C, H, W = 2, 96, 16, 16
    conv, bn, lif = _layer(C, 64, 3, stride, 1, seed=11 + stride)
    g = _gen(31 + T)
    x = (torch.rand(T, B, C, H, W, generator=g) < 0.05).float()
    x[:, :, 32:64] = 0.0                       # a chunk inactive everywhere
    x[1] = 0.0                                 # a step with no input at all
    r = _runner(conv, bn, lif, cuda)
    xd = x.to(cuda)
    Ho = (H + 2 - 3) // stride + 1
    v0 = (torch.rand(B, 64, Ho, Ho, generator=g) * 0.5).to(cuda)
    s_dense, v_dense = r.run_mfma(xd, v0, static_zero=False)
    s_sparse, v_sparse = r.run_mfma(xd, v0, sparse=dict(block_h=8, block_w=8, group_size=32))
    assert torch.equal(s_sparse, s_dense) and torch.equal(v_sparse, v_dense)
    s_nov, v_nov = r.run_mfma(xd, v0, want_v_out=False)
    assert v_nov is None and torch.equal(s_nov, s_dense)
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif, v_in=v0.cpu())
    lif_parity(s_dense.cpu().numpy(), v_dense.cpu().numpy(), s_ref, v_ref, h_ref,
               what=f"multiblock s{stride} T{T}")


@pytest.mark.parametrize("ntiles,T,frac", [(1, 1, 1.0), (7, 4, 0.3), (1024, 4, 0.05),
                                             (1025, 2, 0.5), (3000, 4, 0.0), (3000, 3, 1.0)])
def test_compact_tiles_order(cuda, ntiles, T, frac):
    """cf_compact_tiles: order[0] = tiles active at some step, then the
    active tiles ascending, then the inactive ones ascending (numpy)."""
    from catfuse_amd import runtime
    g = _gen(ntiles + T)
    act = torch.rand(T, ntiles, generator=g) < frac
    bits = torch.randint(1, 1 << 20, (T, ntiles), generator=g, dtype=torch.int32)
    ag = torch.where(act, bits, torch.zeros_like(bits))
    order = runtime.compact_tiles(ag.reshape(-1).to(cuda), T, ntiles).cpu().numpy()
    any_act = (ag.numpy() != 0).any(axis=0)
    expect = np.concatenate([np.flatnonzero(any_act), np.flatnonzero(~any_act)])
    assert order[0] == int(any_act.sum())
    assert np.array_equal(order[1:], expect)


@pytest.mark.parametrize("frac,groups", [(0.02, 8), (0.3, 16), (0.9, 32)])
def test_compact_tiles_dispatch_score(cuda, frac, groups):
    """The dispatch score of cf_compact_tiles: R = 1 - group bits set at some
    step / (ntiles * groups) (numpy), S = R * macs_per_tile; order[0] stays the
    active-tile count when R >= 0.99 or (R >= r_min and S > tau), else -1;
    the permutation is written either way."""
    from catfuse_amd import runtime
    T, ntiles = 4, 700
    g = _gen(groups)
    bits = (torch.rand(T, ntiles, groups, generator=g) < frac).int()
    ag = (bits << torch.arange(groups, dtype=torch.int32)).sum(-1).int()
    R = 1.0 - float(bits.any(0).sum()) / (ntiles * groups)
    n_act = int((ag != 0).any(0).sum())
    macs = 1.0e6
    for tau, r_min in ((-1.0, 0.0), (0.0, 0.0), (R * macs * 0.99, 0.0), (R * macs * 1.01, 0.0),
                       (0.0, min(R + 0.01, 1.0)), (0.0, max(R - 0.01, 0.0))):
        order = runtime.compact_tiles(ag.reshape(-1).to(cuda), T, ntiles, groups,
                                      macs_per_tile=macs, tau=tau, r_min=r_min).cpu()
        keep = tau < 0 or R >= 0.99 or (R >= r_min and R * macs > tau)
        assert int(order[0]) == (n_act if keep else -1), (tau, r_min, R)
        assert sorted(order[1:].tolist()) == list(range(ntiles))


def test_sparse_route_dispatch_score_gate_bitwise(cuda):
    """A SparseFlow launch the dispatch score rejects (tau above S) takes the
    dense route inside the conv; one it accepts runs SparseFlow: both equal
    the dense evaluation bit for bit."""
    T, B, C, H = 4, 3, 64, 20
    conv, bn, lif = _layer(C, 64, 3, 1, 1, seed=91)
    x = _half_silent_input(T, B, C, H, H, seed=92)
    r = _runner(conv, bn, lif, cuda)
    xd = x.to(cuda)
    s_dense, v_dense = r.run_mfma(xd, static_zero=False)
    geo = dict(block_h=8, block_w=8, group_size=16)
    for egd in ((1e30, 0.15), (0.0, 0.0)):
        s2, v2 = r.run_mfma(xd, sparse=dict(geo, egd=egd), sparse_threshold=-1.0)
        assert torch.equal(s2, s_dense) and torch.equal(v2, v_dense)
        if egd[0] > 1e20:
            assert int(r.last_order[0]) == -1             # rejected: dense route
    assert int(r.last_order[0]) > 0                       # accepted: active tiles


def _half_silent_input(T, B, C, H, W, seed, rate=0.08):
    """Spikes where whole 16-channel groups, half of some 32-channel chunks,
    are silent (only the group's other half active), activity concentrated
    in a corner of some images and whole (t, b) images silent."""
    g = _gen(seed)
    x = (torch.rand(T, B, C, H, W, generator=g) < rate).float()
    for c0 in range(0, C, 64):
        x[:, :, c0 + 16:c0 + 32] = 0.0          # second half of every other chunk
    x[:, 0, :, H // 2:, :] = 0.0                 # image 0: top half only
    x[:, 0, :, :, W // 2:] = 0.0
    x[1, -1] = 0.0                               # a silent (t, b) image
    return x


@pytest.mark.parametrize("k,stride,T,tile,C", [(3, 1, 4, (8, 8), 128), (3, 2, 5, (8, 8), 96),
                                               (1, 1, 4, (8, 8), 64), (3, 1, 7, (8, 16), 64),
                                               (3, 1, 4, (8, 8), 256)])
def test_sparse_compaction_and_half_skip_bitwise(cuda, k, stride, T, tile, C):
    """The SparseFlow route with the compacted tile order and (16-channel
    groups) the skipped silent chunk halves equals the route without the
    order and the dense route bit for bit, and the oracle."""
    from catfuse_amd.sparseflow.sparse_helpers import choose_group_size
    B, H = 3, 28 if tile[1] == 16 else 20
    p = 1 if k == 3 else 0
    conv, bn, lif = _layer(C, 64, k, stride, p, seed=70 + C + k, lif=None)
    x = _half_silent_input(T, B, C, H, H, seed=C + T)
    r = _runner(conv, bn, lif, cuda)
    xd = x.to(cuda)
    Ho = (H + 2 * p - k) // stride + 1
    v0 = (torch.rand(B, 64, Ho, Ho, generator=_gen(5)) * 0.5).to(cuda)
    gs = choose_group_size(C)
    geo = dict(block_h=tile[0], block_w=tile[1], group_size=gs)
    s_dense, v_dense = r.run_mfma(xd, v0, static_zero=False)
    s_ord, v_ord = r.run_mfma(xd, v0, sparse=dict(geo, compact="always"))
    s_lin, v_lin = r.run_mfma(xd, v0, sparse=dict(geo, compact=False))
    for s2, v2 in ((s_ord, v_ord), (s_lin, v_lin)):
        assert torch.equal(s2, s_dense) and torch.equal(v2, v_dense)
    from catfuse_amd import runtime
    assert runtime.route_from_nnz(r.last_nnz, r.last_numel, 0.7).item() == 1   # SPARSE
    tc, ag = r.last_tiles
    GH, GW = -(-Ho // tile[0]), -(-Ho // tile[1])
    active = (ag.view(T, B * GH * GW) != 0).any(0)
    assert 0 < int(active.sum()) < B * GH * GW            # some tiles run the epilogue only
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif, v_in=v0.cpu())
    lif_parity(s_dense.cpu().numpy(), v_dense.cpu().numpy(), s_ref, v_ref, h_ref,
               what=f"compact k{k} s{stride} T{T} C{C}")


@pytest.mark.parametrize("T,variant,zero", [(4, 0, False), (2, 0, False), (5, 5, False),
                                             (4, 2, False), (4, 0, True)])
def test_conv_halo_pair_bitwise(cuda, T, variant, zero):
    """cf_conv_halo_pair (a stride-2 3x3 conv and a stride-2 1x1 conv of the
    same input in one launch) equals the two convs' own launches bit for
    bit: spikes, membranes, published counts; with a carried membrane, T
    below, at and above the time blocks, every LIF specialisation and the
    StaticZero route."""
    from catfuse_amd import runtime, snn
    p = LIF_VARIANTS[variant]
    B, C, Cout, H = 3, 64, 128, 19
    lif = snn.LIFNode(tau=p["tau"], v_threshold=p["v_threshold"], v_reset=p["v_reset"],
                      decay_input=p["decay_input"])
    conv_a, bn_a, _ = _layer(C, Cout, 3, 2, 1, seed=81)
    conv_b, bn_b, _ = _layer(C, Cout, 1, 2, 0, seed=82)
    ra, rb = _runner(conv_a, bn_a, lif, cuda), _runner(conv_b, bn_b, lif, cuda)
    x = (torch.rand(T, B, C, H, H, generator=_gen(T + variant)) < 0.2).float()
    if zero:
        x.zero_()
    xd = x.to(cuda)
    Ho = (H + 2 - 3) // 2 + 1
    g = _gen(7)
    va = (torch.rand(B, Cout, Ho, Ho, generator=g) * 0.5).to(cuda)
    vb = (torch.rand(B, Cout, Ho, Ho, generator=g) * 0.5).to(cuda)
    for v_a, v_b in ((None, None), (va, vb)):
        sa, wa = ra.run_mfma(xd, v_a)
        sb, wb = rb.run_mfma(xd, v_b)
        ca, cb = int(runtime.count_of(sa)[1]), int(runtime.count_of(sb)[1])
        pa, qa, pb, qb = runtime.run_halo_pair(ra, rb, xd, v_a, v_b)
        torch.cuda.synchronize()
        assert torch.equal(pa, sa) and torch.equal(qa, wa)
        assert torch.equal(pb, sb) and torch.equal(qb, wb)
        assert int(runtime.count_of(pa)[1]) == ca and int(runtime.count_of(pb)[1]) == cb
        if not zero:
            assert bool(sa.any()) and bool(sb.any())
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv_a, bn_a, lif, v_in=va.cpu())
    lif_parity(pa.cpu().numpy(), qa.cpu().numpy(), s_ref, v_ref, h_ref,
               v_th=p["v_threshold"], what="pair 3x3")


def test_sew_block_downsample_pair_matches_separate(cuda):
    """A SEW block with a stride-2 downsample runs conv1 and the downsample
    as one paired launch; its output and every state equal the block run
    with the pair disabled (separate launches), and the downsample
    module's hooks still see its output."""
    import copy
    from catfuse_amd import snn
    from catfuse_amd.patterns import CTFSEWBasicBlock
    import catfuse_amd
    g = _gen(5)
    ds = torch.nn.Sequential(snn.Conv2d(64, 128, 1, 2, bias=False), snn.BatchNorm2d(128))
    blk = snn.BasicBlock(64, 128, stride=2, downsample=ds, cnf="ADD", v_threshold=0.5)
    snn.kaiming_init(blk, g)
    snn.randomize_bn(blk, g)
    snn.functional.set_step_mode(blk, "m")
    fused = CTFSEWBasicBlock.from_sj_block(blk.eval()).to(cuda)
    plain = copy.deepcopy(fused)
    seen = []
    fused.fused_downsample.register_forward_hook(lambda m, a, o: seen.append(o))
    x = (torch.rand(4, 2, 64, 16, 16, generator=g) < 0.3).float().to(cuda)
    y = fused(x)
    calls = []
    orig = plain.fused_first.__class__.forward

    def no_pair(self, x, sew_identity=None):
        self._pair_with = None
        calls.append(1)
        return orig(self, x, sew_identity)
    plain.fused_first.forward = no_pair.__get__(plain.fused_first)
    y2 = plain(x)
    torch.cuda.synchronize()
    catfuse_amd.check_status()
    assert calls and torch.equal(y, y2) and bool(y.any())
    for a, b in ((fused.fused_first, plain.fused_first),
                 (fused.fused_downsample, plain.fused_downsample),
                 (fused.fused_second, plain.fused_second)):
        assert torch.equal(a.state.tensor, b.state.tensor)
    assert len(seen) == 1 and seen[0].shape == (4, 2, 128, 8, 8)


def _elision_chain(cuda, elide):
    """A chain of fused convs over all-zero and live inputs, each layer's
    output and state materialised at the end; with elide the StaticZero
    launches may leave their outputs unwritten (output descriptors)."""
    from catfuse_amd import runtime, snn
    runtime.COPY_ELISION = elide
    try:
        T, B, C, H = 4, 2, 64, 16
        lif = snn.LIFNode(tau=2.0, v_threshold=0.5, v_reset=0.0)

        def layer(seed, k=3, s=1, p=1, bias_fill=None, cout=C):
            conv, bn, _ = _layer(C, cout, k, s, p, seed=seed)
            if bias_fill is not None:
                with torch.no_grad():
                    bn.bias.copy_(bias_fill(bn.bias))
            return _runner(conv, bn, lif, cuda)

        quiet = lambda b: torch.full_like(b, -0.2)   # no channel fires on its bias
        r0 = layer(31)
        r_kill = layer(32, bias_fill=lambda b: torch.full_like(b, -8.0))
        r1, r2, r3 = layer(33, bias_fill=quiet), layer(34, bias_fill=quiet), layer(35)

        def one_hot_bias(b):
            b = b.clone()
            b[5] = 4.0   # channel 5 fires on its bias alone
            return b
        r4 = layer(36, bias_fill=one_hot_bias)
        ra = layer(37, 3, 2, 1, bias_fill=quiet, cout=128)
        rb = layer(38, 1, 2, 0, bias_fill=quiet, cout=128)
        x0 = (torch.rand(T, B, C, H, H, generator=_gen(40)) < 0.3).float().to(cuda)
        s0, v0 = r0.run_mfma(x0)                       # live
        z1, v1 = r_kill.run_mfma(s0)                   # dense route, all-zero output
        z2, v2 = r1.run_mfma(z1)                       # StaticZero, no identity
        a3, v3 = r2.run_mfma(z2, identity=s0)          # StaticZero, equal to its identity
        d4, v4 = r3.run_mfma(a3)                       # dense route over a3
        f5, v5 = r4.run_mfma(z2)                       # StaticZero, one channel fires
        e6, v6 = r2.run_mfma(z2, identity=z2)          # StaticZero, all-zero identity
        pa, qa, pb, qb = runtime.run_halo_pair(ra, rb, z2)
        pc, qc, pd, qd = runtime.run_halo_pair(ra, rb, a3)
        states = {}
        for name, t in (("z2", z2), ("a3", a3), ("f5", f5), ("e6", e6), ("pa", pa), ("pb", pb)):
            d = runtime.desc_of(t)
            states[name] = None if d is None else d.clone()
        pools = []
        for t in (z2, a3, f5):
            xp = runtime.shadow_of(t, (T * B, H, H, C), resolve=False)
            pools.append(runtime.global_avgpool_nhwc(xp, C, desc=runtime.desc_of(t)))
        mp = runtime.maxpool_nhwc(a3, 3, 2, 1)     # through the alias
        mz = runtime.maxpool_nhwc(z2, 3, 2, 1)     # of an all-zero copy: elided
        states["mz"] = None if runtime.desc_of(mz) is None else runtime.desc_of(mz).clone()
        outs = [s0, z1, z2, a3, d4, f5, e6, pa, pb, pc, pd, mp, mz] + pools
        vs = [v0, v1, v2, v3, v4, v5, v6, qa, qb, qc, qd]
        # (a runner called twice republishes its block: the later outputs')
        counts = [int(runtime.count_of(t)[1]) != 0 for t in (z1, z2, d4, f5, e6, pc, pd)]
        res = ([o.clone() for o in outs], [v.clone() for v in vs], counts, states,
               runtime.shadow_of(s0, (T * B, H, H, C)).data_ptr())
        torch.cuda.synchronize()
        return res
    finally:
        runtime.COPY_ELISION = True


def test_static_zero_output_elision_bitwise(cuda):
    """StaticZero launches that provably output nothing new leave their
    copies unwritten (all zero, or an alias of the identity's copy) and
    their state per channel; every output, state and count-block verdict of
    a chain that reads such outputs (convs through the descriptors, the
    paired launch, the global average pool, the max pool and
    materialisation through a fill) equals the always-writing path's."""
    outs_e, vs_e, counts_e, st, s0_ptr = _elision_chain(cuda, True)
    outs_w, vs_w, counts_w, st_w, _ = _elision_chain(cuda, False)
    assert all(v is None for v in st_w.values())
    names = ["s0", "z1", "z2", "a3", "d4", "f5", "e6", "pa", "pb", "pc", "pd", "mp", "mz",
             "pool_z2", "pool_a3", "pool_f5"]
    for n, a, b in zip(names, outs_e, outs_w):
        assert torch.equal(a, b), n
    for i, (a, b) in enumerate(zip(vs_e, vs_w)):
        assert torch.equal(a, b), f"state {i}"
    assert counts_e == counts_w
    # the chain exercised what it names: live data, a zero copy, an alias
    assert bool(outs_w[0].any()) and not bool(outs_w[2].any()) and bool(outs_w[5].any())
    assert bool(outs_w[4].any()) and torch.equal(outs_w[3], outs_w[0])
    # a layer with a channel that fires on its bias always writes its copy:
    # no descriptor is attached to its output
    assert st.pop("f5") is None
    copy = {k: int(v[0].item() & 0xffffffff) for k, v in st.items()}
    vstate = {k: int(v[0].item() >> 32) for k, v in st.items()}
    assert copy == {"z2": 1, "a3": 2, "e6": 1, "pa": 1, "pb": 1, "mz": 1}
    assert vstate == {"z2": 1, "a3": 1, "e6": 1, "pa": 1, "pb": 1, "mz": 0}
    assert int(st["a3"][1].item()) == s0_ptr


def test_static_zero_route_equals_bias_only(cuda):
    T, B, C, H, W = 4, 2, 64, 8, 8
    conv, bn, lif = _layer(C, C, 3, 1, 1, seed=8)
    r = _runner(conv, bn, lif, cuda)
    x = torch.zeros(T, B, C, H, W, device=cuda)
    spk, v = r.run_mfma(x, sparse=dict(block_h=8, block_w=8, group_size=16))
    sc, sh = oracle.bn_fold(bn.weight, bn.bias, bn.running_mean, bn.running_var, bn.eps)
    z = sh.view(1, 1, C, 1, 1).expand(T, B, C, H, W)
    s_ref, v_ref, _ = oracle.lif_multistep(z)
    np.testing.assert_array_equal(spk.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(v.cpu().numpy(), v_ref)


def test_conv_bias_and_sew_identity(cuda):
    T, B, Cin, Cout, H, W = 2, 2, 64, 64, 12, 12
    conv, bn, lif = _layer(Cin, Cout, 3, 1, 1, seed=13, bias=True)
    x = (torch.rand(T, B, Cin, H, W, generator=_gen(2)) < 0.3).float()
    ident = (torch.rand(T, B, Cout, H, W, generator=_gen(3)) < 0.5).float()
    r = _runner(conv, bn, lif, cuda)
    spk, v = r.run_mfma(x.to(cuda))
    out, _ = r.run_mfma(x.to(cuda), identity=ident.to(cuda))
    assert torch.equal(out.cpu(), ident + spk.cpu())
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x, conv, bn, lif)
    lif_parity(spk.cpu().numpy(), v.cpu().numpy(), s_ref, v_ref, h_ref, what="bias")
    # an identity produced by a fused conv carries an fp16 NHWC copy, which
    # the epilogue reads instead of the NCHW tensor: same bits; the copy of
    # a SEW sum (values 0, 1, 2) is exact
    from catfuse_amd import runtime
    r2 = _runner(*_layer(Cin, Cout, 3, 1, 1, seed=14), cuda)
    ident2, _ = r2.run_mfma(x.to(cuda))
    ident3, _ = r2.run_mfma(x.to(cuda), identity=ident2)
    assert runtime.shadow_of(ident3, (T * B, H, W, 64)) is not None
    for idt in (ident2, ident3):
        with_copy, v1 = r.run_mfma(x.to(cuda), identity=idt)
        without, v2 = r.run_mfma(x.to(cuda), identity=idt.clone())
        assert torch.equal(with_copy, without) and torch.equal(v1, v2)
        assert torch.equal(with_copy, idt + spk)


@pytest.mark.parametrize("dedupe", [True, False])
def test_conv_direct_stem_parity(cuda, dedupe):
    T, B, H, W = 4, 2, 64, 64
    conv, bn, lif = _layer(3, 64, 7, 2, 3, seed=21)
    img = torch.randn(B, 3, H, W, generator=_gen(4))
    x = img.unsqueeze(0).expand(T, B, 3, H, W)
    xd = img.to(cuda).unsqueeze(0).expand(T, B, 3, H, W) if dedupe else x.contiguous().to(cuda)
    r = _runner(conv, bn, lif, cuda)
    spk, v = r.run_direct(xd)
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x.contiguous(), conv, bn, lif)
    lif_parity(spk.cpu().numpy(), v.cpu().numpy(), s_ref, v_ref, h_ref, what="stem")


DIRECT_AVG_CASES = [
    # name, T, B, Cin, Cout, H, W, pad, LIF variant, direct encoding, v_in
    ("vgg0", 4, 2, 3, 64, 32, 32, 1, 0, True, False),
    ("odd_steps", 3, 3, 3, 32, 37, 35, 1, 2, False, True),
    ("c1_pad0", 5, 2, 1, 16, 6, 7, 0, 5, True, True),
    ("t9_c4", 9, 1, 4, 48, 20, 18, 2, 3, False, False),
]


@pytest.mark.parametrize("case", DIRECT_AVG_CASES, ids=[c[0] for c in DIRECT_AVG_CASES])
def test_conv_direct_avgpool_lif_bitwise(cuda, case):
    """cf_conv_direct_avgpool_lif (analog Conv 3x3 -> BN -> AvgPool 2x2 ->
    LIF) equals cf_conv_direct's z followed by cf_avgpool2x2_lif bit for
    bit: odd sizes (the pool's floor, partial 16 x 16 tiles), a stride-0
    time axis and a time-varying input, an initial state, generic LIF forms;
    its count block says whether any pooled spike fired."""
    from catfuse_amd import runtime, snn
    name, T, B, Cin, Cout, H, W, p, variant, direct, with_v = case
    lif = snn.LIFNode(**LIF_VARIANTS[variant])
    conv, bn, lif = _layer(Cin, Cout, 3, 1, p, seed=len(name) + 7 * T, bias=True, lif=lif)
    r = _runner(conv, bn, lif, cuda)
    g = _gen(T + 3 * Cout)
    if direct:
        img = torch.randn(B, Cin, H, W, generator=g).to(cuda)
        x = img.unsqueeze(0).expand(T, B, Cin, H, W)
    else:
        x = torch.randn(T, B, Cin, H, W, generator=g).to(cuda)
    Ho, Wo = H + 2 * p - 2, W + 2 * p - 2
    v0 = (torch.randn(B, Cout, Ho // 2, Wo // 2, generator=g) * 0.4).to(cuda) if with_v else None
    nz = runtime.count_block(cuda)
    s, v = r.run_direct_avgpool(x, v0, nz_out=nz, gen_cell=[0])
    z, _ = r.run_direct(x, epilogue=runtime.EPI_Z)
    s_ref, v_ref = runtime.avgpool2x2_lif(z, v0, **LIF_VARIANTS[variant])
    torch.cuda.synchronize()
    assert (int(runtime.count_of(s)[1].item()) != 0) == bool(s_ref.any()), name
    assert s.shape == s_ref.shape and torch.equal(s.cpu(), s_ref.cpu()), name
    assert torch.equal(v.cpu(), v_ref.cpu()), name


STEM_CASES = [
    # name, T, B, H, W, Cout, lif, continue_state
    ("rn_stem", 4, 2, 64, 64, 64, None, False),
    ("odd", 4, 2, 70, 58, 40, None, False),
    ("t20_state", 20, 1, 48, 48, 64, None, True),
    ("t1_c128", 1, 3, 32, 32, 128, None, False),
    ("soft_nodecay", 6, 2, 40, 40, 64, dict(tau=1.7, v_threshold=0.6, v_reset=None,
                                            decay_input=False), False),
    ("vreset", 4, 2, 48, 48, 64, dict(tau=2.0, v_threshold=1.0, v_reset=-0.2,
                                      decay_input=True), True),
    ("tau4_t12", 12, 1, 40, 40, 64, dict(tau=4.0, v_threshold=0.8, v_reset=0.0,
                                         decay_input=True), False),
]


# the patch splitter's first stage: Conv 3x3/1 (name, T, B, H, W, Cout, lif,
# continue_state, padding)
STEM_S1_CASES = [
    ("sps0", 4, 2, 32, 32, 48, None, False, 1),
    ("sps0_odd", 3, 2, 29, 23, 32, None, True, 1),
    ("sps0_t12", 12, 1, 24, 24, 64, dict(tau=4.0, v_threshold=0.8, v_reset=0.0,
                                         decay_input=True), False, 2),
    ("sps0_soft", 5, 2, 20, 18, 16, dict(tau=1.7, v_threshold=0.6, v_reset=None,
                                         decay_input=False), True, 0),
]


@pytest.mark.parametrize("case", STEM_CASES + STEM_S1_CASES,
                         ids=[c[0] for c in STEM_CASES + STEM_S1_CASES])
def test_conv_stem_lif_maxpool_parity(cuda, case):
    """Fused stem (Conv 7x7/2 or 3x3/1 -> BN -> LIF -> MaxPool 3/2/1, direct
    encoding) against the oracle's conv (fp64) -> BN -> LIF, max-pooled on
    the CPU; the fp16 NHWC copy equals the fp32 output; channels past Cout
    are zero; the count block says whether any pooled spike fired."""
    from catfuse_amd import runtime, snn
    name, T, B, H, W, Cout, lifp, cont = case[:8]
    k, s_, p_ = (3, 1, case[8]) if len(case) > 8 else (7, 2, 3)
    lif = snn.LIFNode(**lifp) if lifp else None
    conv, bn, lif = _layer(3, Cout, k, s_, p_, seed=61, lif=lif)
    img = torch.randn(B, 3, H, W, generator=_gen(62))
    r = _runner(conv, bn, lif, cuda)
    x = img.to(cuda).unsqueeze(0).expand(T, B, 3, H, W)
    assert r.stem_supported(x, (3, 2, 1))
    v_in = None
    if cont:  # continue from the state a first call leaves (same v_in for both)
        _, v_in = r.run_stem_pool(x)
    v_in_ref = None if v_in is None else v_in.cpu()
    runtime.clear_status(cuda)
    blk = runtime.count_block(cuda)
    out, v = r.run_stem_pool(x, v_in, nz_out=blk, gen_cell=[0])
    torch.cuda.synchronize()
    assert runtime.read_status(cuda) == 0
    assert runtime.count_of(out) is blk
    assert (int(blk[1].item()) == 0) == (not bool(out.any())), name
    s_ref, v_ref, h_ref = oracle.conv_bn_lif(x.cpu().contiguous(), conv, bn, lif,
                                              v_in=v_in_ref)
    vth = lif.v_threshold
    pooled_parity(out.cpu().numpy(), s_ref, h_ref, v_th=vth, what=name)
    membrane_parity(v.cpu().numpy(), v_ref, h_ref, v_th=vth, what=name)
    Hp, Wp = out.shape[3], out.shape[4]
    cp = runtime.pad32(Cout)
    sh = runtime.shadow_of(out, (T * B, Hp, Wp, cp))
    assert sh is not None and not sh[..., Cout:].any()
    assert torch.equal(sh[..., :Cout].float(), out.reshape(T * B, Cout, Hp, Wp).permute(0, 2, 3, 1))


@pytest.mark.parametrize("v_reset,copy", [(0.0, "f16"), (-0.2, "f16"), (0.0, "u8")])
def test_conv_stem_lean_matches_general(cuda, v_reset, copy):
    """The lean stem instantiation (no initial state passed, T = 4, hard
    reset, a 7-row filter, every channel real, the NHWC copy only) equals the
    general one bit for bit: the same call with the initial state passed
    explicitly (v_in = v_reset everywhere) takes the general kernel's
    stepped LIF; spikes (the copy), final potentials and the count agree."""
    from catfuse_amd import runtime, snn
    lif = snn.LIFNode(tau=2.0, v_threshold=0.7, v_reset=v_reset, decay_input=True)
    conv, bn, lif = _layer(3, 64, 7, 2, 3, seed=64, lif=lif)
    img = torch.randn(3, 3, 61, 77, generator=_gen(65)) * 1.5
    r = _runner(conv, bn, lif, cuda)
    x = img.to(cuda).unsqueeze(0).expand(4, 3, 3, 61, 77)
    prev = runtime.SPIKE_COPY
    runtime.set_spike_copy(copy)
    try:
        blk_a, blk_b = runtime.count_block(cuda), runtime.count_block(cuda)
        out_a, v_a = r.run_stem_pool(x, nz_out=blk_a, gen_cell=[0])
        v0 = torch.full_like(v_a, v_reset)
        out_b, v_b = r.run_stem_pool(x, v0, nz_out=blk_b, gen_cell=[0])
        torch.cuda.synchronize()
        Hp, Wp = out_a.shape[3], out_a.shape[4]
        sh_a = runtime.shadow_of(out_a, (12, Hp, Wp, 64), u8_ok=True)
        sh_b = runtime.shadow_of(out_b, (12, Hp, Wp, 64), u8_ok=True)
        assert sh_a.dtype == sh_b.dtype == (torch.uint8 if copy == "u8" else torch.float16)
        assert bool(sh_a.any())
        assert torch.equal(sh_a, sh_b)
        assert torch.equal(v_a.view(torch.int32), v_b.view(torch.int32))
        assert int(blk_a[1].item()) == int(blk_b[1].item())
    finally:
        runtime.set_spike_copy(prev)


def test_conv_stem_range_flag(cuda):
    """An image value outside fp16's range raises the sticky status bit."""
    from catfuse_amd import runtime
    conv, bn, lif = _layer(3, 64, 7, 2, 3, seed=63)
    r = _runner(conv, bn, lif, cuda)
    img = torch.randn(1, 3, 32, 32)
    img[0, 1, 5, 7] = 1e6
    runtime.clear_status(cuda)
    r.run_stem_pool(img.to(cuda).unsqueeze(0).expand(2, 1, 3, 32, 32))
    assert runtime.read_status(cuda) & runtime.STATUS_FP16_RANGE
    runtime.clear_status(cuda)


@pytest.mark.parametrize("C,gs", [(64, 16), (96, 16), (256, 32), (40, 16)])
def test_scan_nhwc_matches_pack(cuda, C, gs):
    """cf_scan_nhwc on the fp16 NHWC copy gives cf_pack_input's activity bits
    and nonzero count, bit for bit (values include ones, twos and tiny ones)."""
    from catfuse_amd import runtime
    g = _gen(C)
    x = (torch.rand(6, C, 9, 11, generator=g) < 0.2).float()
    x += (torch.rand(x.shape, generator=g) < 0.05).float()
    x[0, 0, 0, 0] = 2.0 ** -21  # below the 1e-6 activity threshold, still nonzero
    xd = x.to(cuda)
    n1 = runtime.count_block(cuda)
    n2 = runtime.count_block(cuda)
    for _ in range(2):  # a second pass republishes the same count
        xp, act = runtime.pack_input(xd, cp=runtime.pad32(C), group_size=gs, nnz=n1)
        act2 = runtime.scan_nhwc(xp, C, group_size=gs, nnz=n2)
        torch.cuda.synchronize()
        assert torch.equal(act, act2)
        assert int(n1[1].item()) == int(n2[1].item()) == int((x != 0).sum())
        assert not bool(n1[0].item()) and not bool(n1[16::16].any())
        assert not bool(n2[0].item()) and not bool(n2[16::16].any())


@pytest.mark.parametrize("NB,H,W,C,cp,gs,thr", [(128, 56, 56, 64, 64, 16, 1e-6),
                                                  (16, 14, 14, 250, 256, 32, 0.5),
                                                  (3, 5, 7, 12, 16, 8, 1e-6),
                                                  (5, 9, 9, 96, 96, 16, -1.0),
                                                  (7, 6, 6, 40, 64, 16, 3.0e-5)])
def test_scan_nhwc_thresholds_and_sizes(cuda, NB, H, W, C, cp, gs, thr):
    """cf_scan_nhwc against torch on fp16 copies holding signed values, -0,
    subnormals and values at the threshold: bit g of a pixel iff some
    channel c < C of group g has |x| > thr; the count is that of nonzero
    halves (channels >= C included, -0 not); sizes from a few pixels to a
    grid-stride pass over 400k pixels."""
    from catfuse_amd import runtime
    g = _gen(NB + C)
    vals = torch.tensor([0.0, -0.0, 1.0, -1.0, 2.0, 2.0 ** -24, -(2.0 ** -20), 0.5, 3.0e-5, 1e-6],
                        dtype=torch.float16)
    idx = torch.randint(0, len(vals), (NB, H, W, cp), generator=g)
    keep = torch.rand(NB, H, W, cp, generator=g) < 0.1
    xp = torch.where(keep, vals[idx], torch.zeros((), dtype=torch.float16))
    blk = runtime.count_block(cuda)
    act = runtime.scan_nhwc(xp.to(cuda), C, group_size=gs, threshold=thr, nnz=blk).cpu()
    mag = xp.float().abs()[..., :C]
    hit = mag > thr
    ng = -(-C // gs)
    pad = ng * gs - C
    hit = torch.nn.functional.pad(hit, (0, pad)).reshape(NB, H, W, ng, gs).any(-1)
    expect = (hit.int() << torch.arange(ng, dtype=torch.int32)).sum(-1).int()
    assert torch.equal(act.view(NB, H, W), expect)
    nz = int(((xp.view(torch.int16) & 0x7fff) != 0).sum())
    assert int(blk[1].item()) == nz


def test_sparseflow_on_nhwc_copy_bitwise(cuda):
    """A SparseFlow layer fed an input that carries its NHWC copy (activity
    from cf_scan_nhwc) equals the same layer fed a plain tensor (cf_pack_input)."""
    from catfuse_amd.sparseflow.sparse_helpers import choose_group_size
    c1, b1, l1 = _layer(64, 64, 3, 1, 1, seed=51)
    c2, b2, l2 = _layer(64, 128, 3, 1, 1, seed=52)
    r1, r2 = _runner(c1, b1, l1, cuda), _runner(c2, b2, l2, cuda)
    x = (torch.rand(4, 2, 64, 16, 16, generator=_gen(53)) < 0.1).float().to(cuda)
    y1, _ = r1.run_mfma(x)
    geom = dict(block_h=8, block_w=8, group_size=choose_group_size(64))
    a, va = r2.run_mfma(y1, sparse=geom, sparse_threshold=0.5)
    tiles_a = [t.clone() for t in r2.last_tiles]
    b_, vb = r2.run_mfma(y1.clone(), sparse=geom, sparse_threshold=0.5)
    assert torch.equal(a, b_) and torch.equal(va, vb)
    for ta, tb in zip(tiles_a, r2.last_tiles):
        assert torch.equal(ta, tb)


def test_lazy_fp32_output_matches_written_fp32(cuda):
    """A fused conv that emits its NHWC copy returns an NHWCSpikes tensor
    whose fp32 values appear on first read and equal the fp32 the kernel
    writes when asked to; torch results on it are plain tensors."""
    from catfuse_amd import runtime
    c1, b1, l1 = _layer(64, 96, 3, 1, 1, seed=71)
    r1 = _runner(c1, b1, l1, cuda)
    x = (torch.rand(4, 2, 64, 12, 10, generator=_gen(72)) < 0.3).float().to(cuda)
    lazy, v1 = r1.run_mfma(x)
    eager, v2 = r1.run_mfma(x, emit_nhwc=False)
    assert isinstance(lazy, runtime.NHWCSpikes) and lazy._cf_pending
    assert runtime.shadow_of(lazy, (8, 12, 10, 96)) is not None
    assert lazy._cf_pending  # metadata queries and the copy lookup do not fill it
    s = lazy * 1.0
    assert not lazy._cf_pending and type(s) is torch.Tensor
    assert torch.equal(lazy, eager) and torch.equal(v1, v2)
    lazy2, _ = r1.run_mfma(x)
    assert torch.equal(lazy2.detach().cpu(), eager.cpu())


def test_nhwc_shadow_handoff_bitwise_and_invalidated(cuda):
    """A fused conv's output carries an fp16 NHWC copy that the next fused
    conv reads instead of re-packing; results are bit-identical, and an
    in-place change of the fp32 output invalidates the copy."""
    from catfuse_amd import runtime
    c1, b1, l1 = _layer(64, 64, 3, 1, 1, seed=41)
    c2, b2, l2 = _layer(64, 96, 1, 2, 0, seed=42)
    r1, r2 = _runner(c1, b1, l1, cuda), _runner(c2, b2, l2, cuda)
    x = (torch.rand(4, 2, 64, 16, 16, generator=_gen(43)) < 0.3).float().to(cuda)
    y1, _ = r1.run_mfma(x)
    assert runtime.shadow_of(y1, (8, 16, 16, 64)) is not None
    ref_xp = torch.zeros(8, 16, 16, 64, dtype=torch.float16, device=cuda)
    ref_xp[..., :64] = y1.reshape(8, 64, 16, 16).permute(0, 2, 3, 1).half()
    assert torch.equal(runtime.shadow_of(y1, (8, 16, 16, 64)), ref_xp)
    y2_shadow, v2a = r2.run_mfma(y1)
    y2_pack, v2b = r2.run_mfma(y1.clone())          # clone: no shadow -> pack pass
    assert torch.equal(y2_shadow, y2_pack) and torch.equal(v2a, v2b)
    y1.mul_(0.0)                                      # in-place change
    assert runtime.shadow_of(y1, (8, 16, 16, 64)) is None
    y2_zero, _ = r2.run_mfma(y1)
    y2_ref, _ = r2.run_mfma(torch.zeros_like(y1))
    assert torch.equal(y2_zero, y2_ref)
    # direct (analog) conv emits a copy with zero-padded channels
    c3, b3, l3 = _layer(3, 40, 3, 1, 1, seed=44)
    r3 = _runner(c3, b3, l3, cuda)
    img = torch.randn(4, 2, 3, 8, 8, generator=_gen(45)).to(cuda)
    y3, _ = r3.run_direct(img, emit_nhwc=True)
    sh = runtime.shadow_of(y3, (8, 8, 8, 64))
    assert sh is not None and not sh[..., 40:].any()
    assert torch.equal(sh[..., :40], y3.reshape(8, 40, 8, 8).permute(0, 2, 3, 1).half())


def test_resolve_copy_and_expand_state_descriptors(cuda):
    """cf_resolve_copy fills a copy its descriptor records as all zero or as
    an alias (and leaves a written one alone); cf_expand_state broadcasts the
    per-channel potentials when the descriptor says so (and leaves v alone
    otherwise)."""
    from catfuse_amd import _hip
    L, st = _hip.lib(), _hip.stream(cuda)
    n = 3 * 1024 + 48                       # halves: a multiple of 8 (16-byte units)
    src = torch.arange(n, dtype=torch.float16, device=cuda) % 7
    for state, expect in ((0, "keep"), (1, "zero"), (2, "alias")):
        buf = torch.full((n,), 5.0, dtype=torch.float16, device=cuda)
        desc = torch.zeros(2, dtype=torch.int64, device=cuda)
        desc[0] = state                     # copy state (low word), vstate 0
        desc[1] = src.data_ptr() if state == 2 else 0
        assert L.cf_resolve_copy(buf.data_ptr(), n * 2, desc.data_ptr(), st) == 0
        torch.cuda.synchronize()
        ref = {"keep": torch.full_like(buf, 5.0), "zero": torch.zeros_like(buf), "alias": src}[expect]
        assert torch.equal(buf, ref), expect
    B, C, HW = 3, 40, 49
    v_chan = torch.randn(C, device=cuda)
    for vstate in (0, 1):
        v = torch.full((B, C, HW), -3.0, device=cuda)
        desc = torch.zeros(2, dtype=torch.int64, device=cuda)
        desc[0] = vstate << 32
        assert L.cf_expand_state(v.data_ptr(), v_chan.data_ptr(), desc.data_ptr(), B, C, HW,
                                 st) == 0
        torch.cuda.synchronize()
        ref = v_chan.view(1, C, 1).expand(B, C, HW) if vstate else torch.full_like(v, -3.0)
        assert torch.equal(v, ref), vstate
