"""Spiking transformer path (Spikformer, config C4) against the CPU oracle.

Fused Linear -> BN1d -> LIF layers and the attention core under the LIF
tolerance of tests/parity.py (bit-exact where the arithmetic is exact: the
attention with scale 0.125 and binary Q, K, V); the concatenated QKV layer
bit for bit against three separate layers; a small Spikformer layer by layer
on the inputs each fused layer actually received, and its logits.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from parity import lif_parity, pooled_parity

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _triple(I, O, seed, v_threshold=1.0):
    from catfuse_amd import snn
    g = _gen(seed)
    lin = torch.nn.Linear(I, O)
    bn = torch.nn.BatchNorm1d(O).eval()
    with torch.no_grad():
        lin.weight.copy_(torch.randn(O, I, generator=g) * (2.0 / I) ** 0.5 * 1.5)
        lin.bias.copy_(torch.randn(O, generator=g) * 0.1)
        bn.running_mean.copy_(torch.randn(O, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(O, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(O, generator=g) * 0.4 + 0.8)
        bn.bias.copy_(torch.randn(O, generator=g) * 0.1)
    return lin, bn, snn.LIFNode(step_mode="m", v_threshold=v_threshold)


LINEAR_CASES = [
    # name, T, B, N, I, O  (N = 196: 14 x 14 token grid, halo kernel; N = 10:
    # flat tiles; N = 0: [T, B, I] input)
    ("grid14", 4, 2, 196, 64, 96),
    ("n10", 3, 2, 10, 96, 64),
    ("vec", 4, 3, 0, 128, 64),
    ("wide", 2, 2, 64, 384, 384),
]


@pytest.mark.parametrize("case", LINEAR_CASES, ids=[c[0] for c in LINEAR_CASES])
def test_fused_linear_bn_lif_parity(cuda, case):
    from catfuse_amd.transformer import FusedLinearBNLIF
    name, T, B, N, I, O = case
    lin, bn, lif = _triple(I, O, seed=hash(name) % 97)
    shape = (T, B, N, I) if N else (T, B, I)
    x = (torch.rand(shape, generator=_gen(1)) < 0.3).float()
    f = FusedLinearBNLIF.from_sj_modules(lin, bn, lif).to(cuda)
    y = f(x.to(cuda))
    xs = x if N else x.unsqueeze(2)
    s_ref, v_ref, h_ref = oracle.linear_bn_lif(xs, lin, bn, lif)
    v = f.membrane().cpu().numpy()   # [B, N, O]
    yo = y.cpu().numpy() if N else y.unsqueeze(2).cpu().numpy()
    lif_parity(yo, v, s_ref, v_ref, h_ref, what=name)
    # residual added in the epilogue (integer-valued, read from a packed copy)
    idv = ((torch.rand(s_ref.shape, generator=_gen(2)) < 0.5).float()
           * torch.randint(1, 3, s_ref.shape, generator=_gen(3)).float())
    f.reset()
    y2 = f(x.to(cuda), identity=(idv if N else idv.squeeze(2)).to(cuda))
    y2o = y2.cpu() if N else y2.unsqueeze(2).cpu()
    lif_parity((y2o - idv).numpy(), None, s_ref, None, h_ref, what=name + "+residual")
    # a second call carries the state like one longer sequence
    f.reset()
    a = f(x[:T // 2].to(cuda))
    b = f(x[T // 2:].to(cuda))
    assert torch.equal(torch.cat([a, b]).cpu(), y.cpu())


def test_concatenated_qkv_bitwise(cuda):
    from catfuse_amd.transformer import FusedLinearBNLIF
    triples = [_triple(128, 128, seed=s) for s in (5, 6, 7)]
    x = (torch.rand(4, 2, 196, 128, generator=_gen(8)) < 0.25).float().to(cuda)
    cat = FusedLinearBNLIF.concatenated(triples).to(cuda)
    y = cat(x)
    for i, t in enumerate(triples):
        f = FusedLinearBNLIF.from_sj_modules(*t).to(cuda)
        assert torch.equal(f(x), y[..., 128 * i:128 * (i + 1)])


@pytest.mark.parametrize("N,heads,T,scale", [(196, 2, 4, 0.125), (64, 3, 6, 0.125),
                                             (256, 1, 2, 0.125), (196, 2, 4, 32 ** -0.5),
                                             (37, 2, 3, 0.125)])
def test_spike_attention_parity(cuda, N, heads, T, scale):
    from catfuse_amd import runtime, snn
    B, C = 2, 32 * heads
    g = _gen(N + heads)
    q, k, v = ((torch.rand(T, B, N, C, generator=g) < r).float() for r in (0.3, 0.2, 0.25))
    lif = snn.LIFNode(step_mode="m", v_threshold=4.0)
    copy = runtime.pack_tokens(torch.cat([q, k, v], -1).to(cuda), 3 * C)
    out, v_out = runtime.spike_attention_lif(copy, T, B, N, heads, (0, C, 2 * C), scale,
                                             v_threshold=4.0)
    s_ref, v_ref, h_ref = oracle.spike_attention_lif(q, k, v, heads, scale, lif)
    if scale == 0.125:
        # integers times a power of two: every value exact on both sides
        np.testing.assert_array_equal(out.cpu().numpy(), s_ref)
        np.testing.assert_array_equal(v_out.cpu().numpy(), v_ref)
    else:
        lif_parity(out.cpu().numpy(), v_out.cpu().numpy(), s_ref, v_ref, h_ref,
                   v_th=4.0, what="attention")
    assert s_ref.any() and not s_ref.all()
    # v_in carried: the second half of the sequence from the first half's state
    out1, v1 = runtime.spike_attention_lif(
        runtime.pack_tokens(torch.cat([q, k, v], -1)[: T // 2].to(cuda), 3 * C), T // 2, B, N,
        heads, (0, C, 2 * C), scale, v_threshold=4.0)
    out2, _ = runtime.spike_attention_lif(
        runtime.pack_tokens(torch.cat([q, k, v], -1)[T // 2:].to(cuda), 3 * C), T - T // 2, B,
        N, heads, (0, C, 2 * C), scale, v_threshold=4.0, v_in=v1)
    assert torch.equal(torch.cat([out1, out2]).cpu(), out.cpu())


def test_spike_attention_zero_route_bitwise(cuda):
    """A Q, K, V copy whose count block publishes zero takes the zero route
    (no operand reads, z = 0); with a carried membrane (so the LIF still
    spikes) it equals the full evaluation of the same zero input bit for
    bit, and a nonzero published count takes the full evaluation."""
    from catfuse_amd import runtime
    T, B, N, heads = 4, 3, 100, 2
    C = heads * 32
    copy = torch.zeros((T * B * N, 3 * C), dtype=torch.float16, device=cuda)
    v_in = (torch.rand(B, N, C, generator=_gen(3)) * 4.0).to(cuda)   # half charges past 1
    ref, v_ref = runtime.spike_attention_lif(copy, T, B, N, heads, (0, C, 2 * C), 0.125,
                                             v_in=v_in)
    for count in (0, 7):
        blk = runtime.count_block(cuda)
        blk[1] = count
        out, v_out = runtime.spike_attention_lif(copy, T, B, N, heads, (0, C, 2 * C), 0.125,
                                                 v_in=v_in, nnz=blk)
        assert torch.equal(out, ref) and torch.equal(v_out, v_ref)
    assert bool(ref.any()) and not bool(ref.all())


def test_spike_attention_zero_route_elision_bitwise(cuda):
    """From the initial state, a zero count drives every neuron with z = 0:
    a LIF that never fires on it leaves the output unwritten (descriptor:
    all zero, count zero) and the state uniform; the next token linear reads
    it through the descriptor; outputs, states and counts equal the
    always-writing path bit for bit."""
    from catfuse_amd import runtime
    T, B, N, heads = 4, 3, 100, 2
    C = heads * 32
    copy = torch.zeros((T * B * N, 3 * C), dtype=torch.float16, device=cuda)
    w = (torch.randn(64, C, 1, 1, generator=_gen(8)) * 0.2).to(cuda)
    proj = runtime.ConvLIFRunner(w, torch.ones(64, device=cuda),
                                 torch.full((64,), -0.2, device=cuda), None, 1, 0, 2.0, 1.0,
                                 0.0, True)

    def run(elide):
        runtime.COPY_ELISION = elide
        try:
            blk = runtime.count_block(cuda)
            nz = runtime.count_block(cuda)
            out, v = runtime.spike_attention_lif(copy, T, B, N, heads, (0, C, 2 * C), 0.125,
                                                 nnz=blk, nz_out=nz, gen_cell=[0])
            d = runtime.desc_of(out)
            st = None if d is None else int(d[0].item())
            y, vy = proj.run_tokens(out)
            return (out.clone(), v.clone(), y.clone(), vy.clone(), int(nz[1].item()), st)
        finally:
            runtime.COPY_ELISION = True

    e, w_ = run(True), run(False)
    for a, b in zip(e[:4], w_[:4]):
        assert torch.equal(a, b)
    assert e[4] == w_[4] == 0
    assert e[5] == (1 | (1 << 32)) and w_[5] is None    # all zero, state uniform
    assert not bool(e[0].any())


def _small_spikformer(seed=41):
    from catfuse_amd import snn
    m = snn.Spikformer(img_size=32, num_classes=10, embed_dim=64, num_heads=2, depth=2, T=4,
                       pools=(2, 3), v_threshold=1.0)
    g = _gen(seed)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    with torch.no_grad():   # keep every layer active: a stronger drive than kaiming's
        for blk in m.blocks:
            for lin in (blk.attn.q, blk.attn.k, blk.attn.v, blk.attn.proj, blk.mlp.fc1,
                        blk.mlp.fc2):
                lin.weight.mul_(3.0)
        sps = m.patch_embed
        for conv in [getattr(sps, f"conv{i}") for i in range(4)] + [sps.rpe_conv]:
            conv.weight.mul_(3.0)
    return m.eval()


def _spikformer_parity(cuda, m, x, live):
    """Every fused layer of the optimized Spikformer against the oracle on
    the input it received: the SPS stages (conv0 with its pool fused, when
    direct-encoded, through the pooled spikes the next stage received), the
    rpe conv, every Linear-BN1d-LIF (Q/K/V concatenated), the attention core
    on the Q, K, V its block produced; the pre-head LIF and head on the
    fused features; with live, every layer's input and output must be
    active.  Returns the number of near-threshold flips."""
    import catfuse_amd
    from catfuse_amd.transformer import FusedLinearBNLIF
    T = x.shape[0]
    fused, stats = catfuse_amd.optimize(m, T=T)
    assert stats["fused_lif_nodes"] == stats["total_lif_nodes"]   # pre_head_lif: FusedLIF
    recs = []
    origs = {}
    for bi, (fb, ob) in enumerate(zip(fused.blocks, m.blocks)):
        a, mm = ob.attn, ob.mlp
        origs[id(fb.attn.qkv)] = [(a.q, a.q_bn, a.q_lif), (a.k, a.k_bn, a.k_lif),
                                  (a.v, a.v_bn, a.v_lif)]
        origs[id(fb.attn.proj)] = [(a.proj, a.proj_bn, a.proj_lif)]
        origs[id(fb.mlp.fc1)] = [(mm.fc1, mm.fc1_bn, mm.fc1_lif)]
        origs[id(fb.mlp.fc2)] = [(mm.fc2, mm.fc2_bn, mm.fc2_lif)]
    handles = []
    for mod in fused.modules():
        if isinstance(mod, FusedLinearBNLIF):
            def hook(md, args, kwargs, out):
                ident = kwargs.get("identity")
                recs.append((id(md), args[0].detach().cpu(),
                             None if ident is None else ident.detach().cpu(), out.detach().cpu()))
            handles.append(mod.register_forward_hook(hook, with_kwargs=True))
    sps_f, sps_o = fused.patch_embed, m.patch_embed
    stage_recs = {}
    for i, st in enumerate(list(sps_f.stages) + [sps_f.rpe]):
        def shook(md, args, kwargs, out, i=i):
            ident = kwargs.get("sew_identity")
            stage_recs[i] = (args[0].detach().cpu(), None if ident is None else
                             ident.detach().cpu(), out.detach().cpu())
        handles.append(st.register_forward_hook(shook, with_kwargs=True))
    feats = []
    handles.append(fused.pre_head_lif.register_forward_hook(
        lambda md, a, o: feats.append(a[0].detach().cpu())))
    with torch.no_grad():
        y = fused(x.to(cuda))
    torch.cuda.synchronize()
    for h in handles:
        h.remove()
    catfuse_amd.check_status()
    flips = 0
    # SPS: stage i's spikes (before its pool); the pooled spikes are the next
    # stage's recorded input, so conv0 + pool fused in one launch is checked
    # through stage 1's input
    stage_in = [stage_recs[i][0] if i in stage_recs else None for i in range(5)]
    stage_in[0] = x
    for i in range(5):
        conv, bn, lif = ((sps_o.rpe_conv, sps_o.rpe_bn, sps_o.rpe_lif) if i == 4 else
                         (getattr(sps_o, f"conv{i}"), getattr(sps_o, f"bn{i}"),
                          getattr(sps_o, f"lif{i}")))
        s_ref, _, h_ref = oracle.conv_bn_lif(stage_in[i].contiguous(), conv, bn, lif)
        pool = None if i == 4 else getattr(sps_o, f"pool{i}", None)
        if i in stage_recs:
            xin, ident, out = stage_recs[i]
            spikes = out - ident if ident is not None else out
            flips += lif_parity(spikes.numpy(), None, s_ref, None, h_ref,
                                v_th=lif.v_threshold, what=f"sps{i}")
            if live:
                assert bool((xin != 0).any()) and bool((spikes != 0).any()), f"sps{i} silent"
            if pool is not None:
                p = F.max_pool2d(out.flatten(0, 1), 3, 2, 1)
                assert torch.equal(p.reshape(stage_in[i + 1].shape), stage_in[i + 1])
            elif i < 4:
                assert torch.equal(out, stage_in[i + 1]), f"sps{i} -> sps{i + 1} link"
        else:
            assert pool is not None, f"stage {i} ran no hooked module and has no pool"
            flips += pooled_parity(stage_in[i + 1].numpy(), s_ref, h_ref,
                                   v_th=lif.v_threshold, what=f"sps{i}+pool")
            if live:
                assert bool((stage_in[i + 1] != 0).any()), f"sps{i} silent"
    n_lin = 4 * len(m.blocks)
    assert len(recs) == n_lin
    # the links between layers: SPS output -> tokens -> each block's
    # residuals and linears -> the next block
    rpe_out = stage_recs[4][2]
    tokens = rpe_out.flatten(-2).transpose(-1, -2)
    rec_of = {mid: (xin, ident, out) for mid, xin, ident, out in recs}
    for fb in fused.blocks:
        q_in = rec_of[id(fb.attn.qkv)][0]
        assert torch.equal(q_in, tokens), "block input differs from the previous output"
        p_in, p_id, p_out = rec_of[id(fb.attn.proj)]
        assert torch.equal(p_id, q_in), "attention residual is not the block input"
        f1_in = rec_of[id(fb.mlp.fc1)][0]
        assert torch.equal(f1_in, p_out), "fc1 input is not the attention output"
        f2_in, f2_id, f2_out = rec_of[id(fb.mlp.fc2)]
        assert torch.equal(f2_id, p_out), "MLP residual is not the attention output"
        tokens = f2_out
    torch.testing.assert_close(feats[0], tokens.mean(dim=2), rtol=1e-6, atol=1e-6)
    by_id = {}
    for mid, xin, ident, out in recs:
        outs = [oracle.linear_bn_lif(xin, *t) for t in origs[mid]]
        s_ref = np.concatenate([o[0] for o in outs], -1)
        h_ref = np.concatenate([o[2] for o in outs], -1)
        spikes = out - ident if ident is not None else out
        flips += lif_parity(spikes.numpy(), None, s_ref, None, h_ref,
                            v_th=origs[mid][0][2].v_threshold, what="linear")
        if live:
            assert bool((xin != 0).any()) and bool((spikes != 0).any()), "a linear is silent"
        by_id[mid] = (xin, out)
    for fb, ob in zip(fused.blocks, m.blocks):
        qkv_in, qkv = by_id[id(fb.attn.qkv)]
        att, _ = by_id[id(fb.attn.proj)]
        C = ob.attn.dim
        s_ref, _, h_ref = oracle.spike_attention_lif(qkv[..., :C], qkv[..., C:2 * C],
                                                     qkv[..., 2 * C:], ob.attn.num_heads,
                                                     ob.attn.scale, ob.attn.attn_lif)
        flips += lif_parity(att.numpy(), None, s_ref, None, h_ref,
                            v_th=ob.attn.attn_lif.v_threshold, what="attention")
        if live:
            assert bool((att != 0).any()), "an attention core is silent"
    # pre-head LIF and head on the fused features
    s_ph, _, _ = oracle.lif_multistep(feats[0], None, **oracle.lif_params_of(m.pre_head_lif))
    ref = F.linear(torch.from_numpy(s_ph).double(), m.head.weight.detach().double(),
                   m.head.bias.detach().double()).float()
    np.testing.assert_allclose(y.cpu().numpy(), ref.numpy(), rtol=1e-4, atol=1e-4)
    rec = {}
    y_ref = oracle.spikformer_forward(m, x, record=rec)
    if flips == 0:
        # with no flip anywhere, the oracle's own end-to-end layers equal the
        # fused ones: name the first that does not
        got = {f"patch_embed.conv{i}": stage_recs[i] for i in range(4) if i in stage_recs}
        got["patch_embed.rpe_conv"] = stage_recs[4]
        for bi, fb in enumerate(fused.blocks):
            for nm, mod in (("attn.qkv", fb.attn.qkv), ("attn.proj", fb.attn.proj),
                            ("mlp.fc1", fb.mlp.fc1), ("mlp.fc2", fb.mlp.fc2)):
                got[f"blocks.{bi}.{nm}"] = rec_of[id(mod)]
        for name, (r_in, r_s, _) in rec.items():
            if name not in got:
                continue
            g_in, g_id, g_out = got[name]
            g_s = g_out - g_id if g_id is not None else g_out
            assert torch.equal(torch.as_tensor(np.asarray(r_in)).reshape(g_in.shape).float(),
                               g_in.float()), f"{name}: input differs from the oracle's"
            assert torch.equal(torch.as_tensor(np.asarray(r_s)).reshape(g_s.shape), g_s), \
                f"{name}: spikes differ from the oracle's"
        # the unfused pre-head LIF on the token mean: GPU and CPU means of
        # the same integer tokens may differ by an ulp, which can flip a
        # spike whose charge sits on the threshold (k/N can land on it)
        x_att = rec[f"blocks.{len(m.blocks) - 1}.mlp.fc1"][0]
        f_ref = (x_att + rec[f"blocks.{len(m.blocks) - 1}.mlp.fc2"][1]).mean(dim=2)
        s_r, _, h_r = oracle.lif_multistep(f_ref, None, **oracle.lif_params_of(m.pre_head_lif))
        # (the unfused SpikingJelly LIF, on a few hundred neurons: the margin
        # rule only, the flip-fraction rule is for the fused layers' tensors)
        diff = (s_ph != s_r).reshape(s_r.shape[0], -1)
        if diff.any():
            first = diff.argmax(axis=0)[diff.any(axis=0)]
            cols = np.where(diff.any(axis=0))[0]
            margin = np.abs(h_r.reshape(h_r.shape[0], -1)[first, cols]
                            - m.pre_head_lif.v_threshold)
            assert (margin < 1e-4).all(), f"pre-head LIF flip {margin.max():.3e} from threshold"
        else:
            np.testing.assert_allclose(y.cpu().numpy(), y_ref.numpy(), rtol=1e-4, atol=1e-4)
    snn_reset = catfuse_amd.snn.functional.reset_net
    snn_reset(fused)
    with torch.no_grad():
        y2 = fused(x.to(cuda))
    assert torch.equal(y, y2)
    return flips, fused


def test_spikformer_layers_and_logits(cuda):
    m = _small_spikformer()
    img = torch.randn(2, 3, 32, 32, generator=_gen(42))
    _spikformer_parity(cuda, m, img.unsqueeze(0).expand(4, 2, 3, 32, 32), live=True)


@pytest.mark.parametrize("v_th", [1.0, 0.1], ids=["kaiming", "live"])
def test_spikformer_8_384_c4_size(cuda, v_th):
    """Config C4's model at its real dims (384 channels, 12 heads of 32, 8
    blocks, MLP 1536, 224^2 image: 196 tokens; T=4, B=1 of the 32) against
    the oracle layer by layer.  v_th = 0.1 keeps every layer active
    (asserted), so every token linear and attention core runs its
    matrix-core route; v_th = 1.0 is the configured kaiming net, silent
    after the SPS conv1."""
    from catfuse_amd import snn
    m = snn.spikformer_8_384(img_size=224, T=4, v_threshold=v_th)
    g = _gen(43)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    m.eval()
    img = torch.randn(1, 3, 224, 224, generator=g)
    _spikformer_parity(cuda, m, img.unsqueeze(0).expand(4, 1, 3, 224, 224), live=v_th < 1.0)


def test_spikformer_gemm_core_for_other_shapes(cuda):
    """Head dim 64 (the reference's spikformer_cifar_tiny layout), more than
    256 tokens per image and the two-pool patch splitter's 56 x 56 = 3,136
    tokens at 224 x 224 run the two-pass attention kernels
    (cf_spike_attention_kv_lif): no call reaches the library-GEMM core, and
    the network stays at oracle parity."""
    from catfuse_amd import snn
    m = snn.Spikformer(img_size=32, num_classes=10, embed_dim=128, num_heads=2, depth=1, T=4,
                       pools=(0,), v_threshold=0.1)   # head dim 64, 16x16 = 256 tokens
    g = _gen(44)
    snn.kaiming_init(m, g)
    snn.randomize_bn(m, g)
    m.eval()
    img = torch.randn(2, 3, 32, 32, generator=g)
    _, fused = _spikformer_parity(cuda, m, img.unsqueeze(0).expand(4, 2, 3, 32, 32), live=True)
    assert fused.blocks[0].attn.gemm_core_calls == 0
    m2 = snn.Spikformer(img_size=40, num_classes=10, embed_dim=64, num_heads=2, depth=1, T=2,
                        pools=(0,), v_threshold=0.1)   # head dim 32, 20x20 = 400 tokens
    g = _gen(45)
    snn.kaiming_init(m2, g)
    snn.randomize_bn(m2, g)
    m2.eval()
    img = torch.randn(1, 3, 40, 40, generator=g)
    _, fused = _spikformer_parity(cuda, m2, img.unsqueeze(0).expand(2, 1, 3, 40, 40), live=True)
    assert fused.blocks[0].attn.gemm_core_calls == 0
    m3 = snn.Spikformer(img_size=224, num_classes=10, embed_dim=128, num_heads=2, depth=1, T=2,
                        pools=(2, 3), v_threshold=0.1)   # head dim 64, 56x56 = 3,136 tokens
    g = _gen(46)
    snn.kaiming_init(m3, g)
    snn.randomize_bn(m3, g)
    m3.eval()
    img = torch.randn(1, 3, 224, 224, generator=g)
    _, fused = _spikformer_parity(cuda, m3, img.unsqueeze(0).expand(2, 1, 3, 224, 224),
                                  live=True)
    assert fused.blocks[0].attn.gemm_core_calls == 0


def _qkv_copy(T, B, N, C, rate, seed, dev):
    g = _gen(seed)
    qkv = torch.zeros(T * B * N, 3 * C + 32, dtype=torch.float16)   # pitch beyond 3C
    qkv[:, :3 * C] = (torch.rand(T * B * N, 3 * C, generator=g) < rate).half()
    return qkv.to(dev)


@pytest.mark.parametrize("N,heads,dh", [(196, 12, 32), (256, 4, 32), (400, 2, 32), (64, 3, 64),
                                        (256, 2, 64), (3136, 2, 64), (1000, 3, 32)])
def test_attention_two_pass_bitwise(cuda, N, heads, dh):
    """cf_spike_attention_kv_lif: equal to the single-pass kernel bit for bit
    where both apply (head dim 32, N <= 256), and to the exact float64
    evaluation + one rounding + the oracle LIF everywhere (spikes and final
    potentials bit for bit: the products are exact and the LIF tails are
    bit-exact)."""
    from catfuse_amd import runtime
    T, B, scale = 4, 2, 0.125
    lif = dict(tau=2.0, v_threshold=0.5, v_reset=0.0, decay_input=True)
    C = heads * dh
    qkv = _qkv_copy(T, B, N, C, 0.3, seed=N + dh, dev=cuda)
    v0 = (torch.rand(B, N, C, generator=_gen(7)) * 0.3).to(cuda)
    a2, v2 = runtime.spike_attention_lif(qkv, T, B, N, heads, (0, C, 2 * C), scale, v_in=v0,
                                         head_dim=dh, two_pass=True, **lif)
    if dh == 32 and N <= 256:
        a1, v1 = runtime.spike_attention_lif(qkv, T, B, N, heads, (0, C, 2 * C), scale, v_in=v0,
                                             head_dim=dh, two_pass=False, **lif)
        assert torch.equal(a1.cpu(), a2.cpu()) and torch.equal(v1.cpu(), v2.cpu())
    # with the initial state: the oracle's v_in
    s_ref, v_ref, _ = oracle.lif_multistep(
        _attn_z(qkv, T, B, N, heads, dh, scale), v0.cpu(), **lif)
    np.testing.assert_array_equal(a2.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(v2.cpu().numpy(), v_ref)


def _attn_z(qkv, T, B, N, heads, dh, scale):
    C = heads * dh
    t = qkv[:, :3 * C].cpu().double().view(T, B, N, 3, heads, dh).permute(3, 0, 1, 4, 2, 5)
    y = t[0] @ (t[1].transpose(-1, -2) @ t[2])
    return y.permute(0, 1, 3, 2, 4).reshape(T, B, N, C).float() * scale


def test_attention_two_pass_zero_route(cuda):
    """An all-zero Q/K/V copy with its count block publishing zero: the
    two-pass kernels read nothing, z = 0 into the LIF (the initial state
    given, so the output is written), the same as the single-pass kernel."""
    from catfuse_amd import runtime
    T, B, N, heads, dh = 4, 2, 196, 6, 32
    C = heads * dh
    qkv = torch.zeros(T * B * N, 3 * C, dtype=torch.float16, device=cuda)
    nnz = runtime.count_block(cuda)
    v0 = (1.0 + torch.rand(B, N, C, generator=_gen(8)) * 2.0).to(cuda)   # z = 0 halves v
    outs = [runtime.spike_attention_lif(qkv, T, B, N, heads, (0, C, 2 * C), 0.125, v_in=v0,
                                        nnz=nnz, two_pass=tp) for tp in (False, True)]
    assert torch.equal(outs[0][0].cpu(), outs[1][0].cpu())
    assert torch.equal(outs[0][1].cpu(), outs[1][1].cpu())
    assert bool(outs[0][0].cpu().any())          # v0 >= 2 fires at the first step


@pytest.mark.parametrize("shape,k,s,p", [((3, 2, 40, 17, 23), 3, 2, 1), ((2, 3, 96, 20, 15), 3, 2, 1),
                                         ((1, 2, 200, 9, 33), 3, 2, 1), ((2, 2, 64, 8, 8), 2, 2, 0),
                                         ((2, 1, 96, 9, 9), 3, 1, 1)])
def test_maxpool_nhwc_bitwise(cuda, shape, k, s, p):
    """The NHWC max pool of a fused output equals torch's max_pool2d of the
    fp32 tensor, and publishes its output's count block."""
    from catfuse_amd import runtime
    T, B, C, H, W = shape
    v = ((torch.rand(shape, generator=_gen(C)) < 0.2).float()
         * torch.randint(1, 3, shape, generator=_gen(C + 1)).float())
    cp = runtime.pad32(C)
    nhwc = torch.zeros(T * B, H, W, cp, dtype=torch.float16)
    nhwc[..., :C] = v.reshape(T * B, C, H, W).permute(0, 2, 3, 1).half()
    x = runtime.lazy_output(shape, nhwc.to(cuda), cuda)
    blk = runtime.count_block(cuda)
    y = runtime.maxpool_nhwc(x, k, s, p, [0], blk)
    ref = torch.nn.functional.max_pool2d(v.flatten(0, 1), k, s, p)
    assert torch.equal(y.cpu(), ref.reshape(T, B, *ref.shape[1:]))
    assert (int(blk[1].item()) == 0) == (not bool(ref.any()))
    assert runtime.count_of(y) is blk
    zero = runtime.lazy_output(shape, torch.zeros(T * B, H, W, cp, dtype=torch.float16,
                                                  device=cuda), cuda)
    runtime.maxpool_nhwc(zero, k, s, p, [0], blk)
    assert int(blk[1].item()) == 0


DIRECT_POOL_CASES = [
    # (T, B, Cin, Cout, H, W, pad, direct_encoded, with_v_in)
    (4, 2, 3, 48, 32, 32, 1, True, False),
    (3, 2, 3, 32, 29, 23, 1, True, True),
    (2, 3, 4, 64, 17, 30, 2, False, False),
    (5, 1, 1, 16, 15, 16, 0, True, True),
]


@pytest.mark.parametrize("case", DIRECT_POOL_CASES, ids=[f"c{c[3]}_{c[4]}x{c[5]}_p{c[6]}"
                                                          for c in DIRECT_POOL_CASES])
def test_conv_direct_lif_maxpool_bitwise(cuda, case):
    """Analog 3x3 conv -> BN -> LIF -> MaxPool2d(3, 2, 1) in one launch equals
    the direct conv's spikes pooled by torch (bit for bit), its membrane
    equals the direct conv's, and its count block is published."""
    from catfuse_amd import runtime
    T, B, Cin, Cout, H, W, pad, direct, with_v = case
    g = _gen(Cout + H)
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * 0.9
    sc = torch.rand(Cout, generator=g) + 0.5
    sh = torch.randn(Cout, generator=g) * 0.2
    r = runtime.ConvLIFRunner(w.to(cuda), sc.to(cuda), sh.to(cuda), None, 1, pad, 2.0, 1.0,
                              0.0, True)
    img = torch.randn(B, Cin, H, W, generator=g).to(cuda)
    x = (img.unsqueeze(0).expand(T, B, Cin, H, W) if direct
         else torch.randn(T, B, Cin, H, W, generator=g).to(cuda))
    Ho, Wo = r.out_hw(H, W)
    v_in = (torch.rand(B, Cout, Ho, Wo, generator=g) * 0.8).to(cuda) if with_v else None
    assert r.direct_pool_supported(x, (3, 2, 1))
    ref_s, ref_v = r.run_direct(x, v_in)
    ref = torch.nn.functional.max_pool2d(ref_s.flatten(0, 1), 3, 2, 1)
    blk = runtime.count_block(cuda)
    y, v = r.run_direct_pool(x, v_in, nz_out=blk, gen_cell=[0])
    assert tuple(y.shape) == (T, B, Cout) + tuple(ref.shape[-2:])
    assert torch.equal(y.reshape(T * B, *ref.shape[1:]), ref)
    assert torch.equal(v, ref_v)
    cp = runtime.pad32(Cout)
    copy = runtime.shadow_of(y, (T * B,) + tuple(ref.shape[-2:]) + (cp,))
    assert copy is not None and not bool(copy[..., Cout:].any())
    assert (int(blk[1].item()) == 0) == (not bool(ref.any()))
    assert runtime.count_of(y) is blk
    # a second call on the same block (smaller batch) republishes
    y2, _ = r.run_direct_pool(x[:, :1], None if v_in is None else v_in[:1], nz_out=blk,
                              gen_cell=[0])
    assert torch.equal(y2.reshape(T, *ref.shape[1:]), ref.reshape(T, B, *ref.shape[1:])[:, 0])


@pytest.mark.parametrize("B,N,C,silent", [(4, 196, 384, False), (2, 64, 96, False),
                                          (3, 50, 40, False), (4, 196, 384, True)])
def test_token_mean_reads_copy(cuda, B, N, C, silent):
    """x.mean(dim=2) of a token layer's lazy output [T, B, N, C] is computed
    from its fp16 copy (through its descriptor; an elided all-zero copy gives
    zeros) without materialising x, bit-identical to torch's mean of the
    fp32 values."""
    from catfuse_amd import runtime
    T, Cin = 4, 64
    g = _gen(B * N + C)
    w = torch.randn(C, Cin, 1, 1, generator=g) * 0.4
    sh = torch.full((C,), -0.5) if silent else torch.randn(C, generator=g) * 0.5
    r = runtime.ConvLIFRunner(w.to(cuda), torch.ones(C, device=cuda), sh.to(cuda), None, 1, 0,
                              2.0, 1.0, 0.0, True)
    x = (torch.rand(T, B, N, Cin, generator=g) < (0.0 if silent else 0.3)).float().to(cuda)
    y, _ = r.run_tokens(x)
    if silent:   # StaticZero with a silent bias response: the copy is elided
        d = runtime.desc_of(y)
        assert d is not None and int(d[0].item() & 0xffffffff) == 1
    m = y.mean(dim=2)
    m2 = y.mean(-2)
    assert y.__dict__.get("_cf_pending"), "the mean materialised the tokens"
    ref = y.clone().mean(dim=2)
    assert m.shape == (T, B, C) and torch.equal(m, ref) and torch.equal(m2, ref)
    assert bool(ref.any()) != silent


def test_spike_attention_count_block(cuda):
    """The attention core publishes its output's count block (zero iff no
    spike) and attaches it to the output, so the proj linear can take the
    StaticZero route on it."""
    from catfuse_amd import runtime
    T, B, N, heads = 4, 2, 64, 2
    C = 32 * heads
    blk = runtime.count_block(cuda)
    for density, v_th in ((0.3, 0.5), (0.0, 1.0)):
        qkv = (torch.rand(T * B * N, 3 * C, generator=_gen(7)) < density).half().to(cuda)
        out, _ = runtime.spike_attention_lif(qkv, T, B, N, heads, (0, C, 2 * C), 0.125,
                                             v_threshold=v_th, nz_out=blk, gen_cell=[0])
        assert runtime.count_of(out) is blk
        assert (int(blk[1].item()) == 0) == (not bool(out.any()))
        if density == 0.0:
            assert int(blk[1].item()) == 0
        else:
            assert bool(out.any())
