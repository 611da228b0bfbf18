"""cf_conv_sparse_noalloc (routing workspace in the library's static device
array, no allocation) against the existing path it replaces for callers
that cannot allocate: cf_scan_nhwc + cf_prescan_tiles + cf_conv_mfma with
caller buffers.  Both through the C-ABI, results compared bit for bit, on
consecutive calls of different sizes (the second smaller, so stale
workspace from the first call would show)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

CF_ERROR_NOALLOC_LIMIT = 7001


def _layer(Cin, Cout, dev, seed, k=3, s=1, p=1):
    from catfuse_amd.runtime import ConvLIFRunner
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(Cout, Cin, k, k, generator=g) * (2.0 / (Cin * k * k)) ** 0.5
    scale = torch.rand(Cout, generator=g) + 0.5
    shift = torch.randn(Cout, generator=g) * 0.1
    r = ConvLIFRunner(w.to(dev), scale.to(dev), shift.to(dev), None, s, p, 2.0, 1.0, 0.0, True)
    r._ensure_packed(dev)
    return r


def _input(T, B, C, H, W, cp, rate, dev, seed):
    """A fused layer's output copy: fp16 NHWC spikes [T*B, H, W, cp] with
    8x8 blocks silent in all channels (so SparseFlow skips chunks)."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T * B, H, W, C, generator=g) < rate).half()
    keep = (torch.rand(T * B, (H + 7) // 8, (W + 7) // 8, 1, generator=g) > 0.6).half()
    keep = keep.repeat_interleave(8, 1).repeat_interleave(8, 2)[:, :H, :W]
    xp = torch.zeros(T * B, H, W, cp, dtype=torch.float16)
    xp[..., :C] = x * keep
    return xp.to(dev)


def _outputs(r, T, B, H, W, dev):
    Cout, cp = r.Cout, ((r.Cout + 31) // 32) * 32
    out = torch.full((T, B, Cout, H, W), -7.0, device=dev)
    nhwc = torch.full((T * B, H, W, cp), -7.0, dtype=torch.float16, device=dev)
    v_out = torch.full((B, Cout, H, W), -7.0, device=dev)
    nz = torch.zeros(272, dtype=torch.int64, device=dev)
    return out, nhwc, v_out, nz


def _lif():
    return (2.0, 1.0, 0.0, 1, 1)


def _geom(H, W, k, s, p):
    return (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1


def _existing(r, xp, T, B, C, H, W, tile, gs, thr, dev, k=3, s=1, p=1):
    """scan + prescan + routed conv with caller-allocated workspace."""
    from catfuse_amd import _hip
    from catfuse_amd._hip import ptr
    L, st = _hip.lib(), _hip.stream(dev)
    NB = T * B
    act = torch.empty((NB, H, W), dtype=torch.int32, device=dev)
    blk = torch.zeros(272, dtype=torch.int64, device=dev)
    Ho, Wo = _geom(H, W, k, s, p)
    GH, GW = -(-Ho // tile[0]), -(-Wo // tile[1])
    ag = torch.empty(NB * GH * GW, dtype=torch.int32, device=dev)
    tc = torch.empty(NB * GH * GW, dtype=torch.int32, device=dev)
    assert L.cf_scan_nhwc(ptr(xp), NB, H, W, r.Cp, C, ptr(act), gs, 1e-6, ptr(blk), st) == 0
    assert L.cf_prescan_tiles(ptr(act), NB, H, W, Ho, Wo, k, s, p, tile[0], tile[1], -(-C // gs),
                              ptr(ag), ptr(tc), st) == 0
    out, nhwc, v_out, nz = _outputs(r, T, B, Ho, Wo, dev)
    cp = nhwc.shape[-1]
    assert L.cf_conv_mfma(ptr(xp), ptr(r.w_packed), ptr(r.alpha), ptr(r.beta), None, ptr(v_out),
                          ptr(out), ptr(nhwc), cp, None, None, cp, 1, ptr(ag), None, ptr(blk), ptr(nz),
                          None, None, None, 0, None, NB * C * H * W, thr, T, B, r.Cp, r.Cout, r.Coutp,
                          H, W, Ho, Wo, k, k, s, p, B, tile[0], tile[1], gs, 0, *_lif(), st) == 0
    return out, nhwc, v_out, nz, blk


def _noalloc(r, xp, T, B, C, H, W, tile, gs, thr, dev, k=3, s=1, p=1):
    from catfuse_amd import _hip
    from catfuse_amd._hip import ptr
    L, st = _hip.lib(), _hip.stream(dev)
    Ho, Wo = _geom(H, W, k, s, p)
    out, nhwc, v_out, nz = _outputs(r, T, B, Ho, Wo, dev)
    cp = nhwc.shape[-1]
    rc = L.cf_conv_sparse_noalloc(ptr(xp), C, ptr(r.w_packed), ptr(r.alpha), ptr(r.beta), None,
                                  ptr(v_out), ptr(out), ptr(nhwc), cp, None, None, cp, 1, ptr(nz),
                                  thr, T, B, r.Cp, r.Cout, r.Coutp, H, W, Ho, Wo, k, s, p, tile[0],
                                  tile[1], gs, 0, *_lif(), st)
    assert rc == 0, rc
    return out, nhwc, v_out, nz


CASES = [
    # T, B, Cin, Cout, H, W, tile, group size, rate, SparseFlow threshold, (k, s, p)
    (4, 8, 256, 256, 14, 14, (8, 8), 32, 0.05, 0.7, (3, 1, 1)),   # config C1 shape (B = 8)
    (2, 3, 64, 64, 20, 22, (8, 16), 16, 0.1, 0.7, (3, 1, 1)),     # smaller: second call
    (3, 2, 96, 64, 9, 11, (8, 8), 32, 0.2, 1.0, (3, 1, 1)),       # dense route
    (2, 2, 64, 64, 8, 8, (8, 8), 16, 0.0, 0.7, (3, 1, 1)),        # all zero: StaticZero
    (4, 4, 64, 128, 28, 28, (8, 8), 16, 0.05, 0.7, (3, 2, 1)),    # stride-2 3x3 (one halo buffer)
    (4, 4, 128, 256, 28, 28, (8, 8), 32, 0.05, 0.7, (1, 2, 0)),   # 1x1 stride-2 downsample
    (2, 3, 64, 128, 16, 16, (8, 8), 16, 0.1, 0.7, (1, 1, 0)),     # 1x1 stride 1
]


def test_noalloc_equals_existing_path_on_consecutive_calls(cuda):
    for i, (T, B, Cin, Cout, H, W, tile, gs, rate, thr, (k, s, p)) in enumerate(CASES):
        r = _layer(Cin, Cout, cuda, seed=10 + i, k=k, s=s, p=p)
        xp = _input(T, B, Cin, H, W, r.Cp, rate, cuda, seed=20 + i)
        geo = dict(k=k, s=s, p=p)
        print(f"no-alloc case {i}: T={T} B={B} {Cin}->{Cout} {H}x{W} k{k} s{s}", flush=True)
        a_out, a_nhwc, a_v, a_nz, blk = _existing(r, xp, T, B, Cin, H, W, tile, gs, thr, cuda, **geo)
        b_out, b_nhwc, b_v, b_nz = _noalloc(r, xp, T, B, Cin, H, W, tile, gs, thr, cuda, **geo)
        torch.cuda.synchronize()
        what = f"case {i} {(T, B, Cin, Cout, H, W, k, s)}"
        assert torch.equal(a_out, b_out), what
        assert torch.equal(a_nhwc, b_nhwc), what
        assert torch.equal(a_v, b_v), what
        assert int(a_nz[1]) == int(b_nz[1]), what
        nnz = int(blk[1])
        assert nnz == int(torch.count_nonzero(xp)), what
        assert (rate == 0.0) == (nnz == 0), what
        # a second call of the same case: same results (the workspace kept
        # from the call before does not leak into this one)
        c_out, c_nhwc, c_v, _ = _noalloc(r, xp, T, B, Cin, H, W, tile, gs, thr, cuda, **geo)
        assert torch.equal(a_nhwc, c_nhwc) and torch.equal(a_v, c_v), what


def test_noalloc_rejects_inputs_beyond_its_workspace(cuda):
    from catfuse_amd import _hip
    L = _hip.lib()
    r = _layer(64, 64, cuda, seed=3)
    # 2^21 + 1 input pixels: rejected before any launch
    T, B, H, W = 1, 1, 1, (1 << 21) + 1
    rc = L.cf_conv_sparse_noalloc(1, 64, 1, 1, 1, None, 1, 1, None, 64, None, None, 64, 1, None,
                                  0.7, T, B, 64, 64, 64, H, W, H, W, 3, 1, 1, 8, 8, 16, 0, 2.0,
                                  1.0, 0.0, 1, 1, _hip.stream(cuda))
    assert rc == CF_ERROR_NOALLOC_LIMIT
    assert b"workspace" in L.cf_error_string(rc)
