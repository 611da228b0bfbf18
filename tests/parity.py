"""Parity criteria shared by the GPU tests.

Floating-point LIF layers after a convolution are compared with the CPU
oracle under the north-star tolerance:
  * spikes: a disagreement is allowed only where the oracle's charged
    potential h at that step satisfies |h - v_th| < 1e-4 (checked at the
    first disagreeing step of each neuron; later steps of that neuron follow
    a different reset history), and fewer than 1e-4 of all spikes may flip;
  * membrane potential: for neurons whose spike trains agree,
    |v - v_ref| <= 1e-4 * max(|v_ref|, v_th)  (1e-4 relative, with the
    threshold as the scale for potentials near zero).
Integer/bitmask outputs and element-wise LIF tails are compared bit-exactly
elsewhere.
"""
import numpy as np

SPIKE_FLIP_FRACTION = 1e-4
V_REL_TOL = 1e-4
NEAR_THRESHOLD = 1e-4


def lif_parity(spikes, v, spikes_ref, v_ref, h_ref, v_th=1.0, what=""):
    spikes = np.asarray(spikes, dtype=np.float32)
    spikes_ref = np.asarray(spikes_ref, dtype=np.float32)
    T = spikes.shape[0]
    s = spikes.reshape(T, -1)
    sr = spikes_ref.reshape(T, -1)
    h = np.asarray(h_ref).reshape(T, -1)
    diff = s != sr
    n_flip = int(diff.sum())
    frac = n_flip / max(1, s.size)
    assert frac < SPIKE_FLIP_FRACTION, f"{what}: {n_flip} flipped spikes ({frac:.2e})"
    neurons = np.where(diff.any(axis=0))[0]
    if neurons.size:
        first_t = diff[:, neurons].argmax(axis=0)
        margin = np.abs(h[first_t, neurons] - v_th)
        assert (margin < NEAR_THRESHOLD).all(), (
            f"{what}: flip with |h - v_th| = {margin.max():.3e} >= {NEAR_THRESHOLD}")
    if v is not None:
        vv = np.asarray(v, dtype=np.float32).reshape(-1)
        vr = np.asarray(v_ref, dtype=np.float32).reshape(-1)
        ok = np.ones(vv.shape, bool)
        ok[neurons] = False
        scale = np.maximum(np.abs(vr[ok]), v_th)
        err = np.abs(vv[ok] - vr[ok]) / scale
        assert err.size == 0 or err.max() <= V_REL_TOL, (
            f"{what}: membrane rel err {err.max():.3e} > {V_REL_TOL}")
    return n_flip


def pooled_parity(pooled, spikes_ref, h_ref, pool=(3, 2, 1), v_th=1.0, what=""):
    """Max-pooled spikes of a fused Conv->BN->LIF->MaxPool against
    max_pool2d of the oracle's conv-resolution spikes.  A pooled output may
    differ only where some neuron of its window was within NEAR_THRESHOLD of
    v_th at some step up to t (its spike could have flipped), and fewer than
    SPIKE_FLIP_FRACTION of the outputs may differ."""
    import torch
    import torch.nn.functional as F
    k, s, p = pool
    sr = torch.from_numpy(np.asarray(spikes_ref, dtype=np.float32))
    T, B, C, Hc, Wc = sr.shape
    ref = F.max_pool2d(sr.reshape(T * B, C, Hc, Wc), k, s, p)
    near = torch.from_numpy(np.abs(np.asarray(h_ref) - v_th) < NEAR_THRESHOLD)
    near = torch.cummax(near.reshape(T, -1).to(torch.int32), dim=0).values.float()
    near = F.max_pool2d(near.reshape(T * B, C, Hc, Wc), k, s, p)
    got = torch.as_tensor(np.asarray(pooled, dtype=np.float32)).reshape(ref.shape)
    diff = got != ref
    frac = int(diff.sum()) / max(1, diff.numel())
    assert frac < SPIKE_FLIP_FRACTION, f"{what}: {int(diff.sum())} pooled outputs differ"
    assert bool((near[diff] > 0).all()), f"{what}: pooled output differs away from threshold"
    return int(diff.sum())


def membrane_parity(v, v_ref, h_ref, v_th=1.0, what=""):
    """Final membrane of neurons never within NEAR_THRESHOLD of v_th (whose
    spike trains cannot have flipped): |v - v_ref| <= V_REL_TOL * max(|v_ref|, v_th)."""
    h = np.asarray(h_ref)
    T = h.shape[0]
    safe = ~(np.abs(h.reshape(T, -1) - v_th) < NEAR_THRESHOLD).any(axis=0)
    vv = np.asarray(v, dtype=np.float32).reshape(-1)[safe]
    vr = np.asarray(v_ref, dtype=np.float32).reshape(-1)[safe]
    err = np.abs(vv - vr) / np.maximum(np.abs(vr), v_th)
    assert err.size == 0 or err.max() <= V_REL_TOL, f"{what}: membrane rel err {err.max():.3e}"
