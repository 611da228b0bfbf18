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
