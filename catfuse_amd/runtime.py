"""Launch layer: torch tensors in, gfx950 C-ABI calls out.

Each function validates shapes/dtypes/devices on the host, allocates its
outputs with torch (device memory plumbing) and launches on torch's current
HIP stream.  Nothing here computes on the CPU and nothing falls back: a
missing library or a non-GPU tensor raises.

`ConvLIFRunner` owns the per-layer device state of a fused Conv->BN->LIF:
packed fp16 hi/lo weights, the folded epilogue affine, the fp16 NHWC staging
buffer, prescan buffers and the nonzero counter.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

from catfuse_amd import _hip
from catfuse_amd._hip import check, ptr, require_gpu_tensor

EPI_LIF, EPI_Z, EPI_POOL = 0, 1, 2
ID_ADD_SPIKE, ID_ADD_Z = 1, 2
ROUTE_ZERO, ROUTE_SPARSE, ROUTE_DENSE = 0, 1, 2
STATUS_INEXACT_FP16 = 1
STATUS_FP16_RANGE = 2

_status_words: dict = {}


class KernelTimer:
    """Optional live timing of kernel launches with HIP events recorded on
    the launch stream (torch's current stream, which every wrapper here
    launches on).  Each record carries the launch's algorithmic work (FLOPs
    and/or bytes) so callers can report achieved rates per kernel.

    settle_cycles > 0 queues a bounded spin kernel (torch.cuda._sleep) ahead
    of each start event, so the GPU is still busy while the host prepares
    and issues the launch: start event, kernel and end event then run back
    to back and the interval is the kernel's own duration, also for launches
    shorter than the host's per-launch overhead."""

    def __init__(self, settle_cycles: int = 0):
        self.records = []   # (name, start_event, end_event, flops, bytes, route probe)
        self.settle_cycles = int(settle_cycles)

    def start(self):
        if self.settle_cycles > 0:
            torch.cuda._sleep(self.settle_cycles)
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def stop(self, name, ev0, flops=0, nbytes=0, route=None):
        ev1 = torch.cuda.Event(enable_timing=True)
        ev1.record()
        self.records.append((name, ev0, ev1, int(flops), int(nbytes), route))

    def summary(self):
        """{name: dict(launches, ms_total, ms_avg, flops, bytes)} (synchronises).
        A conv launch that took the StaticZero route (read from its input's
        count block when the summary is made) is listed under
        name + "_staticzero" with no FLOPs and the output bytes it stored
        ("elided": launches that stored none, their descriptor recording the
        outputs)."""
        torch.cuda.synchronize()
        out = {}
        for name, e0, e1, fl, nb, route in self.records:
            el = 0
            if route is not None and route.is_zero():
                name, fl, nb = name + "_staticzero", 0, route.bytes_stored()
                el = int(nb == 0)
            d = out.setdefault(name, dict(launches=0, ms_total=0.0, flops=0, bytes=0, elided=0))
            d["launches"] += 1
            d["ms_total"] += e0.elapsed_time(e1)
            d["flops"] += fl
            d["bytes"] += nb
            d["elided"] += el
        for d in out.values():
            d["ms_avg"] = d["ms_total"] / max(1, d["launches"])
        return out


_timer = None


def set_timer(timer):
    """Install (or remove with None) the process-wide KernelTimer."""
    global _timer
    _timer = timer


def _t0():
    return _timer.start() if _timer is not None else None


def _t1(name, ev0, flops=0, nbytes=0, route=None):
    if ev0 is not None:
        _timer.stop(name, ev0, flops, nbytes, route)


class _RouteProbe:
    """The StaticZero decision of a conv launch, read back from the input's
    count block (published count zero) after the launches complete, and
    the output bytes it stored on that route.  parts: one (output
    descriptor or None, copy bytes, state bytes) per output; a descriptor
    that records the copy / the state as unwritten removes those bytes."""
    __slots__ = ("blk", "parts")

    def __init__(self, blk, parts):
        self.blk = blk
        self.parts = tuple(parts)

    def is_zero(self) -> bool:
        return int(self.blk[1].item()) == 0

    def bytes_stored(self) -> int:
        b = 0
        for d, copy_bytes, state_bytes in self.parts:
            w = 0 if d is None else int(d[0].item())
            copy, vstate = w & 0xffffffff, (w >> 32) & 0xffffffff
            b += (copy_bytes if copy == 0 else 0) + (state_bytes if vstate == 0 else 0)
        return b


def status_word(device) -> torch.Tensor:
    """Per-device sticky status word (int32[1]) OR-ed by the pack kernel."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    t = _status_words.get(key)
    if t is None:
        t = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", key))
        _status_words[key] = t
    return t


def read_status(device=None) -> int:
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    return int(status_word(dev).item())


def clear_status(device=None) -> None:
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    status_word(dev).zero_()


def _lif_args(tau, v_threshold, v_reset, decay_input):
    hard = v_reset is not None
    return (float(tau), float(v_threshold), float(v_reset) if hard else 0.0, int(hard),
            int(bool(decay_input)))


# ---------------------------------------------------------------------------
# LIF family
# ---------------------------------------------------------------------------

def lif_multistep(z: torch.Tensor, v_in: Optional[torch.Tensor] = None, *, tau=2.0,
                  v_threshold=1.0, v_reset=0.0, decay_input=True, mode=0,
                  z2: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None,
                  shift: Optional[torch.Tensor] = None, channels: int = 1, hw: int = 1,
                  spike_dtype=torch.float32, want_v_out: bool = True):
    """z [T, ...] -> (spikes [T, ...], v_out [...] or None) on the GPU."""
    require_gpu_tensor(z, "z")
    T = z.shape[0]
    N = z[0].numel() if T > 0 else 0
    if z2 is not None:
        require_gpu_tensor(z2, "z2")
        if z2.shape != z.shape:
            raise ValueError(f"z2 shape {tuple(z2.shape)} != z shape {tuple(z.shape)}")
    for name, t in (("scale", scale), ("shift", shift)):
        if t is not None:
            require_gpu_tensor(t, name)
            if t.numel() != channels:
                raise ValueError(f"{name} has {t.numel()} entries, expected {channels}")
    if v_in is not None:
        require_gpu_tensor(v_in, "v_in")
        if v_in.numel() != N:
            raise ValueError(f"v_in has {v_in.numel()} elements, expected {N}")
    if mode in (1, 2, 4) and (N % (channels * hw) != 0):
        raise ValueError("N must be a multiple of channels*hw for per-channel modes")
    sd = {torch.float32: 0, torch.uint8: 1}.get(spike_dtype)
    if sd is None:
        raise TypeError("spike_dtype must be float32 or uint8")
    spikes = torch.empty(z.shape, dtype=spike_dtype, device=z.device)
    v_out = torch.empty(z.shape[1:], dtype=torch.float32, device=z.device) if want_v_out else None
    ev = _t0()
    rc = _hip.lib().cf_lif_multistep(ptr(z), ptr(z2), ptr(scale), ptr(shift), int(mode), ptr(v_in),
                                     ptr(spikes), sd, ptr(v_out), T, N, int(channels), int(hw),
                                     *_lif_args(tau, v_threshold, v_reset, decay_input),
                                     _hip.stream(z.device))
    check(rc, "cf_lif_multistep")
    nbytes = T * N * (4 + (4 if z2 is not None else 0) + spikes.element_size()) + \
        4 * N * ((v_in is not None) + (v_out is not None))
    _t1(f"lif_multistep_mode{mode}", ev, nbytes=nbytes)
    return spikes, v_out


def avgpool2x2_lif(x: torch.Tensor, v_in: Optional[torch.Tensor] = None, *, tau=2.0,
                   v_threshold=1.0, v_reset=0.0, decay_input=True, spike_dtype=torch.float32):
    """x [T, B, C, H, W] -> (spikes [T, B, C, H//2, W//2], v_out)."""
    require_gpu_tensor(x, "x")
    if x.dim() != 5:
        raise ValueError("x must be [T, B, C, H, W]")
    T, B, C, H, W = x.shape
    if H < 2 or W < 2:
        raise ValueError("AvgPool2x2 needs H, W >= 2")
    Ho, Wo = H // 2, W // 2
    if v_in is not None:
        require_gpu_tensor(v_in, "v_in")
        if v_in.numel() != B * C * Ho * Wo:
            raise ValueError("v_in has the wrong size")
    sd = {torch.float32: 0, torch.uint8: 1}[spike_dtype]
    spikes = torch.empty((T, B, C, Ho, Wo), dtype=spike_dtype, device=x.device)
    v_out = torch.empty((B, C, Ho, Wo), dtype=torch.float32, device=x.device)
    ev = _t0()
    rc = _hip.lib().cf_avgpool2x2_lif(ptr(x), ptr(v_in), ptr(spikes), sd, ptr(v_out), T, B * C, H,
                                      W, *_lif_args(tau, v_threshold, v_reset, decay_input),
                                      _hip.stream(x.device))
    check(rc, "cf_avgpool2x2_lif")
    n_out = B * C * Ho * Wo
    _t1("avgpool2x2_lif", ev, nbytes=T * n_out * (16 + spikes.element_size()) +
        4 * n_out * (1 + (v_in is not None)))
    return spikes, v_out


# ---------------------------------------------------------------------------
# Prescan
# ---------------------------------------------------------------------------

# Element of the NHWC spike copies fused layers exchange: "f16" (two bytes
# per channel) or "u8" (one byte; the copies hold integers 0..255: spikes,
# SEW sums).  The halo convolutions (single and paired), the stem, the head
# average pool and materialisation read and write byte copies natively;
# every other reader gets the copy widened to fp16 (cf_copy_u8_to_f16,
# counted in U8_WIDENED).  Results are the same bit for bit in both formats.
SPIKE_COPY = os.environ.get("CATFUSE_SPIKE_COPY", "f16")
U8_WIDENED = [0]


def set_spike_copy(fmt: str) -> None:
    """Select the spike-copy format of the fused layers that produce copies
    from now on: "f16" or "u8"."""
    global SPIKE_COPY
    if fmt not in ("f16", "u8"):
        raise ValueError("spike copy format must be 'f16' or 'u8'")
    SPIKE_COPY = fmt


def spike_copy() -> str:
    return SPIKE_COPY


def _widen(x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """x's byte copy t (resolved first) as a new fp16 copy of the same
    layout, for a reader that takes fp16 copies only."""
    _resolve(x, t)
    w = torch.empty(t.shape, dtype=torch.float16, device=t.device)
    check(_hip.lib().cf_copy_u8_to_f16(ptr(t), ptr(w), t.numel(), _hip.stream(t.device)),
          "cf_copy_u8_to_f16")
    U8_WIDENED[0] += 1
    return w


def pad32(c: int) -> int:
    return ((c + 31) // 32) * 32


# ---------------------------------------------------------------------------
# fp32 outputs kept as their fp16 NHWC copy until first read
# ---------------------------------------------------------------------------

def _metadata_functions():
    T = torch.Tensor
    props = ("shape", "dtype", "device", "is_cuda", "ndim", "_version", "requires_grad",
             "layout", "is_sparse", "is_quantized", "is_meta", "grad_fn", "names")
    fns = {getattr(T, p).__get__ for p in props if hasattr(T, p)}
    fns |= {T.dim, T.size, T.stride, T.numel, T.nelement, T.is_contiguous, T.storage_offset,
            T.element_size, T.is_floating_point, T.get_device, T.__len__}
    return fns


_METADATA = None


def _ver(x: torch.Tensor) -> int:
    """x._version, read from the plain tensor a lazy output was made from
    (it shares x's version counter) so no torch-function dispatch runs."""
    return x.__dict__.get("_cf_base", x)._version


def _meta_of(base: torch.Tensor) -> tuple:
    """(shape, dtype, device, numel, contiguous) of a plain tensor."""
    return (base.shape, base.dtype, base.device, base.numel(), base.is_contiguous())


class _LazyTensor(torch.Tensor):
    """Base of the tensors whose values a fused launch left elsewhere (a
    copy, a per-channel buffer): cf_materialize() fills the storage, which
    happens the first time anything other than a metadata query touches
    the tensor.  Results of torch operations are plain tensors."""

    def cf_materialize(self) -> None:  # pragma: no cover - overridden
        raise NotImplementedError

    # Metadata recorded when the tensor is made (_cf_meta: shape, dtype,
    # device, numel, contiguous), served while it is pending without the
    # torch-function dispatch a tensor subclass otherwise pays for every
    # query (the fused layers ask several per launch).  Nothing but
    # metadata queries has touched a pending tensor (any other operation
    # materialises it first), so the record is current; afterwards the
    # queries take the ordinary path.
    def _cf_meta_now(self):
        d = self.__dict__
        return d.get("_cf_meta") if d.get("_cf_pending", False) else None

    @property
    def shape(self):
        m = self._cf_meta_now()
        return m[0] if m is not None else super().shape

    @property
    def dtype(self):
        m = self._cf_meta_now()
        return m[1] if m is not None else super().dtype

    @property
    def device(self):
        m = self._cf_meta_now()
        return m[2] if m is not None else super().device

    @property
    def is_cuda(self):
        m = self._cf_meta_now()
        return m[2].type == "cuda" if m is not None else super().is_cuda

    @property
    def ndim(self):
        m = self._cf_meta_now()
        return len(m[0]) if m is not None else super().ndim

    def dim(self):
        m = self._cf_meta_now()
        return len(m[0]) if m is not None else super().dim()

    def numel(self):
        m = self._cf_meta_now()
        return m[3] if m is not None else super().numel()

    def is_contiguous(self, memory_format=torch.contiguous_format):
        m = self._cf_meta_now()
        if m is not None and memory_format is torch.contiguous_format:
            return m[4]
        return super().is_contiguous(memory_format=memory_format)

    def contiguous(self, memory_format=torch.contiguous_format):
        m = self._cf_meta_now()
        if m is not None and memory_format is torch.contiguous_format and m[4]:
            return self
        return super().contiguous(memory_format=memory_format)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        global _METADATA
        if _METADATA is None:
            _METADATA = _metadata_functions()
        kwargs = kwargs or {}
        if func is torch.mean or func is torch.Tensor.mean:
            y = _token_mean(args, kwargs)
            if y is not None:
                return y
        self_ok = func is torch.Tensor.contiguous and args and args[0].is_contiguous()
        if not self_ok and func not in _METADATA:
            for a in _tensors_in(args, kwargs):
                if isinstance(a, _LazyTensor):
                    a.cf_materialize()
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)


def _token_mean(args, kwargs) -> Optional[torch.Tensor]:
    """x.mean(dim=-2) of a token-major fused output x [..., N, C] (the token
    average of a spiking transformer's head) from x's fp16 copy, read
    through its descriptor, without the fp32 form: cf_global_avgpool_nhwc
    over the N tokens of each row (an exact integer sum times float(1/N),
    the value torch's mean computes).  None for any other call."""
    if not args or len(args) > 2 or set(kwargs) - {"dim"}:
        return None
    x = args[0]
    dim = args[1] if len(args) > 1 else kwargs.get("dim")
    if not (isinstance(x, NHWCSpikes) and x.__dict__.get("_cf_pending", False)
            and x.__dict__.get("_cf_tokens", False) and x.dim() >= 3):
        return None
    if isinstance(dim, (tuple, list)):
        if len(dim) != 1:
            return None
        dim = dim[0]
    if not isinstance(dim, int) or dim % x.dim() != x.dim() - 2:
        return None
    N, C = int(x.shape[-2]), int(x.shape[-1])
    copy = token_shadow(x, pad32(C), resolve=False)
    if copy is None or copy.shape[0] % N:
        return None
    y = global_avgpool_nhwc(copy.view(copy.shape[0] // N, N, 1, copy.shape[1]), C,
                            desc=desc_of(x))
    return y.view(*x.shape[:-2], C)


class NHWCSpikes(_LazyTensor):
    """An fp32 NCHW [T, B, C, H, W] output of a fused layer whose values were
    written only as the fp16 NHWC copy the next fused layer reads.  The fp32
    storage is filled (cf_nhwc_to_nchw) the first time anything other than a
    metadata query touches the tensor, so code outside the fused chain sees
    an ordinary tensor with the right values; fused layers that take the copy
    never pay for the fp32 form.  A copy its producer did not write (output
    descriptor: all zero, or an alias of the identity's copy) is resolved
    first (cf_resolve_copy)."""

    @staticmethod
    def __new__(cls, base: torch.Tensor, nhwc: torch.Tensor, tokens: bool = False, meta=None):
        # meta: base's _meta_of record when the caller already holds it
        t = base.as_subclass(cls)
        t._cf_meta = _meta_of(base) if meta is None else meta
        t._cf_base = base
        t._cf_pending = True
        t._cf_tokens = tokens
        t._cf_nhwc = (nhwc, base._version)
        return t

    def cf_materialize(self) -> None:
        if not self.__dict__.get("_cf_pending", False):
            return
        self._cf_pending = False
        with torch._C.DisableTorchFunctionSubclass():
            nhwc = self._cf_nhwc[0]
            _resolve(self, nhwc)
            cp = nhwc.shape[-1]
            if nhwc.dtype == torch.uint8 and self.__dict__.get("_cf_tokens", False):
                nhwc = _widen(self, nhwc)
            if self.__dict__.get("_cf_tokens", False):
                # token-major [..., N, C]: a cast of the copy, dropping padding
                C = self.shape[-1]
                check(_hip.lib().cf_tokens_to_f32(nhwc.data_ptr(), self.data_ptr(),
                                                  self.numel() // C, C, cp,
                                                  _hip.stream(self.device)), "cf_tokens_to_f32")
                return
            T, B, C, H, W = self.shape
            fn = (_hip.lib().cf_nhwc_to_nchw_u8 if nhwc.dtype == torch.uint8
                  else _hip.lib().cf_nhwc_to_nchw)
            check(fn(nhwc.data_ptr(), self.data_ptr(), T * B, C, H, W, cp,
                     _hip.stream(self.device)), "cf_nhwc_to_nchw")


class ChannelState(_LazyTensor):
    """A fused layer's membrane state [B, C, H, W] that its launch may have
    kept as one potential per channel (on the StaticZero route with no
    initial state every pixel of a channel ends at the same value; the
    output descriptor says whether it did).  Expanded into the storage
    (cf_expand_state) on first use.  A state made inside a HIP graph
    capture is expanded again on every use until it is changed in place,
    since each replay rewrites the per-channel values."""

    @staticmethod
    def __new__(cls, base: torch.Tensor, v_chan: torch.Tensor, desc: torch.Tensor,
                uniform: bool = False, meta=None):
        # meta: base's _meta_of record when the caller already holds it
        t = base.as_subclass(cls)
        t._cf_meta = _meta_of(base) if meta is None else meta
        t._cf_base = base
        t._cf_pending = True
        t._cf_state = (v_chan, desc, base._version)
        t._cf_sticky = torch.cuda.is_current_stream_capturing()
        t._cf_uniform = uniform      # one value (v_chan[0]) for every element
        return t

    def cf_materialize(self) -> None:
        if not self.__dict__.get("_cf_pending", False):
            return
        with torch._C.DisableTorchFunctionSubclass():
            v_chan, desc, ver = self._cf_state
            if not (self.__dict__.get("_cf_sticky", False) and self._version == ver):
                self._cf_pending = False
            if self._version != ver:
                return   # changed in place after an earlier expansion
            if self.__dict__.get("_cf_uniform", False):
                B, C = 1, 1
            else:
                B, C = self.shape[0], self.shape[1]
            check(_hip.lib().cf_expand_state(self.data_ptr(), v_chan.data_ptr(), desc.data_ptr(),
                                             B, C, self.numel() // (B * C),
                                             _hip.stream(self.device)), "cf_expand_state")


def lazy_view(t: torch.Tensor, *shape) -> torch.Tensor:
    """t.view(*shape), keeping a ChannelState lazy (the view expands itself
    on first use, from the same per-channel values)."""
    if isinstance(t, ChannelState):
        v_chan, desc, _ = t._cf_state
        with torch._C.DisableTorchFunctionSubclass():
            base = torch.Tensor.view(t, *shape)
        v = ChannelState(base, v_chan, desc, uniform=t.__dict__.get("_cf_uniform", False))
        v._cf_sticky = t.__dict__.get("_cf_sticky", False)
        return v
    return t.view(*shape)


def _tensors_in(args, kwargs):
    stack = list(args) + list(kwargs.values())
    while stack:
        a = stack.pop()
        if isinstance(a, torch.Tensor):
            yield a
        elif isinstance(a, (list, tuple)):
            stack.extend(a)
        elif isinstance(a, dict):
            stack.extend(a.values())


def lazy_output(shape, nhwc: torch.Tensor, device) -> NHWCSpikes:
    """Uninitialised fp32 storage of `shape` that fills itself from `nhwc`."""
    return NHWCSpikes(torch.empty(shape, dtype=torch.float32, device=device), nhwc)


def lazy_tokens(shape, copy: torch.Tensor, device) -> NHWCSpikes:
    """Token-major fp32 [..., N, C] output whose values live in its fp16
    copy (any shape with rows * cp elements, e.g. a conv's NHWC
    [T*B, H, W, cp] with H*W = N); filled from the copy on first outside read."""
    return NHWCSpikes(torch.empty(shape, dtype=torch.float32, device=device), copy, tokens=True)


def token_view(B: int, N: int):
    """(nimg, H, W): how a token layer's launch views the B * N tokens of a
    step as images.  8 x 8 images of 64 consecutive tokens when 64 divides
    B * N (the halo kernel's 8 x 8 pixel tile, no idle rows); else each
    image's N tokens on a square grid (N a square of at least 16) or a
    column (N, 1)."""
    if (B * N) % 64 == 0:
        return B * N // 64, 8, 8
    r = int(round(N ** 0.5))
    return (B, r, r) if (r * r == N and r >= 4) else (B, N, 1)


def pixel_tokens(x: torch.Tensor) -> Optional[torch.Tensor]:
    """A fused layer's output x [T, B, C, 1, 1] whose values are still only
    in its fp16 NHWC copy, as token-major [T, B, C] over the same copy (for
    one-pixel images the NHWC and NCHW orders agree): the flatten of a
    network head that a fused linear layer reads without a pack.  Carries
    x's count block and copy descriptor.  None for any other x."""
    if (not isinstance(x, NHWCSpikes) or not x.__dict__.get("_cf_pending", False)
            or x.__dict__.get("_cf_tokens", False) or x.dim() != 5
            or x.shape[3] != 1 or x.shape[4] != 1):
        return None
    nhwc, ver = x._cf_nhwc
    if ver != _ver(x):
        return None
    T, B, C = x.shape[:3]
    with torch._C.DisableTorchFunctionSubclass():
        base = torch.Tensor.view(x, T, B, C)
    y = NHWCSpikes(base, nhwc, tokens=True)
    for a in ("_cf_count", "_cf_desc"):
        if a in x.__dict__:
            setattr(y, a, x.__dict__[a])
    return y


def token_membrane(v: torch.Tensor, B: int, N: int) -> torch.Tensor:
    """A token layer's state [nimg, C, H * W] (per view image) as [B, N, C]."""
    return v.transpose(1, 2).reshape(B, N, v.shape[1])


def token_shadow(x: torch.Tensor, cp: int, resolve: bool = True) -> Optional[torch.Tensor]:
    """The current fp16 copy of a token-major x [..., N, C] as [rows, cp]
    (rows = x.numel() / C), or None; resolve as shadow_of."""
    sh = getattr(x, "_cf_nhwc", None)
    if sh is None:
        return None
    t, ver = sh
    rows = x.numel() // x.shape[-1]
    if (ver != _ver(x) or t.device != x.device or t.shape[-1] != cp
            or t.numel() != rows * cp):
        return None
    if t.dtype == torch.uint8:
        return _widen(x, t).reshape(rows, cp)
    if resolve:
        _resolve(x, t)
    return t.reshape(rows, cp)


def pack_tokens(x: torch.Tensor, cp: int, nnz: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None):
    """Token-major fp32 x [..., C] -> its fp16 copy [rows, cp] (channels
    >= C zero); count_nonzero(x) published into nnz when given."""
    require_gpu_tensor(x, "x")
    _require_block(nnz)
    x = x.contiguous()
    C = x.shape[-1]
    rows = x.numel() // C
    xp = out if out is not None else torch.empty((rows, cp), dtype=torch.float16, device=x.device)
    ev = _t0()
    check(_hip.lib().cf_pack_tokens(ptr(x), rows, C, cp, ptr(xp), ptr(nnz), ptr(status),
                                    _hip.stream(x.device)), "cf_pack_tokens")
    _t1("pack_tokens", ev, nbytes=4 * rows * C + 2 * rows * cp)
    return xp


def attach_shadow(out: torch.Tensor, nhwc: torch.Tensor) -> None:
    """Record the fp16 NHWC copy a fused conv wrote next to its fp32 output,
    tagged with the output's version counter (any in-place change of `out`
    invalidates it)."""
    out._cf_nhwc = (nhwc, _ver(out))


def shadow_of(x: torch.Tensor, shape, resolve: bool = True,
              u8_ok: bool = False) -> Optional[torch.Tensor]:
    """The current NHWC copy of x with the given shape, or None.  With
    resolve (the default) a copy its producer did not write (output
    descriptor: all zero, or an alias) is filled first; a caller that reads
    the copy through its descriptor (desc_of) passes resolve=False.  A byte
    copy is returned as it is to a caller that reads byte copies (u8_ok),
    else widened to a new fp16 copy (resolved first: x then has no
    descriptor)."""
    sh = getattr(x, "_cf_nhwc", None)
    if sh is None:
        return None
    t, ver = sh
    if ver != _ver(x) or tuple(t.shape) != tuple(shape) or t.device != x.device:
        return None
    if t.dtype == torch.uint8 and not u8_ok:
        return _widen(x, t)
    if resolve:
        _resolve(x, t)
    return t


# Output descriptors (16 bytes each: uint32 copy state, uint32 state kind,
# alias pointer) let a StaticZero launch leave its outputs unwritten; off
# for comparisons against the always-writing path.
COPY_ELISION = True

# Launch plans cached per input signature for the common fused-conv and
# token-layer launches (ConvLIFRunner._dense_repeat, ConvLIFRunner.
# _tokens_repeat, halo_pair_repeat); off for comparisons against the general
# path.
REPEAT_PLANS = True


def new_out_desc(device) -> torch.Tensor:
    """One output's descriptor (16 bytes), written by the launch that
    receives it before any reader runs."""
    return torch.empty(2, dtype=torch.int64, device=device)


_WRITTEN_DESC = {}


def written_desc(device) -> torch.Tensor:
    """A read-only descriptor that says "written", for a fused layer's copy
    whose producer keeps no descriptor (an identity copy may then be
    aliased: it holds spike counts)."""
    d = _WRITTEN_DESC.get(device)
    if d is None:
        d = _WRITTEN_DESC[device] = torch.zeros(2, dtype=torch.int64, device=device)
    return d


def attach_desc(out: torch.Tensor, desc: torch.Tensor, keep=()) -> None:
    """Record the output descriptor of out's copy; keep: the copies its
    values may alias (held alive with it)."""
    out._cf_desc = (desc, _ver(out), tuple(keep))


def desc_of(x: torch.Tensor) -> Optional[torch.Tensor]:
    """The descriptor of x's current copy (None: the copy is written)."""
    d = getattr(x, "_cf_desc", None)
    if d is None or d[1] != _ver(x):
        return None
    return d[0]


def keep_of(x: torch.Tensor) -> tuple:
    """The copies x's copy may alias (see attach_desc)."""
    d = getattr(x, "_cf_desc", None)
    return () if d is None else d[2]


def _resolve(x: torch.Tensor, t: torch.Tensor) -> None:
    """Make x's copy t hold its values if its producer left it unwritten."""
    d = x.__dict__.get("_cf_desc")
    if d is None:
        return
    x._cf_desc = None
    check(_hip.lib().cf_resolve_copy(t.data_ptr(), t.numel() * t.element_size(),
                                     d[0].data_ptr(), _hip.stream(t.device)), "cf_resolve_copy")


COUNT_BLOCK_WORDS = 272  # CF_COUNT_BLOCK_WORDS of the C-ABI


def count_block(device) -> torch.Tensor:
    """A count block (COUNT_BLOCK_WORDS int64): [0] the accumulator of a
    producer pass, zero between passes; [1] the count the last completed
    pass published; then per-group accumulators that spread the pass's
    atomics.  The producer kernels (cf_pack_input, cf_scan_nhwc, a fused conv
    writing its output) clear the accumulators themselves, so a block is
    zeroed once, here."""
    return torch.zeros(COUNT_BLOCK_WORDS, dtype=torch.int64, device=device)


def _require_block(blk: Optional[torch.Tensor]) -> None:
    if blk is not None and (blk.dtype != torch.int64 or blk.numel() < COUNT_BLOCK_WORDS
                            or not blk.is_contiguous() or not blk.is_cuda):
        raise ValueError(f"a count block is a contiguous int64 GPU tensor of "
                         f"{COUNT_BLOCK_WORDS} elements (count_block)")


def attach_count(out: torch.Tensor, blk: torch.Tensor, gen_cell: list) -> None:
    """Record the count block a fused conv published for its output (the
    number of its workgroups that wrote a nonzero value: zero iff the output
    is all zero).  gen_cell is the producing layer's call counter: a later
    call of the same layer republishes the block, which then no longer
    describes this output."""
    out._cf_count = (blk, gen_cell, gen_cell[0], _ver(out))


def count_of(x: torch.Tensor) -> Optional[torch.Tensor]:
    """The count block describing x's current values, or None."""
    c = getattr(x, "_cf_count", None)
    if c is None:
        return None
    blk, cell, gen, ver = c
    if ver != _ver(x) or cell[0] != gen or blk.device != x.device:
        return None
    return blk


def pack_input(x4: torch.Tensor, *, cp: Optional[int] = None, want_xp=True, group_size=0,
               threshold=1e-6, nnz: Optional[torch.Tensor] = None, act_out=None, xp_out=None,
               status: Optional[torch.Tensor] = None):
    """x4 [NB, C, H, W] fp32 -> (xp fp16 [NB, H, W, Cp] | None, act int32 [NB, H, W] | None);
    count_nonzero(x4) is published in the count block nnz (count_block) when given."""
    require_gpu_tensor(x4, "x")
    _require_block(nnz)
    NB, C, H, W = x4.shape
    cp = pad32(C) if cp is None else cp
    xp = None
    if want_xp:
        xp = xp_out if xp_out is not None else torch.empty((NB, H, W, cp), dtype=torch.float16,
                                                          device=x4.device)
        if xp.shape != (NB, H, W, cp) or xp.dtype != torch.float16:
            raise ValueError("xp_out has the wrong shape/dtype")
    act = None
    if group_size > 0:
        act = act_out if act_out is not None else torch.empty((NB, H, W), dtype=torch.int32,
                                                              device=x4.device)
    ev = _t0()
    rc = _hip.lib().cf_pack_input(ptr(x4), NB, C, H, W, cp, ptr(xp), ptr(act), int(group_size),
                                  float(threshold), ptr(nnz), ptr(status), _hip.stream(x4.device))
    check(rc, "cf_pack_input")
    _t1("pack_input", ev, nbytes=4 * NB * C * H * W + (2 * NB * H * W * cp if xp is not None else 0)
        + (4 * NB * H * W if act is not None else 0))
    return xp, act


def scan_nhwc(xp: torch.Tensor, C: int, *, group_size: int, threshold=1e-6,
              nnz: Optional[torch.Tensor] = None, act_out=None):
    """xp fp16 NHWC [NB, H, W, Cp] (a fused conv's output copy) -> act int32
    [NB, H, W] with cf_pack_input's bits; the nonzero count is published in
    the count block nnz when given."""
    require_gpu_tensor(xp, "xp", dtype=torch.float16)
    _require_block(nnz)
    NB, H, W, cp = xp.shape
    act = act_out if act_out is not None else torch.empty((NB, H, W), dtype=torch.int32,
                                                          device=xp.device)
    ev = _t0()
    rc = _hip.lib().cf_scan_nhwc(ptr(xp), NB, H, W, cp, C, ptr(act), int(group_size),
                                 float(threshold), ptr(nnz), _hip.stream(xp.device))
    check(rc, "cf_scan_nhwc")
    _t1("scan_nhwc", ev, nbytes=2 * NB * H * W * cp + 4 * NB * H * W)
    return act


def global_avgpool_nhwc(xp: torch.Tensor, C: int, out: Optional[torch.Tensor] = None,
                        desc: Optional[torch.Tensor] = None):
    """xp NHWC copy [NB, H, W, cp] (fp16 or one byte per channel) -> fp32
    [NB, C]: the mean over H, W (AdaptiveAvgPool2d((1, 1)) of the fp32
    tensor the copy stands for); desc: the copy's output descriptor when its
    producer kept one."""
    u8 = xp.dtype == torch.uint8
    require_gpu_tensor(xp, "xp", dtype=torch.uint8 if u8 else torch.float16)
    NB, H, W, cp = xp.shape
    y = out if out is not None else torch.empty((NB, C), dtype=torch.float32, device=xp.device)
    ev = _t0()
    fn = _hip.lib().cf_global_avgpool_nhwc_u8 if u8 else _hip.lib().cf_global_avgpool_nhwc
    check(fn(ptr(xp), ptr(desc), ptr(y), NB, H * W, C, cp, _hip.stream(xp.device)),
          "cf_global_avgpool_nhwc")
    _t1("global_avgpool_nhwc", ev, nbytes=xp.element_size() * NB * H * W * C + 4 * NB * C)
    return y


def linear_tokens(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None
                  ) -> Optional[torch.Tensor]:
    """x @ weight.T + bias for a token-major fused output x [..., K] read from
    its fp16 copy through its descriptor (cf_linear_tokens), fp32 [..., O];
    None when x carries no current copy (the caller then runs F.linear)."""
    K = x.shape[-1]
    O = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K or O > 4096:
        return None
    copy = token_shadow(x, pad32(K), resolve=False)
    if copy is None:
        return None
    require_gpu_tensor(weight, "weight")
    if bias is not None:
        require_gpu_tensor(bias, "bias")
    rows = copy.shape[0]
    out = torch.empty(tuple(x.shape[:-1]) + (O,), dtype=torch.float32, device=x.device)
    ev = _t0()
    check(_hip.lib().cf_linear_tokens(ptr(copy), ptr(desc_of(x)), ptr(weight), ptr(bias),
                                      ptr(out), rows, K, copy.shape[1], O,
                                      _hip.stream(x.device)), "cf_linear_tokens")
    _t1("linear_tokens_head", ev, nbytes=2 * rows * K + 4 * O * K + 4 * rows * O)
    return out


def maxpool_nhwc(x: torch.Tensor, kernel_size: int, stride: int, padding: int,
                 gen_cell: Optional[list] = None, nz_out: Optional[torch.Tensor] = None):
    """MaxPool2d of a fused layer's output x [T, B, C, H, W] read from its
    fp16 NHWC copy (through its descriptor when the producer kept one);
    returns a lazy output carrying the pooled copy (and, with nz_out and
    gen_cell, its count block), or None when x has no copy.  The pool of an
    elided all-zero copy is itself recorded as all zero, not written."""
    T, B, C, H, W = x.shape
    xp = shadow_of(x, (T * B, H, W, pad32(C)), resolve=False)
    if xp is None:
        return None
    _require_block(nz_out)
    in_desc = desc_of(x)
    Ho = (H + 2 * padding - kernel_size) // stride + 1
    Wo = (W + 2 * padding - kernel_size) // stride + 1
    cp = xp.shape[-1]
    out = torch.empty((T * B, Ho, Wo, cp), dtype=torch.float16, device=x.device)
    out_desc = new_out_desc(x.device) if (COPY_ELISION and in_desc is not None) else None
    ev = _t0()
    check(_hip.lib().cf_maxpool_nhwc(ptr(xp), ptr(in_desc), ptr(out), ptr(out_desc), T * B, H,
                                     W, cp, kernel_size, stride, padding, ptr(nz_out),
                                     _hip.stream(x.device)),
          "cf_maxpool_nhwc")
    _t1("maxpool_nhwc", ev, nbytes=2 * T * B * (H * W + Ho * Wo) * cp)
    y = lazy_output((T, B, C, Ho, Wo), out, x.device)
    if out_desc is not None:
        attach_desc(y, out_desc)   # all zero or written: it aliases nothing
    if nz_out is not None and gen_cell is not None:
        gen_cell[0] += 1
        attach_count(y, nz_out, gen_cell)
    return y


# The single-pass attention kernel's shapes (one workgroup per image and
# head holds every token): head dim 32, at most 256 tokens.  Other shapes
# (head dim 64, longer token rows) take the two-pass kernels.
ATTN_ONE_PASS_DIM = 32
ATTN_ONE_PASS_TOKENS = 256


def attention_covers(head_dim: int, N: int) -> bool:
    """Whether the hand-written attention kernels cover the shape."""
    return head_dim in (32, 64) and N < 65536 and head_dim * N < 2 ** 24


def spike_attention_lif(qkv: torch.Tensor, T: int, B: int, N: int, heads: int, offsets,
                        scale: float, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True,
                        v_in: Optional[torch.Tensor] = None, want_v_out=True,
                        nz_out: Optional[torch.Tensor] = None, gen_cell: Optional[list] = None,
                        nnz: Optional[torch.Tensor] = None, head_dim: int = 32,
                        two_pass: Optional[bool] = None):
    """Spikformer's SSA core on the fp16 token copy qkv [T*B*N, pitch] that
    holds Q, K, V at channel offsets (qoff, koff, voff) (head h at
    off + head_dim h ..): LIF_T(((Q K^T) V) * scale) per head, evaluated as
    Q (K^T V) on the matrix cores; nnz: the copy's count block (a zero count
    skips the products: z = 0).  Head dim 32 with at most 256 tokens runs the
    single-pass kernel, other shapes (head dim 64, longer rows) the two-pass
    one (two_pass forces the choice; both give the same values).  Returns
    (TokenSpikes [T, B, N, heads*head_dim], carrying the count block nz_out
    when it and gen_cell are given, so the next fused linear routes on it;
    v_out [B, N, heads*head_dim] or None)."""
    require_gpu_tensor(qkv, "qkv", dtype=torch.float16)
    _require_block(nz_out)
    _require_block(nnz)
    if not attention_covers(head_dim, N):
        raise ValueError(f"no attention kernel for head dim {head_dim} and {N} tokens")
    if two_pass is None:
        two_pass = head_dim != ATTN_ONE_PASS_DIM or N > ATTN_ONE_PASS_TOKENS
    elif not two_pass and (head_dim != ATTN_ONE_PASS_DIM or N > ATTN_ONE_PASS_TOKENS):
        raise ValueError("the single-pass attention kernel needs head dim 32, N <= 256")
    dev = qkv.device
    pitch = qkv.shape[-1]
    C = heads * head_dim
    cp = pad32(C)
    if qkv.numel() != T * B * N * pitch:
        raise ValueError("qkv does not hold T * B * N tokens")
    if v_in is not None:
        require_gpu_tensor(v_in, "v_in")
        if v_in.numel() != B * N * C:
            raise ValueError("v_in has the wrong size")
    copy = torch.empty((T * B * N, cp), dtype=torch.float16, device=dev)
    v_out = torch.empty((B, N, C), dtype=torch.float32, device=dev) if want_v_out else None
    qoff, koff, voff = (int(o) for o in offsets)
    lif = _lif_args(tau, v_threshold, v_reset, decay_input)
    # on the zero route from the initial state the output may be left
    # unwritten (all zero) and the state uniform: the LIF's response to z = 0
    desc = v_uniform = None
    zero_info = 0
    if COPY_ELISION and nnz is not None and v_in is None:
        r = zero_drive_response(dev, T, lif)
        if r is not None and r[1]:
            desc = new_out_desc(dev)
            v_uniform = r[0] if v_out is not None else None
            zero_info = 1 | (2 if v_uniform is not None else 0)
    ev = _t0()
    if two_pass:
        kv_ws = torch.empty((T * B * heads, head_dim, head_dim), dtype=torch.float32, device=dev)
        check(_hip.lib().cf_spike_attention_kv_lif(
            ptr(qkv), ptr(qkv), ptr(qkv), qoff, koff, voff, pitch, ptr(copy), cp, ptr(v_in),
            ptr(v_out), ptr(kv_ws), ptr(nnz), ptr(nz_out), ptr(desc), zero_info, T, B, N, heads,
            head_dim, float(scale), *lif, _hip.stream(dev)), "cf_spike_attention_kv_lif")
    else:
        check(_hip.lib().cf_spike_attention_lif(
            ptr(qkv), ptr(qkv), ptr(qkv), qoff, koff, voff, pitch, ptr(copy), cp, ptr(v_in),
            ptr(v_out), ptr(nnz), ptr(nz_out), ptr(desc), zero_info, T, B, N, heads, 32,
            float(scale), *lif, _hip.stream(dev)), "cf_spike_attention_lif")
    _t1("spike_attention", ev, flops=4 * T * B * heads * N * head_dim * head_dim,
        nbytes=2 * T * B * N * 3 * C + 2 * T * B * N * cp,
        route=None if nnz is None else _RouteProbe(
            nnz, [(desc, 2 * T * B * N * cp, 4 * B * N * C if v_out is not None else 0)]))
    out = lazy_tokens((T, B, N, C), copy, dev)
    if desc is not None:
        attach_desc(out, desc)
    if nz_out is not None and gen_cell is not None:
        gen_cell[0] += 1
        attach_count(out, nz_out, gen_cell)
    if v_uniform is not None:
        v_out = ChannelState(v_out, v_uniform, desc, uniform=True)
    return out, v_out


_ZERO_DRIVE = {}


def zero_drive_response(device, T: int, lif) -> Optional[tuple]:
    """(v_final [1] fp32, silent) of a LIF with parameters lif (the C-ABI's
    tau, v_th, v_reset, hard, decay_input) driven by z = 0 for T steps from
    its initial state (cf_bias_response of a zero affine), computed once per
    device, T and parameters; None while a graph is being captured and the
    value is not yet known."""
    key = (str(device), int(T), tuple(lif))
    r = _ZERO_DRIVE.get(key)
    if r is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        z = torch.zeros(1, dtype=torch.float32, device=device)
        v = torch.empty(1, dtype=torch.float32, device=device)
        f = torch.empty(1, dtype=torch.int32, device=device)
        check(_hip.lib().cf_bias_response(ptr(z), ptr(z), 1, T, 0, *lif, ptr(v), ptr(f),
                                          _hip.stream(device)), "cf_bias_response")
        r = _ZERO_DRIVE[key] = (v, not bool(f.item()))
    return r


def prescan_tiles(act: torch.Tensor, H: int, W: int, H_out: int, W_out: int, kernel_size: int,
                  stride: int, padding: int, block_h: int, block_w: int, num_groups: int,
                  ag_mask_out=None, tile_class_out=None):
    NB = act.shape[0]
    GH, GW = -(-H_out // block_h), -(-W_out // block_w)
    n = NB * GH * GW
    ag = ag_mask_out if ag_mask_out is not None else torch.empty(n, dtype=torch.int32,
                                                                 device=act.device)
    tc = tile_class_out if tile_class_out is not None else torch.empty(n, dtype=torch.int32,
                                                                      device=act.device)
    if ag.numel() < n or tc.numel() < n:
        raise ValueError("prescan output buffers are too small")
    ev = _t0()
    rc = _hip.lib().cf_prescan_tiles(ptr(act), NB, H, W, H_out, W_out, kernel_size, stride,
                                     padding, block_h, block_w, num_groups, ptr(ag), ptr(tc),
                                     _hip.stream(act.device))
    check(rc, "cf_prescan_tiles")
    _t1("prescan_tiles", ev, nbytes=4 * NB * H * W + 8 * n)
    return tc[:n], ag[:n]


def compact_tiles(ag_mask: torch.Tensor, T: int, ntiles: int, num_groups: int = 32,
                  order_out=None, *, macs_per_tile: float = 0.0, tau: float = -1.0,
                  r_min: float = 0.0) -> torch.Tensor:
    """Device-side active-tile order (cf_compact_tiles) of tile masks
    [T][ntiles]: int32 [1 + ntiles], the number of tiles active at some step
    (-1 when tau >= 0 and the dispatch score R * macs_per_tile rejects
    SparseFlow), then the tile indices, active ones first."""
    if ag_mask.numel() < T * ntiles:
        raise ValueError("tile masks are smaller than T * ntiles")
    order = order_out if order_out is not None else torch.empty(
        ntiles + 1, dtype=torch.int32, device=ag_mask.device)
    if order.numel() < ntiles + 1:
        raise ValueError("tile order buffer is too small")
    ev = _t0()
    check(_hip.lib().cf_compact_tiles(ptr(ag_mask), T, ntiles, int(num_groups),
                                      float(macs_per_tile), float(tau), float(r_min), ptr(order),
                                      _hip.stream(ag_mask.device)), "cf_compact_tiles")
    _t1("compact_tiles", ev, nbytes=8 * T * ntiles + 4 * ntiles)
    return order[:ntiles + 1]


def zero_counter(c: torch.Tensor) -> None:
    check(_hip.lib().cf_zero_counter(ptr(c), _hip.stream(c.device)), "cf_zero_counter")


def route_from_nnz(nnz: torch.Tensor, numel: int, sparse_threshold: float,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Route word (int32 device tensor) from the count block nnz."""
    _require_block(nnz)
    r = out if out is not None else torch.empty(1, dtype=torch.int32, device=nnz.device)
    check(_hip.lib().cf_route_from_nnz(ptr(nnz), int(numel), float(sparse_threshold), ptr(r),
                                       _hip.stream(nnz.device)), "cf_route_from_nnz")
    return r


# ---------------------------------------------------------------------------
# Conv -> BN -> LIF
# ---------------------------------------------------------------------------

def _copy_record(x):
    """(record dict, copy, version, metadata) of x's current NHWC copy -- its
    producer's copy at x's present version, as shadow_of accepts it -- or
    None: the launch plans' reading of x."""
    d = x.__dict__
    sh = d.get("_cf_nhwc")
    if sh is None:
        return None
    xp, ver = sh
    if ver != d.get("_cf_base", x)._version:
        return None
    meta = d.get("_cf_meta") if d.get("_cf_pending", False) else None
    return d, xp, ver, (_meta_of(x) if meta is None else meta)


def _desc_count(d, ver):
    """(descriptor, count block) of a copy record at version ver, as desc_of
    and count_of return them (None: absent or stale)."""
    dd = d.get("_cf_desc")
    c = d.get("_cf_count")
    return ((dd[0] if dd is not None and dd[1] == ver else None),
            (c[0] if c is not None and c[3] == ver and c[1][0] == c[2] else None))


def _identity_args(idd, ic, iver, dev):
    """The general path's arguments for a spike identity with current copy
    ic (record idd at version iver): the pointers of the copy, of its
    descriptor (written_desc when it keeps none) and of its count block (0
    when absent), and the copies an output aliasing it keeps alive."""
    idesc, inz = _desc_count(idd, iver)
    if idesc is None:
        idesc = written_desc(dev)
    dd = idd.get("_cf_desc")
    return (ic.data_ptr(), idesc.data_ptr(), 0 if inz is None else inz.data_ptr(),
            (ic,) + (() if dd is None else dd[2]))


def _conv_args_block(p):
    """The cf_conv_mfma_args block of plan p with its static fields filled
    (weights, sizes, epilogue, LIF parameters from p.tail, as the positional
    call passes them); a launch fills the per-call ones.  Kept on the plan
    with its address."""
    a = _hip.ConvMfmaArgs()
    a.w_packed, a.alpha, a.beta = p.weights
    a.v_in = a.out = a.identity = a.ag_mask = a.tile_order = None
    a.cp_out = a.cp_id = p.cp_out
    a.identity_mode = ID_ADD_SPIKE
    a.nz_out = p.nz_ptr
    a.numel = p.numel
    (a.T, a.B, a.Cp, a.Cout, a.Coutp, a.H, a.W, a.Ho, a.Wo, a.KH, a.KW, a.stride, a.pad,
     a.x_img_tstride, a.tile_h, a.tile_w, a.group_size, a.epilogue, a.tau, a.v_th, a.v_reset,
     a.hard_reset, a.decay_input) = p.tail
    p.args = a
    p.args_addr = ctypes.addressof(a)


class _DensePlan:
    """What run_mfma's dense route decides from an input signature alone
    (ConvLIFRunner._dense_plan): the copy format, the output shapes, the
    static launch arguments and the layer's bias response."""
    __slots__ = ("u8", "need_v", "vshape", "vmeta", "cshape", "cdtype", "oshape", "ometa",
                 "nz_out", "nz_ptr", "weights", "numel", "T", "cp_out", "bias", "pool", "fn",
                 "tail", "args", "args_addr")


class ConvLIFRunner:
    """Device state + launches for one fused Conv -> (BN) -> LIF layer.

    weight [Cout, Cin, KH, KW] fp32; bn_scale/bn_shift [Cout] (folded eval
    BN, optional); bias [Cout] (optional).  Call `refresh()` after changing
    any of them.
    """

    def __init__(self, weight, bn_scale, bn_shift, bias, stride, padding, tau, v_threshold,
                 v_reset, decay_input):
        self.weight = weight
        self.bn_scale = bn_scale
        self.bn_shift = bn_shift
        self.bias = bias
        self.stride = int(stride)
        self.padding = int(padding)
        self.lif = _lif_args(tau, v_threshold, v_reset, decay_input)
        self.Cout, self.Cin, self.KH, self.KW = (int(s) for s in weight.shape)
        self.Cp = pad32(self.Cin)
        self.Coutp = ((self.Cout + 63) // 64) * 64
        self._packed_key = None
        self.w_packed = self.alpha = self.beta = None
        self.alpha_direct = self.beta_direct = None
        self._ws = {}
        self._plans = {}  # input signature -> _DensePlan (or False: not covered)
        self._gen = [0]  # calls that published the output count block

    def refresh(self):
        self._packed_key = None
        self._stem_key = None

    def _param_key(self, device):
        return (device, self.weight.data_ptr(), getattr(self.weight, "_version", 0),
                None if self.bn_scale is None else (self.bn_scale.data_ptr(),
                                                    self.bn_scale._version),
                None if self.bn_shift is None else (self.bn_shift.data_ptr(),
                                                    self.bn_shift._version),
                None if self.bias is None else (self.bias.data_ptr(), self.bias._version))

    def _ensure_packed(self, device):
        key = self._param_key(device)
        if key == self._packed_key:
            return
        w = self.weight.detach().float().contiguous()
        bs = None if self.bn_scale is None else self.bn_scale.detach().float().contiguous()
        bh = None if self.bn_shift is None else self.bn_shift.detach().float().contiguous()
        bi = None if self.bias is None else self.bias.detach().float().contiguous()
        for name, t in (("weight", w), ("bn_scale", bs), ("bn_shift", bh), ("bias", bi)):
            if t is not None:
                require_gpu_tensor(t, name)
        st = _hip.stream(device)
        self.w_packed = torch.empty((2, self.Coutp, self.KH * self.KW, self.Cp),
                                    dtype=torch.float16, device=device)
        self.alpha = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        self.beta = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        check(_hip.lib().cf_pack_conv_weights(ptr(w), self.Cout, self.Cin, self.KH, self.KW,
                                              self.Coutp, self.Cp, ptr(bs), ptr(bh), ptr(bi),
                                              ptr(self.w_packed), ptr(self.alpha),
                                              ptr(self.beta), st), "cf_pack_conv_weights")
        self.alpha_direct = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        self.beta_direct = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        check(_hip.lib().cf_pack_conv_weights(ptr(w), self.Cout, self.Cin, self.KH, self.KW,
                                              self.Coutp, self.Cp, ptr(bs), ptr(bh), ptr(bi),
                                              None, ptr(self.alpha_direct),
                                              ptr(self.beta_direct), st), "cf_pack_conv_weights")
        self._w_f32 = w
        self._wt_f32 = w.reshape(self.Cout, -1).t().contiguous()   # [Cin*KH*KW][Cout]
        self._bias_resp = {}
        self._plans = {}
        self._packed_key = key

    def bias_response(self, device, T: int, pool: bool = False):
        """(v_final [Cout] fp32, silent) of the layer's bias drive alone over
        T steps (cf_bias_response; pool: the pooled epilogue's drive): each
        channel's final potential on the StaticZero route, and whether no
        channel fires there.  Computed once per (T, pool) (a host read); None
        while a graph is being captured and the value is not yet known."""
        key = (T, bool(pool))
        r = self._bias_resp.get(key)
        if r is None:
            if torch.cuda.is_current_stream_capturing():
                return None
            v = torch.empty(self.Cout, dtype=torch.float32, device=device)
            f = torch.empty(self.Cout, dtype=torch.int32, device=device)
            check(_hip.lib().cf_bias_response(ptr(self.alpha), ptr(self.beta), self.Cout, T,
                                              int(bool(pool)), *self.lif, ptr(v), ptr(f),
                                              _hip.stream(device)),
                  "cf_bias_response")
            r = self._bias_resp[key] = (v, not bool(f.any().item()))
        return r

    def zero_route_info(self, device, T: int, desc, v_out, v_in, pool: bool = False):
        """(bias_info, v_final or None) for a launch with output descriptor
        desc: the bias_info bits of cf_conv_mfma and the per-channel
        potentials that stand for v_out when the launch leaves it unwritten
        (pool: a launch with the pooled epilogue)."""
        if desc is None:
            return 0, None
        r = self.bias_response(device, T, pool)
        if r is None:
            return 0, None
        v_final, silent = r
        hold = v_out is not None and v_in is None
        return (1 if silent else 0) | (2 if hold else 0), (v_final if hold else None)

    def halo_lean_ok(self, T, B, Ho, Wo) -> bool:
        """Whether a launch of this layer at output size Ho x Wo runs the
        halo kernel (3x3, or 1x1 over maps of at least 4x4; stride 1 or 2),
        which the byte-copy path needs."""
        k_ok = ((self.KH, self.KW) == (3, 3)
                or ((self.KH, self.KW) == (1, 1) and Ho >= 4 and Wo >= 4))
        return (k_ok and self.stride in (1, 2) and self.padding <= 2
                and T * B * self.Cout * Ho * Wo <= 2 ** 31 - 1)

    def out_hw(self, H, W):
        return ((H + 2 * self.padding - self.KH) // self.stride + 1,
                (W + 2 * self.padding - self.KW) // self.stride + 1)

    def workspace(self, key, shape, dtype, device):
        t = self._ws.get(key)
        if t is None or t.shape != torch.Size(shape) or t.dtype != dtype or t.device != device:
            t = torch.empty(shape, dtype=dtype, device=device)
            self._ws[key] = t
        return t

    def counter(self, device):
        """Count block of the layer's input when the layer counts it itself
        (cf_pack_input / cf_scan_nhwc publish into it; see count_block)."""
        t = self._ws.get("nnz")
        if t is None or t.device != device:
            t = count_block(device)
            self._ws["nnz"] = t
        return t

    def out_counter(self, device):
        """Count block the conv publishes for its output (workgroups that wrote
        a nonzero value), read by the next fused layer to take the StaticZero
        route without a counting pass."""
        t = self._ws.get("nz_out")
        if t is None or t.device != device:
            t = count_block(device)
            self._ws["nz_out"] = t
        return t

    def _dense_plan(self, key, x, xp, identity, ish, xshape, dev, epilogue=EPI_LIF):
        """The _DensePlan of one input signature (see _dense_repeat), made
        with the checks and choices of run_mfma's general path; False when
        that path would do anything else than one dense launch on the
        copies as they are (repack, widen a byte copy, an fp32 identity, an
        error)."""
        if len(xshape) != 5:
            return False
        T, B, C, H, W = xshape
        Ho, Wo = self.out_hw(H, W)
        cp_out = pad32(self.Cout)
        pool = epilogue == EPI_POOL
        meta = key[0]     # x: fp32, contiguous, on the GPU (require_gpu_tensor)
        ok = (C == self.Cin and Ho >= 1 and Wo >= 1 and meta[1] == torch.float32 and meta[4]
              and dev.type == "cuda" and xp.device == dev
              and tuple(xp.shape) == (T * B, H, W, self.Cp)
              and xp.dtype in (torch.float16, torch.uint8))
        if pool:
            # the pooled epilogue's own conditions (run_mfma raises on them)
            ok = (ok and (self.KH, self.KW, self.stride) == (3, 3, 1) and self.Cout % 32 == 0
                  and Ho >= 2 and Wo >= 2 and identity is None)
        id_u8 = False
        if ok and identity is not None:
            ic = ish[0]
            ok = (tuple(key[3]) == (T, B, self.Cout, Ho, Wo)
                  and key[7] == (torch.float32, dev) and key[8]
                  and ic.device == dev and tuple(ic.shape) == (T * B, Ho, Wo, cp_out)
                  and ic.dtype in (torch.float16, torch.uint8))
            id_u8 = ok and ic.dtype == torch.uint8
        if not ok:
            return False
        u8 = (not pool and SPIKE_COPY == "u8" and self.Cout % 32 == 0
              and self.halo_lean_ok(T, B, Ho, Wo)
              and xp.dtype == torch.uint8 and (identity is None or id_u8))
        if (xp.dtype == torch.uint8 or id_u8) and not u8:
            return False      # the general path widens the byte copy first
        # output and state at the pooled size with the pooled epilogue
        Hs, Ws = (Ho // 2, Wo // 2) if pool else (Ho, Wo)
        p = _DensePlan()
        p.u8 = u8
        p.pool = pool
        p.need_v = key[6] or T > 2
        p.vshape = (B, self.Cout, Hs, Ws)
        p.vmeta = (torch.Size(p.vshape), torch.float32, dev, B * self.Cout * Hs * Ws, True)
        p.cshape = (T * B, Hs, Ws, cp_out)
        p.cdtype = torch.uint8 if u8 else torch.float16
        p.oshape = (T, B, self.Cout, Hs, Ws)
        p.ometa = (torch.Size(p.oshape), torch.float32, dev, T * B * self.Cout * Hs * Ws, True)
        p.nz_out = self.out_counter(dev)
        p.nz_ptr = p.nz_out.data_ptr()
        p.weights = (self.w_packed.data_ptr(), self.alpha.data_ptr(), self.beta.data_ptr())
        p.numel = T * B * C * H * W
        p.T = T
        p.cp_out = cp_out
        p.bias = None
        if u8:
            p.fn = _hip.lib().cf_conv_halo_u8
            p.tail = (T, B, self.Cp, self.Cout, self.Coutp, H, W, Ho, Wo, self.KH, self.stride,
                      self.padding, 0) + tuple(self.lif)
        else:
            p.fn = _hip.lib().cf_conv_mfma_args
            p.tail = (T, B, self.Cp, self.Cout, self.Coutp, H, W, Ho, Wo, self.KH, self.KW,
                      self.stride, self.padding, B, 0, 0, 0, epilogue) + tuple(self.lif)
            _conv_args_block(p)
        return p

    def _plan_outputs(self, p, dev, elide, keep=(), tokens=False):
        """The outputs of a launch from plan p, as _launch makes them: the
        state (when the plan keeps one), the copy and the lazy output with
        its count block; with elide (the input has a count block or a
        descriptor) the output descriptor and the StaticZero bits of the
        layer's bias response (keep: the copies an aliasing output holds).
        Returns (out, v_out, nhwc, desc, info, v_chan)."""
        v_out = torch.empty(p.vshape, dtype=torch.float32, device=dev) if p.need_v else None
        nhwc = torch.empty(p.cshape, dtype=p.cdtype, device=dev)
        base = torch.empty(p.oshape, dtype=torch.float32, device=dev)
        out = NHWCSpikes(base, nhwc, tokens=tokens, meta=p.ometa)
        gen = self._gen
        gen[0] += 1
        out._cf_count = (p.nz_out, gen, gen[0], base._version)
        desc = v_chan = None
        info = 0
        if elide:
            desc = torch.empty(2, dtype=torch.int64, device=dev)
            r = p.bias
            if r is None:
                r = p.bias = self.bias_response(dev, p.T, p.pool)
            if r is not None:
                info = (1 if r[1] else 0) | (2 if v_out is not None else 0)
                if v_out is not None:
                    v_chan = r[0]
            if info & 1:
                out._cf_desc = (desc, base._version, keep)
        return out, v_out, nhwc, desc, info, v_chan

    def _dense_repeat(self, x, identity, want_v_out, sparse_threshold, epilogue=EPI_LIF):
        """run_mfma's launch for its common case from a plan cached per input
        signature: a dense-route LIF (or pooled LIF) launch with no initial
        state whose input (and spike identity) carry a current NHWC copy,
        writing the output's copy, with no kernel timer.  The checks and
        choices that depend only on the signature (shapes, copy formats,
        device, whether the state is wanted, the copy settings) ran once when
        the plan was made; each call reads the copies' descriptors and count
        blocks, allocates the outputs and launches with the arguments the
        general path passes.  None when the case is not covered (run_mfma
        then takes its general path)."""
        rec = _copy_record(x)
        if rec is None:
            return None
        d, xp, ver, meta = rec
        xshape, dev = meta[0], meta[2]
        ish = None
        if identity is not None:
            irec = _copy_record(identity)
            if irec is None:
                return None
            idd, ic, iver, im = irec
            ish = (ic, iver)
            key = (meta, xp.shape, xp.dtype, im[0], ic.shape, ic.dtype, want_v_out, im[1:3],
                   im[4], SPIKE_COPY, COPY_ELISION, epilogue)
        else:
            key = (meta, xp.shape, xp.dtype, None, None, None, want_v_out, None, None,
                   SPIKE_COPY, COPY_ELISION, epilogue)
        self._ensure_packed(dev)
        p = self._plans.get(key)
        if p is None:
            p = self._plans[key] = self._dense_plan(key, x, xp, identity, ish, xshape, dev,
                                                    epilogue)
        if p is False:
            return None
        x_desc, nnz = _desc_count(d, ver)
        id_ptr = id_desc = id_nnz = 0
        id_keep = ()
        if identity is not None:
            id_ptr, id_desc, id_nnz, id_keep = _identity_args(idd, ic, iver, dev)
        out, v_out, nhwc, desc, info, v_chan = self._plan_outputs(
            p, dev, COPY_ELISION and (nnz is not None or x_desc is not None), id_keep)
        w, al, be = p.weights
        vo = v_out.data_ptr() if v_out is not None else None
        dp = desc.data_ptr() if desc is not None else None
        stream = _hip.stream(dev)
        if p.u8:
            rc = p.fn(xp.data_ptr(), w, al, be, None, vo, nhwc.data_ptr(), p.cp_out, id_ptr or None,
                      p.cp_out, None, None, nnz.data_ptr() if nnz is not None else None, p.nz_ptr,
                      x_desc.data_ptr() if x_desc is not None else None, id_desc or None, dp,
                      info, id_nnz or None, p.numel, float(sparse_threshold), *p.tail, stream)
            check(rc, "cf_conv_halo_u8")
        else:
            a = p.args
            a.x = xp.data_ptr()
            a.v_out = vo
            a.out_nhwc = nhwc.data_ptr()
            a.identity_nhwc = id_ptr or None
            a.nnz = nnz.data_ptr() if nnz is not None else None
            a.x_desc = x_desc.data_ptr() if x_desc is not None else None
            a.id_desc = id_desc or None
            a.out_desc = dp
            a.bias_info = info
            a.id_nnz = id_nnz or None
            a.sparse_threshold = float(sparse_threshold)
            a.stream = stream
            check(p.fn(p.args_addr), "cf_conv_mfma")
        self.last_nnz = nnz
        self.last_numel = p.numel
        self.last_tiles = None
        self.last_order = None
        if not want_v_out:
            return out, None
        return out, (ChannelState(v_out, v_chan, desc, meta=p.vmeta) if v_chan is not None
                     else v_out)

    def run_mfma(self, x: torch.Tensor, v_in=None, *, epilogue=EPI_LIF, want_v_out=True,
                 identity=None, identity_mode=ID_ADD_SPIKE, sparse=None, sparse_threshold=0.7,
                 static_zero=True, emit_nhwc=True):
        """x [T, B, Cin, H, W] fp32 (values exact in fp16).  sparse: None for
        the dense route only, or a dict with block_h, block_w, group_size
        (and optionally compact: True / "always" / False, the active-tile
        order) to run the prescan and SparseFlow chunk skipping.  If x carries a current
        fp16 NHWC copy (written by the producing fused conv) the pack pass is
        skipped: a SparseFlow layer scans the copy for its activity bits and
        count, a dense one takes the dense route; with emit_nhwc the output
        carries its own copy for the next layer, and the count block of its
        output (attach_count): a dense layer whose input carries one takes
        the StaticZero route on an all-zero input.  epilogue=EPI_POOL (a
        stride-1 3x3 conv): BN -> AvgPool2d(2, 2) -> LIF in the conv's
        epilogue; out is then the pooled spikes [T, B, Cout, Ho//2, Wo//2]
        (written as the fp16 NHWC copy) and v_out the pooled membrane state.
        Returns (out, v_out)."""
        if (sparse is None and (epilogue == EPI_LIF or epilogue == EPI_POOL) and emit_nhwc
                and static_zero and v_in is None and identity_mode == ID_ADD_SPIKE
                and _timer is None and REPEAT_PLANS):
            r = self._dense_repeat(x, identity, want_v_out, sparse_threshold, epilogue)
            if r is not None:
                return r
        require_gpu_tensor(x, "x")
        T, B, C, H, W = x.shape
        if C != self.Cin:
            raise ValueError(f"expected {self.Cin} input channels, got {C}")
        dev = x.device
        self._ensure_packed(dev)
        Ho, Wo = self.out_hw(H, W)
        if epilogue == EPI_POOL:
            if (self.KH, self.KW, self.stride) != (3, 3, 1) or self.Cout % 32 or Ho < 2 or Wo < 2:
                raise ValueError("the pooled epilogue needs a stride-1 3x3 conv, Cout a "
                                 "multiple of 32 and an output of at least 2x2")
            if identity is not None or not emit_nhwc:
                raise ValueError("the pooled epilogue writes the fp16 copy only, no identity")
            if sparse is not None and (sparse["block_h"], sparse["block_w"]) != (8, 8):
                raise ValueError("the pooled epilogue runs on 8x8 tiles")
        gs = sparse["group_size"] if sparse is not None else 0
        # One-byte copies: a dense-route launch of the halo kernel with the
        # lean LIF epilogue whose input (and SEW identity) arrive as byte
        # copies reads them as they are and writes a byte copy.
        u8 = False
        if (SPIKE_COPY == "u8" and sparse is None and epilogue == EPI_LIF and emit_nhwc
                and self.Cout % 32 == 0 and self.halo_lean_ok(T, B, Ho, Wo)):
            cand = shadow_of(x, (T * B, H, W, self.Cp), resolve=False, u8_ok=True)
            u8 = cand is not None and cand.dtype == torch.uint8
            if u8 and identity is not None:
                ic = (shadow_of(identity, (T * B, Ho, Wo, pad32(self.Cout)), resolve=False,
                                u8_ok=True) if identity_mode == ID_ADD_SPIKE else None)
                u8 = ic is not None and ic.dtype == torch.uint8
        # the dense route reads the copy through its descriptor; SparseFlow
        # scans it, so an unwritten copy is filled first
        xp = shadow_of(x, (T * B, H, W, self.Cp), resolve=sparse is not None, u8_ok=u8)
        x_desc = desc_of(x) if (xp is not None and sparse is None) else None
        nnz = act = None
        if xp is not None and sparse is not None:
            # SparseFlow on an input that carries its fp16 NHWC copy: the
            # activity bits and the nonzero count come from the copy
            nnz = self.counter(dev)
            act = scan_nhwc(xp, C, group_size=gs, nnz=nnz,
                            act_out=self.workspace("act", (T * B, H, W), torch.int32, dev))
        elif xp is not None:
            # dense route on an NHWC input: the producer's count block (if it
            # still describes x) enables StaticZero
            nnz = count_of(x) if static_zero else None
        else:
            st = status_word(dev)
            if static_zero or sparse is not None:
                nnz = self.counter(dev)
            xp = self.workspace("xp", (T * B, H, W, self.Cp), torch.float16, dev)
            act = (self.workspace("act", (T * B, H, W), torch.int32, dev) if sparse is not None
                   else None)
            pack_input(x.reshape(T * B, C, H, W), cp=self.Cp, group_size=gs, nnz=nnz,
                       act_out=act, xp_out=xp, status=st)
        ag = order = None
        th = tw = 0
        if sparse is not None:
            th, tw = sparse["block_h"], sparse["block_w"]
            GH, GW = -(-Ho // th), -(-Wo // tw)
            n = T * B * GH * GW
            ag_buf = self.workspace("ag", (n,), torch.int32, dev)
            tc_buf = self.workspace("tc", (n,), torch.int32, dev)
            G = -(-self.Cin // gs)
            prescan_tiles(act, H, W, Ho, Wo, self.KH, self.stride, self.padding, th, tw, G,
                          ag_buf, tc_buf)
            ag = ag_buf
            # compact: True orders the tiles when the grid does not fit one
            # dispatch wave (256 CUs x 3 workgroups of the 8x8 halo kernel;
            # within one wave the order cannot matter), "always" at any size.
            # egd: (tau, r_min) of the dispatch score, computed by the same
            # launch (so it runs whenever a score is asked for).
            cmode = sparse.get("compact", True)
            egd = sparse.get("egd")
            if (egd is not None or cmode == "always"
                    or (cmode and B * GH * GW * (self.Coutp // 64) > 768)):
                tau, r_min = egd if egd is not None else (-1.0, 0.0)
                macs_tile = Ho * Wo * self.Cout * self.Cin * self.KH * self.KW / (GH * GW)
                order = compact_tiles(ag, T, B * GH * GW, G, self.workspace(
                    "order", (B * GH * GW + 1,), torch.int32, dev), macs_per_tile=macs_tile,
                    tau=tau, r_min=r_min)
        id_nhwc = id_desc = id_nnz = None
        id_keep = ()
        if identity is not None:
            require_gpu_tensor(identity, "identity")
            if identity.shape != (T, B, self.Cout, Ho, Wo):
                raise ValueError("identity shape mismatch")
            if identity_mode == ID_ADD_SPIKE:
                # spike-valued identity: read its fp16 NHWC copy when current
                # (through its descriptor: a fused layer's copy, which an
                # output equal to it may alias)
                id_nhwc = shadow_of(identity, (T * B, Ho, Wo, pad32(self.Cout)), resolve=False,
                                    u8_ok=u8)
                if id_nhwc is not None:
                    id_desc = desc_of(identity)
                    if id_desc is None:
                        id_desc = written_desc(dev)
                    id_nnz = count_of(identity)
                    id_keep = (id_nhwc,) + keep_of(identity)
        out, v_out = self._launch(
            xp, T, B, H, W, Ho, Wo, x.numel(), nnz, ag, order, th, tw, gs, v_in, epilogue,
            want_v_out,
            None if id_nhwc is not None else identity, id_nhwc, identity_mode, sparse_threshold,
            emit_nhwc,
            lambda nhwc: lazy_output((T, B, self.Cout) + tuple(nhwc.shape[1:3]), nhwc, dev),
            "conv_mfma" + ("_sparse" if sparse is not None else ""),
            x_desc=x_desc, id_desc=id_desc, id_nnz=id_nnz, id_keep=id_keep, u8=u8)
        self.last_tiles = None if ag is None else (tc_buf, ag)
        self.last_order = order
        return out, v_out

    def _launch(self, xp, T, B, H, W, Ho, Wo, numel, nnz, ag, order, th, tw, gs, v_in, epilogue,
                want_v_out, identity, id_nhwc, identity_mode, sparse_threshold, emit_nhwc,
                make_lazy, timer_name, x_desc=None, id_desc=None, id_nnz=None, id_keep=(),
                u8=False):
        """One cf_conv_mfma launch on the staged fp16 NHWC input xp (u8: one
        cf_conv_halo_u8 launch, xp, id_nhwc and the output copy one byte per
        channel); the output is make_lazy(nhwc copy) when emitting the copy
        (with its count block attached), else an fp32 NCHW tensor.  x_desc / id_desc: output
        descriptors of the input's / identity's copies (see cf_conv_mfma).
        When the launch may take StaticZero it gets an output descriptor of
        its own (attached to the output, with id_keep: the copies the output
        may alias) and, with no initial state, a per-channel state buffer
        (v_out is then a ChannelState).  Returns (out, v_out)."""
        dev = xp.device
        # the pooled epilogue's output and state are at the pooled size
        Hs, Ws = (Ho // 2, Wo // 2) if epilogue == EPI_POOL else (Ho, Wo)
        if v_in is not None:
            require_gpu_tensor(v_in, "v_in")
            if v_in.numel() != B * self.Cout * Hs * Ws:
                raise ValueError("v_in has the wrong size")
        # the halo kernel carries the membrane state between its time blocks
        # (2 or 4 steps) through v_out, so it gets one whenever T > 2
        v_out = (torch.empty((B, self.Cout, Hs, Ws), dtype=torch.float32, device=dev)
                 if (epilogue != EPI_Z and (want_v_out or T > 2)) else None)
        cp_out = pad32(self.Cout)
        nhwc = (torch.empty((T * B, Hs, Ws, cp_out), dtype=torch.uint8 if u8 else torch.float16,
                            device=dev)
                if (emit_nhwc and epilogue != EPI_Z) else None)
        nz_out = None
        if nhwc is not None:
            # spikes: written as the NHWC copy only; fp32 on first outside read
            out = make_lazy(nhwc)
            out_ptr = None
            nz_out = self.out_counter(dev)
            self._gen[0] += 1
            attach_count(out, nz_out, self._gen)
        else:
            out = torch.empty((T, B, self.Cout, Ho, Wo), dtype=torch.float32, device=dev)
            out_ptr = ptr(out)
        desc = None
        if (COPY_ELISION and nhwc is not None and epilogue != EPI_Z
                and (nnz is not None or x_desc is not None)):
            desc = new_out_desc(dev)
        bias_info, v_chan = self.zero_route_info(dev, T, desc, v_out, v_in,
                                                 pool=epilogue == EPI_POOL)
        if bias_info & 1:
            # the launch may leave the copy unwritten: readers go through
            # the descriptor (otherwise it always writes the copy)
            attach_desc(out, desc, id_keep)
        ev = _t0()
        if u8:
            rc = _hip.lib().cf_conv_halo_u8(
                ptr(xp), ptr(self.w_packed), ptr(self.alpha), ptr(self.beta), ptr(v_in),
                ptr(v_out), ptr(nhwc), cp_out, ptr(id_nhwc), pad32(self.Cout), ptr(ag),
                ptr(order), ptr(nnz), ptr(nz_out), ptr(x_desc), ptr(id_desc), ptr(desc),
                bias_info, ptr(id_nnz), numel, float(sparse_threshold), T, B, self.Cp, self.Cout,
                self.Coutp, H, W, Ho, Wo, self.KH, self.stride, self.padding, gs, *self.lif,
                _hip.stream(dev))
            check(rc, "cf_conv_halo_u8")
        else:
            rc = _hip.lib().cf_conv_mfma(
                ptr(xp), ptr(self.w_packed), ptr(self.alpha), ptr(self.beta), ptr(v_in),
                ptr(v_out), out_ptr, ptr(nhwc), cp_out, ptr(identity), ptr(id_nhwc),
                pad32(self.Cout), int(identity_mode), ptr(ag), ptr(order), ptr(nnz), ptr(nz_out),
                ptr(x_desc), ptr(id_desc), ptr(desc), bias_info, ptr(id_nnz), numel,
                float(sparse_threshold), T, B, self.Cp, self.Cout, self.Coutp, H, W, Ho, Wo,
                self.KH, self.KW, self.stride, self.padding, B, th, tw, gs, int(epilogue),
                *self.lif, _hip.stream(dev))
            check(rc, "cf_conv_mfma")
        if ev is not None:
            copy_bytes = (nhwc.element_size() * T * B * Hs * Ws * cp_out if nhwc is not None
                          else 0) + (4 * T * B * Ho * Wo * self.Cout if out_ptr is not None else 0)
            state_bytes = 4 * B * Hs * Ws * self.Cout if v_out is not None else 0
            _t1(timer_name, ev, flops=2 * T * B * Ho * Wo * self.Cout * self.Cin * self.KH * self.KW,
                route=None if nnz is None else _RouteProbe(nnz, [(desc, copy_bytes, state_bytes)]))
        self.last_nnz = nnz  # count block of this input (None: not counted)
        self.last_numel = numel
        if not want_v_out:
            return out, None
        return out, (ChannelState(v_out, v_chan, desc) if v_chan is not None else v_out)

    def _tokens_plan(self, xp, identity, ish, meta, im, want_v_out, grid):
        """The _DensePlan of one token-layer input signature (see
        _tokens_repeat), made with run_tokens' checks; False when run_tokens
        would do anything else than one launch on the copies as they are
        (pack an input, widen a byte copy, an error)."""
        shape, dtype, dev = meta[0], meta[1], meta[2]
        if ((self.KH, self.KW, self.stride, self.padding) != (1, 1, 1, 0)
                or len(shape) not in (3, 4) or dtype != torch.float32 or not meta[4]
                or dev.type != "cuda"):
            return False
        if len(shape) == 3:
            (T, B, C), N = shape, 1
        else:
            T, B, N, C = shape
        if C != self.Cin:
            return False
        nimg, H, W = token_view(B, N) if grid is None else (B,) + tuple(grid)
        if nimg * H * W != B * N:
            return False
        rows = T * B * N
        # the input's copy as token_shadow takes it
        if (xp.device != dev or xp.dtype != torch.float16 or xp.shape[-1] != self.Cp
                or xp.numel() != rows * self.Cp or not xp.is_contiguous()):
            return False
        out_shape = tuple(shape[:-1]) + (self.Cout,)
        cp_out = pad32(self.Cout)
        if identity is not None:
            # identity: fp32, contiguous, the output's shape (require_gpu_tensor)
            ic = ish[0]
            if (tuple(im[0]) != out_shape or im[1:3] != (torch.float32, dev) or not im[4]
                    or ic.device != dev or ic.dtype != torch.float16 or ic.shape[-1] != cp_out
                    or ic.numel() != rows * cp_out or not ic.is_contiguous()):
                return False
        p = _DensePlan()
        p.u8 = False
        p.pool = False
        p.need_v = want_v_out or T > 2
        p.vshape = (nimg, self.Cout, H, W)
        p.vmeta = (torch.Size((nimg, self.Cout, H * W)), torch.float32, dev,
                   nimg * self.Cout * H * W, True)    # the state as run_tokens returns it
        p.cshape = (T * nimg, H, W, cp_out)
        p.cdtype = torch.float16
        p.oshape = out_shape
        p.ometa = (torch.Size(out_shape), torch.float32, dev, rows * self.Cout, True)
        p.nz_out = self.out_counter(dev)
        p.nz_ptr = p.nz_out.data_ptr()
        p.weights = (self.w_packed.data_ptr(), self.alpha.data_ptr(), self.beta.data_ptr())
        p.numel = rows * C
        p.T = T
        p.cp_out = cp_out
        p.bias = None
        p.fn = _hip.lib().cf_conv_mfma_args
        p.tail = (T, nimg, self.Cp, self.Cout, self.Coutp, H, W, H, W, 1, 1, 1, 0, nimg, 0, 0, 0,
                  EPI_LIF) + tuple(self.lif)
        _conv_args_block(p)
        p.args.sparse_threshold = 2.0
        return p

    def _tokens_repeat(self, x, identity, want_v_out, grid):
        """run_tokens' launch for its common case from a plan cached per input
        signature: no initial state, the input (and the identity, if any)
        carrying a current fp16 copy, no kernel timer.  The checks that
        depend only on the signature ran when the plan was made; a call
        reads the copies' descriptors and count blocks, allocates the
        outputs and launches with the arguments run_tokens passes.  None
        when the case is not covered."""
        rec = _copy_record(x)
        if rec is None:
            return None
        d, xp, ver, meta = rec
        dev = meta[2]
        ish = im = None
        if identity is not None:
            irec = _copy_record(identity)
            if irec is None:
                return None
            idd, ic, iver, im = irec
            ish = (ic, iver)
            key = ("tokens", meta, xp.shape, xp.dtype, want_v_out, im, ic.shape, ic.dtype, grid,
                   COPY_ELISION)
        else:
            key = ("tokens", meta, xp.shape, xp.dtype, want_v_out, None, None, None, grid,
                   COPY_ELISION)
        self._ensure_packed(dev)
        p = self._plans.get(key)
        if p is None:
            p = self._plans[key] = self._tokens_plan(xp, identity, ish, meta, im, want_v_out,
                                                     grid)
        if p is False:
            return None
        x_desc, nnz = _desc_count(d, ver)
        id_ptr = id_desc = id_nnz = 0
        id_keep = ()
        if identity is not None:
            id_ptr, id_desc, id_nnz, id_keep = _identity_args(idd, ic, iver, dev)
        out, v_out, nhwc, desc, info, v_chan = self._plan_outputs(
            p, dev, COPY_ELISION and (nnz is not None or x_desc is not None), id_keep,
            tokens=True)
        a = p.args
        a.x = xp.data_ptr()
        a.v_out = v_out.data_ptr() if v_out is not None else None
        a.out_nhwc = nhwc.data_ptr()
        a.identity_nhwc = id_ptr or None
        a.nnz = nnz.data_ptr() if nnz is not None else None
        a.x_desc = x_desc.data_ptr() if x_desc is not None else None
        a.id_desc = id_desc or None
        a.out_desc = desc.data_ptr() if desc is not None else None
        a.bias_info = info
        a.id_nnz = id_nnz or None
        a.stream = _hip.stream(dev)
        check(p.fn(p.args_addr), "cf_conv_mfma")
        self.last_nnz = nnz
        self.last_numel = p.numel
        if not want_v_out:
            return out, None
        nimg, Cout, H, W = p.vshape
        vv = v_out.view(nimg, Cout, H * W)
        return out, (ChannelState(vv, v_chan, desc, meta=p.vmeta) if v_chan is not None else vv)

    def run_tokens(self, x: torch.Tensor, v_in=None, *, identity=None, want_v_out=True,
                   static_zero=True, grid=None):
        """Linear -> (BN) -> LIF over token-major x [T, B, N, Cin]: a 1x1 conv
        over the token rows of each step, viewed as `nimg` images of H x W
        tokens (token_view: 8 x 8 images of 64 consecutive tokens when 64
        divides B * N, whole MFMA tiles; else each image's N tokens).  x's
        fp16 copy (a fused token layer's output) is read directly, otherwise
        x is packed.  identity [T, B, N, Cout] is added to the spikes (a
        residual), read from its fp16 copy (packed if it has none; its values
        must be fp16-exact).  The membrane state is per view image,
        [nimg, Cout, H * W] (token_membrane gives it as [B, N, Cout]).
        x may also be [T, B, Cin] (one token per sample, N = 1; identity and
        output are then [T, B, Cout]).
        Returns (lazy fp32 tokens [T, B, N, Cout], v_out or None)."""
        if v_in is None and static_zero and _timer is None and REPEAT_PLANS:
            r = self._tokens_repeat(x, identity, want_v_out,
                                    None if grid is None else tuple(grid))
            if r is not None:
                return r
        require_gpu_tensor(x, "x")
        if self.KH != 1 or self.KW != 1 or self.stride != 1 or self.padding != 0:
            raise ValueError("run_tokens needs a 1x1 kernel with stride 1 and no padding")
        if x.dim() == 3:
            (T, B, C), N = x.shape, 1
        else:
            T, B, N, C = x.shape
        out_shape = tuple(x.shape[:-1]) + (self.Cout,)
        if C != self.Cin:
            raise ValueError(f"expected {self.Cin} input channels, got {C}")
        dev = x.device
        self._ensure_packed(dev)
        if grid is None:
            nimg, H, W = token_view(B, N)
        else:
            (H, W), nimg = grid, B
        if nimg * H * W != B * N:
            raise ValueError("token grid does not match N")
        xp = token_shadow(x, self.Cp, resolve=False)
        nnz = x_desc = None
        if xp is not None:
            nnz = count_of(x) if static_zero else None
            x_desc = desc_of(x)
        else:
            nnz = self.counter(dev) if static_zero else None
            xp = pack_tokens(x, self.Cp, nnz=nnz, status=status_word(dev),
                             out=self.workspace("xp", (T * B * N, self.Cp), torch.float16, dev))
        id_cp = pad32(self.Cout)
        id_copy = id_desc = id_nnz = None
        id_keep = ()
        if identity is not None:
            require_gpu_tensor(identity, "identity")
            if tuple(identity.shape) != out_shape:
                raise ValueError("identity shape mismatch")
            id_copy = token_shadow(identity, id_cp, resolve=False)
            if id_copy is not None:
                # a fused layer's copy, read through its descriptor
                id_desc = desc_of(identity)
                if id_desc is None:
                    id_desc = written_desc(dev)
                id_nnz = count_of(identity)
                id_keep = (id_copy,) + keep_of(identity)
            else:
                id_copy = pack_tokens(identity, id_cp, status=status_word(dev),
                                      out=self.workspace("idp", (T * B * N, id_cp),
                                                         torch.float16, dev))
        out, v_out = self._launch(
            xp.view(T * nimg, H, W, self.Cp), T, nimg, H, W, H, W, x.numel(), nnz, None, None,
            0, 0, 0, v_in, EPI_LIF, want_v_out, None,
            None if id_copy is None else id_copy.view(T * nimg, H, W, id_cp), ID_ADD_SPIKE, 2.0,
            True, lambda nhwc: lazy_tokens(out_shape, nhwc, dev), "linear_tokens",
            x_desc=x_desc, id_desc=id_desc, id_nnz=id_nnz, id_keep=id_keep)
        return out, (None if v_out is None else lazy_view(v_out, nimg, self.Cout, H * W))

    def run_direct(self, x: torch.Tensor, v_in=None, *, epilogue=EPI_LIF, want_v_out=True,
                   emit_nhwc=False):
        """Analog-input path (fp32 VALU).  x may have a stride-0 time axis
        (direct encoding), in which case the conv is evaluated once."""
        if not x.is_cuda or x.dtype != torch.float32:
            raise RuntimeError("x must be a float32 GPU tensor")
        T, B, C, H, W = x.shape
        dev = x.device
        self._ensure_packed(dev)
        if x.stride(0) == 0 and x[0].is_contiguous():
            tstride = 0
            xb = x[0]
        else:
            x = x.contiguous()
            tstride = B
            xb = x
        Ho, Wo = self.out_hw(H, W)
        if v_in is not None:
            require_gpu_tensor(v_in, "v_in")
        # the halo kernel carries the membrane state between its time blocks
        # (2 or 4 steps) through v_out, so it gets one whenever T > 2
        v_out = (torch.empty((B, self.Cout, Ho, Wo), dtype=torch.float32, device=dev)
                 if (epilogue == EPI_LIF and (want_v_out or T > 2)) else None)
        cp_out = pad32(self.Cout)
        nhwc = (torch.empty((T * B, Ho, Wo, cp_out), dtype=torch.float16, device=dev)
                if (emit_nhwc and epilogue == EPI_LIF) else None)
        if nhwc is not None:
            # spikes written as the NHWC copy only, fp32 on first outside read
            out = lazy_output((T, B, self.Cout, Ho, Wo), nhwc, dev)
            out_ptr = None
        else:
            out = torch.empty((T, B, self.Cout, Ho, Wo), dtype=torch.float32, device=dev)
            out_ptr = ptr(out)
        ev = _t0()
        rc = _hip.lib().cf_conv_direct(
            ptr(xb), ptr(self._w_f32), ptr(self.alpha_direct), ptr(self.beta_direct), ptr(v_in),
            ptr(v_out), out_ptr, ptr(nhwc), cp_out, T, B, C, self.Cout, H, W, Ho, Wo, self.KH,
            self.KW, self.stride, self.padding, tstride, int(epilogue), *self.lif,
            _hip.stream(dev))
        check(rc, "cf_conv_direct")
        _t1("conv_direct", ev, flops=2 * (1 if tstride == 0 else T) * B * Ho * Wo * self.Cout *
            C * self.KH * self.KW)
        return out, v_out

    # -- analog 3 x 3 conv -> BN -> LIF -> MaxPool(3, 2, 1) ------------------

    def direct_pool_supported(self, x: torch.Tensor, pool) -> bool:
        """cf_conv_direct_lif_maxpool covers a 3 x 3, stride-1 conv (padding
        <= 2) over an fp32 input of at most 4 channels, Cout a multiple of 16,
        followed by MaxPool2d(3, 2, 1)."""
        return (x.dim() == 5 and x.dtype == torch.float32 and x.is_cuda and self.Cin <= 4
                and self.KH == 3 and self.KW == 3 and self.stride == 1 and self.padding <= 2
                and self.Cout % 16 == 0 and x.shape[1] <= 65535
                and tuple(int(p) for p in pool) == (3, 2, 1))

    def run_direct_pool(self, x: torch.Tensor, v_in=None, *, want_v_out=True, nz_out=None,
                        gen_cell=None):
        """x [T, B, Cin, H, W] (a stride-0 time axis evaluates the conv once).
        Returns the pooled spikes [T, B, Cout, Hp, Wp] as a lazy output over
        their fp16 NHWC copy (with nz_out and gen_cell, carrying its count
        block) and the conv-resolution membrane [B, Cout, Ho, Wo]."""
        if not self.direct_pool_supported(x, (3, 2, 1)):
            raise ValueError("input/layer not covered by cf_conv_direct_lif_maxpool")
        _require_block(nz_out)
        T, B, C, H, W = x.shape
        dev = x.device
        self._ensure_packed(dev)
        if x.stride(0) == 0 and x[0].is_contiguous():
            tstride, xb = 0, x[0]
        else:
            x = x.contiguous()
            tstride, xb = B, x
        Ho, Wo = self.out_hw(H, W)
        Hp, Wp = (Ho - 1) // 2 + 1, (Wo - 1) // 2 + 1
        if v_in is not None:
            v_in = v_in.contiguous()   # (a state the stem kernel left is channels-last)
            require_gpu_tensor(v_in, "v_in")
            if v_in.numel() != B * self.Cout * Ho * Wo:
                raise ValueError("v_in has the wrong size")
        v_out = (torch.empty((B, self.Cout, Ho, Wo), dtype=torch.float32, device=dev)
                 if want_v_out else None)
        cp_out = pad32(self.Cout)
        nhwc = torch.empty((T * B, Hp, Wp, cp_out), dtype=torch.float16, device=dev)
        ev = _t0()
        rc = _hip.lib().cf_conv_direct_lif_maxpool(
            ptr(xb), ptr(self._wt_f32), ptr(self.alpha_direct), ptr(self.beta_direct),
            ptr(v_in), ptr(v_out), ptr(nhwc), cp_out, ptr(nz_out), T, B, C, self.Cout, H, W,
            self.padding, tstride, *self.lif, _hip.stream(dev))
        check(rc, "cf_conv_direct_lif_maxpool")
        _t1("conv_direct_pool", ev, flops=2 * (1 if tstride == 0 else T) * B * Ho * Wo *
            self.Cout * C * 9)
        out = lazy_output((T, B, self.Cout, Hp, Wp), nhwc, dev)
        if nz_out is not None and gen_cell is not None:
            gen_cell[0] += 1
            attach_count(out, nz_out, gen_cell)
        return out, v_out

    # -- analog 3 x 3 conv -> BN -> AvgPool(2, 2) -> LIF ---------------------

    def direct_avgpool_supported(self, x: torch.Tensor) -> bool:
        """cf_conv_direct_avgpool_lif covers a 3 x 3, stride-1 conv (padding
        <= 2) over an fp32 input of at most 4 channels, Cout a multiple of 16,
        with a conv output of at least 2 x 2."""
        if not (x.dim() == 5 and x.dtype == torch.float32 and x.is_cuda and self.Cin <= 4
                and self.KH == 3 and self.KW == 3 and self.stride == 1 and self.padding <= 2
                and self.Cout % 16 == 0 and x.shape[1] <= 65535):
            return False
        Ho, Wo = self.out_hw(x.shape[3], x.shape[4])
        return Ho >= 2 and Wo >= 2

    def run_direct_avgpool(self, x: torch.Tensor, v_in=None, *, want_v_out=True, nz_out=None,
                           gen_cell=None):
        """x [T, B, Cin, H, W] analog (a stride-0 time axis evaluates the conv
        once) -> (pooled spikes [T, B, Cout, Ho//2, Wo//2] as a lazy output
        over their fp16 NHWC copy, carrying its count block with nz_out and
        gen_cell; pooled membrane [B, Cout, Ho//2, Wo//2])."""
        if not self.direct_avgpool_supported(x):
            raise ValueError("input/layer not covered by cf_conv_direct_avgpool_lif")
        _require_block(nz_out)
        T, B, C, H, W = x.shape
        dev = x.device
        self._ensure_packed(dev)
        if x.stride(0) == 0 and x[0].is_contiguous():
            tstride, xb = 0, x[0]
        else:
            x = x.contiguous()
            tstride, xb = B, x
        Ho, Wo = self.out_hw(H, W)
        Hp, Wp = Ho // 2, Wo // 2
        if v_in is not None:
            require_gpu_tensor(v_in, "v_in")
            if v_in.numel() != B * self.Cout * Hp * Wp:
                raise ValueError("v_in has the wrong size")
        v_out = (torch.empty((B, self.Cout, Hp, Wp), dtype=torch.float32, device=dev)
                 if want_v_out else None)
        cp_out = pad32(self.Cout)
        nhwc = torch.empty((T * B, Hp, Wp, cp_out), dtype=torch.float16, device=dev)
        ev = _t0()
        rc = _hip.lib().cf_conv_direct_avgpool_lif(
            ptr(xb), ptr(self._wt_f32), ptr(self.alpha_direct), ptr(self.beta_direct),
            ptr(v_in), ptr(v_out), ptr(nhwc), cp_out, ptr(nz_out), T, B, C, self.Cout, H, W,
            self.padding, tstride, *self.lif, _hip.stream(dev))
        check(rc, "cf_conv_direct_avgpool_lif")
        _t1("conv_direct_avgpool", ev, flops=2 * (1 if tstride == 0 else T) * B * Ho * Wo *
            self.Cout * C * 9)
        out = lazy_output((T, B, self.Cout, Hp, Wp), nhwc, dev)
        if nz_out is not None and gen_cell is not None:
            gen_cell[0] += 1
            attach_count(out, nz_out, gen_cell)
        return out, v_out

    # -- fused stem: Conv -> BN -> LIF -> MaxPool(3, 2, 1) -------------------

    def stem_supported(self, x: torch.Tensor, pool) -> bool:
        """cf_conv_stem_lif_maxpool covers a direct-encoded image (stride-0
        time axis, or T = 1), at most 4 input channels, filters up to 7 x 8, conv
        stride 2 or 1, T <= 32 and MaxPool2d(3, 2, 1)."""
        return (x.dim() == 5 and (x.stride(0) == 0 or x.shape[0] == 1) and x[0].is_contiguous()
                and x.dtype == torch.float32 and self.Cin <= 4 and self.KH <= 7
                and self.KW <= 8 and self.stride in (1, 2) and 1 <= x.shape[0] <= 32
                and tuple(int(p) for p in pool) == (3, 2, 1))

    def _ensure_stem_packed(self, device):
        key = ("stem",) + self._param_key(device)
        if key == getattr(self, "_stem_key", None):
            return
        w = self.weight.detach().float().contiguous()
        bs = None if self.bn_scale is None else self.bn_scale.detach().float().contiguous()
        bh = None if self.bn_shift is None else self.bn_shift.detach().float().contiguous()
        bi = None if self.bias is None else self.bias.detach().float().contiguous()
        for name, t in (("weight", w), ("bn_scale", bs), ("bn_shift", bh), ("bias", bi)):
            if t is not None:
                require_gpu_tensor(t, name)
        self.w_stem = torch.empty((2, self.Coutp, self.KH, 32), dtype=torch.float16,
                                  device=device)
        self.alpha_stem = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        self.beta_stem = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        check(_hip.lib().cf_pack_stem_weights(ptr(w), self.Cout, self.Cin, self.KH, self.KW,
                                              self.Coutp, ptr(bs), ptr(bh), ptr(bi),
                                              ptr(self.w_stem), ptr(self.alpha_stem),
                                              ptr(self.beta_stem), _hip.stream(device)),
              "cf_pack_stem_weights")
        self._stem_key = key

    def run_stem_pool(self, x: torch.Tensor, v_in=None, *, want_v_out=True, emit_nhwc=True,
                      nz_out=None, gen_cell=None):
        """x [T, B, Cin, H, W] with a stride-0 time axis.  Returns the pooled
        spikes [T, B, Cout, Hp, Wp] (carrying the fp16 NHWC copy when
        emit_nhwc, and with nz_out and gen_cell its count block) and the
        conv-resolution membrane [B, Cout, Hc, Wc] (channels_last memory
        format)."""
        if not self.stem_supported(x, (3, 2, 1)):
            raise ValueError("input/layer not covered by the fused stem kernel")
        T, B, C, H, W = x.shape
        dev = x.device
        require_gpu_tensor(x[0], "x")
        self._ensure_stem_packed(dev)
        _require_block(nz_out)
        Hc, Wc = self.out_hw(H, W)
        Hp, Wp = (Hc - 1) // 2 + 1, (Wc - 1) // 2 + 1
        # the membrane is kept channels-last (the kernel's state layout)
        if v_in is not None:
            if not isinstance(v_in, torch.Tensor) or tuple(v_in.shape) != (B, self.Cout, Hc, Wc):
                raise ValueError("v_in must be a [B, Cout, Hc, Wc] tensor")
            v_in = v_in.contiguous(memory_format=torch.channels_last)
            require_gpu_tensor(v_in.permute(0, 2, 3, 1), "v_in")   # its [B, Hc, Wc, Cout] storage
        v_out = (torch.empty((B, self.Cout, Hc, Wc), dtype=torch.float32, device=dev,
                             memory_format=torch.channels_last) if want_v_out else None)
        cp_out = pad32(self.Cout)
        u8 = emit_nhwc and SPIKE_COPY == "u8"
        if emit_nhwc:
            nhwc = torch.empty((T * B, Hp, Wp, cp_out), dtype=torch.uint8 if u8 else torch.float16,
                               device=dev)
            out = lazy_output((T, B, self.Cout, Hp, Wp), nhwc, dev)
            out_ptr = None
        else:
            nhwc = None
            out = torch.empty((T, B, self.Cout, Hp, Wp), dtype=torch.float32, device=dev)
            out_ptr = ptr(out)
        ev = _t0()
        stem = (_hip.lib().cf_conv_stem_lif_maxpool_u8 if u8
                else _hip.lib().cf_conv_stem_lif_maxpool)
        rc = stem(
            ptr(x[0]), ptr(self.w_stem), ptr(self.alpha_stem), ptr(self.beta_stem), ptr(v_in),
            ptr(v_out), out_ptr, ptr(nhwc), cp_out, ptr(status_word(dev)), ptr(nz_out), T, B, C,
            self.Cout, self.Coutp, H, W, self.KH, self.KW, self.stride, self.padding, 3, 2, 1,
            *self.lif, _hip.stream(dev))
        check(rc, "cf_conv_stem_lif_maxpool")
        _t1("conv_stem", ev, flops=2 * B * Hc * Wc * self.Cout * C * self.KH * self.KW)
        if nz_out is not None and gen_cell is not None:
            gen_cell[0] += 1
            attach_count(out, nz_out, gen_cell)
        return out, v_out


def halo_pair_supported(ra: "ConvLIFRunner", rb: "ConvLIFRunner", x: torch.Tensor) -> bool:
    """Whether cf_conv_halo_pair computes ra (3x3, stride 2) and rb (1x1,
    stride 2) of x [T, B, Cin, H, W] in one launch: same input channels,
    output size and LIF parameters, whole 32-channel outputs, the shapes
    the halo kernel covers."""
    if x.dim() != 5 or not x.is_cuda or x.dtype != torch.float32:
        return False
    T, B, C, H, W = x.shape
    if (ra.KH, ra.KW, rb.KH, rb.KW) != (3, 3, 1, 1) or ra.stride != 2 or rb.stride != 2:
        return False
    if ra.Cin != C or rb.Cin != C or ra.lif != rb.lif or ra.Cout % 32 or rb.Cout % 32:
        return False
    if ra.padding > 2 or rb.padding > 2 or ra.Cp // 32 > 64:
        return False
    Ho, Wo = ra.out_hw(H, W)
    if rb.out_hw(H, W) != (Ho, Wo) or Ho < 4 or Wo < 4:
        return False
    return T * B * max(ra.Cout, rb.Cout) * Ho * Wo <= 2 ** 31 - 1 and 4 * B * H * W * ra.Cp < 2 ** 31


class _PairPlan:
    """What run_halo_pair decides from an input signature alone
    (halo_pair_repeat): the copy format, the partner, the static launch
    arguments and, per conv, a _DensePlan of its outputs."""
    __slots__ = ("rb", "rb_key", "u8", "fn", "numel", "head", "halves", "args", "args_addr")


def _halo_pair_plan(ra, rb, x, xp, meta):
    """The _PairPlan of one input signature, made with run_halo_pair's
    checks; False when run_halo_pair would do anything else than one paired
    launch on x's copy as it is (pack the input, widen a byte copy, an
    error)."""
    if len(meta[0]) != 5 or meta[1] != torch.float32 or not meta[4]:
        return False
    T, B, C, H, W = meta[0]
    dev = meta[2]
    if not halo_pair_supported(ra, rb, x):
        return False
    if xp.device != dev or tuple(xp.shape) != (T * B, H, W, ra.Cp):
        return False
    u8 = SPIKE_COPY == "u8" and xp.dtype == torch.uint8
    if xp.dtype != (torch.uint8 if u8 else torch.float16):
        return False
    Ho, Wo = ra.out_hw(H, W)
    p = _PairPlan()
    p.rb, p.rb_key = rb, rb._packed_key
    p.u8 = u8
    p.fn = _hip.lib().cf_conv_halo_pair_u8 if u8 else _hip.lib().cf_conv_halo_pair
    p.numel = T * B * C * H * W
    p.head = (p.numel, T, B, ra.Cp, H, W, Ho, Wo)
    halves = []
    for r in (ra, rb):
        h = _DensePlan()
        h.u8, h.pool, h.need_v, h.T, h.bias = u8, False, True, T, None
        h.cp_out = pad32(r.Cout)
        h.vshape = (B, r.Cout, Ho, Wo)
        h.vmeta = (torch.Size(h.vshape), torch.float32, dev, B * r.Cout * Ho * Wo, True)
        h.cshape = (T * B, Ho, Wo, h.cp_out)
        h.cdtype = torch.uint8 if u8 else torch.float16
        h.oshape = (T, B, r.Cout, Ho, Wo)
        h.ometa = (torch.Size(h.oshape), torch.float32, dev, T * B * r.Cout * Ho * Wo, True)
        h.nz_out = r.out_counter(dev)
        h.nz_ptr = h.nz_out.data_ptr()
        h.weights = (r.w_packed.data_ptr(), r.alpha.data_ptr(), r.beta.data_ptr())
        h.numel = p.numel
        h.fn = None
        h.tail = (r.Cout, r.Coutp, r.padding)
        halves.append((r, h))
    p.halves = tuple(halves)
    p.args = p.args_addr = None
    if not u8:
        # the cf_conv_halo_pair_args block, static fields filled
        p.fn = _hip.lib().cf_conv_halo_pair_args
        a = _hip.ConvHaloPairArgs()
        a.numel, a.T, a.B, a.Cp, a.H, a.W, a.Ho, a.Wo = p.head
        for sfx, (r, h) in zip(("_a", "_b"), halves):
            for f, v in zip(("w", "alpha", "beta"), h.weights):
                setattr(a, f + sfx, v)
            setattr(a, "v_in" + sfx, None)
            setattr(a, "cp_out" + sfx, h.cp_out)
            setattr(a, "nz" + sfx, h.nz_ptr)
            for f, v in zip(("Cout", "Coutp", "pad"), h.tail):
                setattr(a, f + sfx, v)
        a.tau, a.v_th, a.v_reset, a.hard_reset, a.decay_input = ra.lif
        p.args = a
        p.args_addr = ctypes.addressof(a)
    return p


def halo_pair_repeat(ra, rb, x):
    """run_halo_pair's launch for its common case from a plan cached per
    input signature: no initial states, x carrying a current NHWC copy, no
    kernel timer.  The checks that depend only on the signature ran when
    the plan was made; each call reads the copy's descriptor and count
    block, allocates the outputs and launches with the arguments the
    general path passes.  None when the case is not covered."""
    if _timer is not None or not REPEAT_PLANS:
        return None
    rec = _copy_record(x)
    if rec is None:
        return None
    d, xp, ver, meta = rec
    dev = meta[2]
    ra._ensure_packed(dev)
    rb._ensure_packed(dev)
    key = ("pair", meta, xp.shape, xp.dtype, SPIKE_COPY, COPY_ELISION)
    p = ra._plans.get(key)
    if p is None or (p is not False and (p.rb is not rb or p.rb_key is not rb._packed_key)):
        p = ra._plans[key] = _halo_pair_plan(ra, rb, x, xp, meta)
    if p is False:
        return None
    x_desc, nnz = _desc_count(d, ver)
    elide = COPY_ELISION and (nnz is not None or x_desc is not None)
    res = []
    args = []
    a = p.args
    for sfx, (r, h) in zip(("_a", "_b"), p.halves):
        out, v_out, nhwc, desc, info, v_chan = r._plan_outputs(h, dev, elide)
        res.append((out, v_out, v_chan, desc, h.vmeta))
        dp = desc.data_ptr() if desc is not None else None
        if a is not None:
            setattr(a, "v_out" + sfx, v_out.data_ptr())
            setattr(a, "out" + sfx, nhwc.data_ptr())
            setattr(a, "desc" + sfx, dp)
            setattr(a, "bias_info" + sfx, info)
        else:
            args += [*h.weights, None, v_out.data_ptr(), nhwc.data_ptr(), h.cp_out, h.nz_ptr, dp,
                     info, *h.tail]
    xd = x_desc.data_ptr() if x_desc is not None else None
    nn = nnz.data_ptr() if nnz is not None else None
    if a is not None:
        a.x, a.nnz, a.x_desc, a.stream = xp.data_ptr(), nn, xd, _hip.stream(dev)
        check(p.fn(p.args_addr), "cf_conv_halo_pair")
    else:
        check(p.fn(xp.data_ptr(), nn, xd, *p.head, *args, *ra.lif, _hip.stream(dev)),
              "cf_conv_halo_pair")
    for r in (ra, rb):
        r.last_nnz = nnz
        r.last_numel = p.numel
    (oa, voa, ca, da, ma), (ob, vob, cb, db, mb) = res
    if ca is not None:
        voa = ChannelState(voa, ca, da, meta=ma)
    if cb is not None:
        vob = ChannelState(vob, cb, db, meta=mb)
    return oa, voa, ob, vob


def run_halo_pair(ra: "ConvLIFRunner", rb: "ConvLIFRunner", x: torch.Tensor, v_in_a=None,
                  v_in_b=None):
    """A ResNet block's stride-2 3x3 conv1 (ra) and 1x1 downsample (rb) of
    the same input in one cf_conv_halo_pair launch, each output exactly
    what run_mfma would return (an NHWC-backed spike tensor with its count
    block).  x: [T, B, Cin, H, W] (its fp16 NHWC copy when it carries one,
    else packed here).  Returns (out_a, v_out_a, out_b, v_out_b)."""
    if v_in_a is None and v_in_b is None:
        r = halo_pair_repeat(ra, rb, x)
        if r is not None:
            return r
    if not halo_pair_supported(ra, rb, x):
        raise ValueError("cf_conv_halo_pair does not cover these convolutions")
    T, B, C, H, W = x.shape
    dev = x.device
    ra._ensure_packed(dev)
    rb._ensure_packed(dev)
    Ho, Wo = ra.out_hw(H, W)
    # byte copies in, byte copies out (cf_conv_halo_pair_u8)
    cand = (shadow_of(x, (T * B, H, W, ra.Cp), resolve=False, u8_ok=True)
            if SPIKE_COPY == "u8" else None)
    u8 = cand is not None and cand.dtype == torch.uint8
    xp = shadow_of(x, (T * B, H, W, ra.Cp), resolve=False, u8_ok=u8)
    x_desc = None
    if xp is not None:
        nnz = count_of(x)
        x_desc = desc_of(x)
    else:
        nnz = ra.counter(dev)
        xp = ra.workspace("xp", (T * B, H, W, ra.Cp), torch.float16, dev)
        pack_input(x.reshape(T * B, C, H, W), cp=ra.Cp, group_size=0, nnz=nnz, xp_out=xp,
                   status=status_word(dev))
    outs = []
    for r, v_in, tb in ((ra, v_in_a, 2), (rb, v_in_b, 4)):
        if v_in is not None:
            require_gpu_tensor(v_in, "v_in")
            if v_in.numel() != B * r.Cout * Ho * Wo:
                raise ValueError("v_in has the wrong size")
        v_out = torch.empty((B, r.Cout, Ho, Wo), dtype=torch.float32, device=dev)
        cp = pad32(r.Cout)
        nhwc = torch.empty((T * B, Ho, Wo, cp), dtype=torch.uint8 if u8 else torch.float16,
                           device=dev)
        out = lazy_output((T, B, r.Cout, Ho, Wo), nhwc, dev)
        nz = r.out_counter(dev)
        r._gen[0] += 1
        attach_count(out, nz, r._gen)
        desc = None
        if COPY_ELISION and (nnz is not None or x_desc is not None):
            desc = new_out_desc(dev)
        info, v_chan = r.zero_route_info(dev, T, desc, v_out, v_in)
        if info & 1:
            # StaticZero may leave the copy unwritten (no identity here)
            attach_desc(out, desc)
        outs.append((r, v_in, v_out, nhwc, cp, nz, out, desc, info, v_chan))
    ((_, va, voa, na, cpa, nza, oa, da, ia, ca),
     (_, vb, vob, nb, cpb, nzb, ob, db, ib, cb)) = outs
    ev = _t0()
    pair = _hip.lib().cf_conv_halo_pair_u8 if u8 else _hip.lib().cf_conv_halo_pair
    check(pair(
        ptr(xp), ptr(nnz), ptr(x_desc), x.numel(), T, B, ra.Cp, H, W, Ho, Wo,
        ptr(ra.w_packed), ptr(ra.alpha), ptr(ra.beta), ptr(va), ptr(voa), ptr(na), cpa, ptr(nza),
        ptr(da), ia, ra.Cout, ra.Coutp, ra.padding,
        ptr(rb.w_packed), ptr(rb.alpha), ptr(rb.beta), ptr(vb), ptr(vob), ptr(nb), cpb, ptr(nzb),
        ptr(db), ib, rb.Cout, rb.Coutp, rb.padding, *ra.lif, _hip.stream(dev)),
        "cf_conv_halo_pair")
    if ev is not None:
        flops = 2 * T * B * Ho * Wo * C * (ra.Cout * 9 + rb.Cout)
        parts = [(d, (1 if u8 else 2) * T * B * Ho * Wo * cp, 4 * B * Ho * Wo * r.Cout)
                 for d, cp, r in ((da, cpa, ra), (db, cpb, rb))]
        _t1("conv_pair", ev, flops=flops, route=None if nnz is None else _RouteProbe(nnz, parts))
    for r in (ra, rb):
        r.last_nnz = nnz
        r.last_numel = x.numel()
    if ca is not None:
        voa = ChannelState(voa, ca, da)
    if cb is not None:
        vob = ChannelState(vob, cb, db)
    return oa, voa, ob, vob


class GroupedConvLIFRunner:
    """Device state + launch of one fused grouped Conv -> (BN) -> LIF layer
    (groups > 1; depthwise when groups == Cin): cf_conv_grouped_lif.

    weight [Cout, Cin/groups, K, K] fp32; bn_scale/bn_shift [Cout] (folded
    eval BN, optional); bias [Cout] (optional).  The membrane state is kept
    channels-last: a [B, Cout, Ho, Wo] tensor in torch's channels_last
    memory format (the kernel's lanes run along channels)."""

    def __init__(self, weight, groups, bn_scale, bn_shift, bias, stride, padding, tau,
                 v_threshold, v_reset, decay_input):
        self.weight, self.groups = weight, int(groups)
        self.bn_scale, self.bn_shift, self.bias = bn_scale, bn_shift, bias
        self.stride, self.padding = int(stride), int(padding)
        self.lif = _lif_args(tau, v_threshold, v_reset, decay_input)
        self.Cout, self.Cg, self.KH, self.KW = (int(s) for s in weight.shape)
        self.Cin = self.Cg * self.groups
        self.Cp = pad32(self.Cin)
        self.Coutp = ((self.Cout + 63) // 64) * 64
        self._key = None
        self._gen = [0]
        self._blocks = {}

    def _ensure(self, device):
        key = (device, self.weight.data_ptr(), self.weight._version,
               *(None if t is None else (t.data_ptr(), t._version)
                 for t in (self.bn_scale, self.bn_shift, self.bias)))
        if key == self._key:
            return
        w = self.weight.detach().float().contiguous()
        ts = [None if t is None else t.detach().float().contiguous()
              for t in (self.bn_scale, self.bn_shift, self.bias)]
        for name, t in zip(("weight", "bn_scale", "bn_shift", "bias"), [w] + ts):
            if t is not None:
                require_gpu_tensor(t, name)
        self.alpha = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        self.beta = torch.empty(self.Coutp, dtype=torch.float32, device=device)
        check(_hip.lib().cf_pack_conv_weights(ptr(w), self.Cout, self.Cg, self.KH, self.KW,
                                              self.Coutp, self.Cp, ptr(ts[0]), ptr(ts[1]),
                                              ptr(ts[2]), None, ptr(self.alpha), ptr(self.beta),
                                              _hip.stream(device)), "cf_pack_conv_weights")
        self._w = w
        self._key = key

    def out_hw(self, H, W):
        return ((H + 2 * self.padding - self.KH) // self.stride + 1,
                (W + 2 * self.padding - self.KW) // self.stride + 1)

    def _out_block(self, device):
        blk = self._blocks.get(device)
        if blk is None:
            blk = count_block(device)
            self._blocks[device] = blk
        return blk

    def run(self, x: torch.Tensor, v_in=None, *, analog=False, want_v_out=True):
        """x [T, B, Cin, H, W] -> (spikes [T, B, Cout, Ho, Wo] held as their
        fp16 NHWC copy with the output's count block attached, v_out
        [B, Cout, Ho, Wo] channels-last).  A spike-valued input is read from
        its fp16 NHWC copy (packed first when it has none); analog=True reads
        the fp32 tensor (a stride-0 time axis reads one image for all T)."""
        if x.dim() != 5 or x.shape[2] != self.Cin:
            raise ValueError(f"expected [T, B, {self.Cin}, H, W], got {tuple(x.shape)}")
        T, B, C, H, W = x.shape
        dev = x.device
        self._ensure(dev)
        Ho, Wo = self.out_hw(H, W)
        xp = x32 = nnz = None
        tstride = 0
        if analog:
            if x.stride(0) == 0 and x[0].is_contiguous():
                x32, tstride = x[0], 0
            else:
                x32, tstride = x.contiguous(), B
            require_gpu_tensor(x32, "x")
        else:
            require_gpu_tensor(x if x.is_contiguous() else x.contiguous(), "x")
            xp = shadow_of(x, (T * B, H, W, self.Cp))
            if xp is not None:
                nnz = count_of(x)
            else:
                xp, _ = pack_input(x.contiguous().reshape(T * B, C, H, W), cp=self.Cp,
                                   status=status_word(dev))
        if v_in is not None:
            if tuple(v_in.shape) != (B, self.Cout, Ho, Wo):
                raise ValueError("v_in must be [B, Cout, Ho, Wo]")
            v_in = v_in.contiguous(memory_format=torch.channels_last)
            require_gpu_tensor(v_in.permute(0, 2, 3, 1), "v_in")
        v_out = (torch.empty((B, self.Cout, Ho, Wo), dtype=torch.float32, device=dev,
                             memory_format=torch.channels_last) if want_v_out else None)
        cp_out = pad32(self.Cout)
        nhwc = torch.empty((T * B, Ho, Wo, cp_out), dtype=torch.float16, device=dev)
        nz_out = self._out_block(dev)
        ev = _t0()
        check(_hip.lib().cf_conv_grouped_lif(
            ptr(xp), ptr(x32), tstride, ptr(self._w), ptr(self.alpha), ptr(self.beta),
            ptr(v_in), ptr(v_out), ptr(nhwc), cp_out, ptr(nnz), ptr(nz_out), T, B, self.Cin,
            self.Cp, self.Cout, self.groups, H, W, Ho, Wo, self.KH, self.stride, self.padding,
            *self.lif, _hip.stream(dev)), "cf_conv_grouped_lif")
        _t1("conv_grouped", ev,
            flops=2 * T * B * Ho * Wo * self.Cout * self.Cg * self.KH * self.KW,
            nbytes=(4 * T * B * H * W * self.Cin if analog else 2 * T * B * H * W * self.Cp)
            + 2 * T * B * Ho * Wo * cp_out + 4 * B * self.Cout * Ho * Wo * (1 + (v_in is not None)))
        out = lazy_output((T, B, self.Cout, Ho, Wo), nhwc, dev)
        self._gen[0] += 1
        attach_count(out, nz_out, self._gen)
        return out, v_out
