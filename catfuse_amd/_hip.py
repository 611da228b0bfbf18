"""ctypes binding of the gfx950 C-ABI library ``_lib/libcatfuse_amd.so``.

Every entry point takes raw device pointers, int64 sizes and the HIP stream
(torch's current stream), returns a ``hipError_t`` as int, never allocates
and never synchronises.  A non-zero return raises ``RuntimeError``.  There is
no CPU or PyTorch fallback: if the library is missing the import of any
kernel wrapper raises, so a GPU run cannot silently take another path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_int64, c_void_p, c_char_p

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libcatfuse_amd.so")

# name -> argtypes (all return c_int unless listed in _RESTYPES)
_P = c_void_p
_I = c_int64
_SIGNATURES = {
    "cf_version": [],
    "cf_error_string": [c_int],
    "cf_probe_mfma_layout": [_P, _P, _P, _P],
    "cf_lif_multistep": [_P, _P, _P, _P, c_int, _P, _P, c_int, _P, _I, _I, _I, _I,
                         c_double, c_double, c_double, c_int, c_int, _P],
    "cf_avgpool2x2_lif": [_P, _P, _P, c_int, _P, _I, _I, _I, _I,
                          c_double, c_double, c_double, c_int, c_int, _P],
    "cf_pack_input": [_P, _I, _I, _I, _I, _I, _P, _P, c_int, c_float, _P, _P, _P],
    "cf_scan_nhwc": [_P, _I, _I, _I, _I, _I, _P, c_int, c_float, _P, _P],
    "cf_nhwc_to_nchw": [_P, _P, _I, _I, _I, _I, _I, _P],
    "cf_global_avgpool_nhwc": [_P, _P, _P, _I, _I, _I, _I, _P],
    "cf_resolve_copy": [_P, _I, _P, _P],
    "cf_bias_response": [_P, _P, _I, _I, c_int, c_double, c_double, c_double, c_int, c_int, _P,
                         _P, _P],
    "cf_expand_state": [_P, _P, _P, _I, _I, _I, _P],
    "cf_pack_tokens": [_P, _I, _I, _I, _P, _P, _P, _P],
    "cf_tokens_to_f32": [_P, _P, _I, _I, _I, _P],
    "cf_maxpool_nhwc": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    "cf_spike_attention_lif": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, c_int,
                               _I, _I, _I, _I,
                               _I, c_double, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_spike_attention_kv_lif": [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P,
                                  c_int, _I, _I, _I, _I, _I, c_double, c_double, c_double,
                                  c_double, c_int, c_int, _P],
    "cf_route_from_nnz": [_P, _I, c_double, _P, _P],
    "cf_zero_counter": [_P, _P],
    "cf_prescan_tiles": [_P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P],
    "cf_pack_conv_weights": [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "cf_compact_tiles": [_P, _I, _I, _I, c_double, c_double, c_double, _P, _P],
    "cf_conv_mfma": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, c_int, _P, _P, _P, _P,
                     _P, _P, _P, c_int, _P, _I,
                     c_double,
                     _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                     c_int, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_halo": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, c_int, _P, _P, _P, _P,
                     _P, _P, _P, c_int, _P, _I,
                     c_double,
                     _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                     c_int, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_halo_pair": [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                          _P, _P, _P, _P, _P, _P, _I, _P, _P, c_int, _I, _I, _I,
                          _P, _P, _P, _P, _P, _P, _I, _P, _P, c_int, _I, _I, _I,
                          c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_halo_u8": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P,
                        c_int, _P, _I, c_double, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                        _I, _I, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_halo_pair_u8": [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                             _P, _P, _P, _P, _P, _P, _I, _P, _P, c_int, _I, _I, _I,
                             _P, _P, _P, _P, _P, _P, _I, _P, _P, c_int, _I, _I, _I,
                             c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_stem_lif_maxpool_u8": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I,
                                    _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, c_double, c_double,
                                    c_double, c_int, c_int, _P],
    "cf_nhwc_to_nchw_u8": [_P, _P, _I, _I, _I, _I, _I, _P],
    "cf_global_avgpool_nhwc_u8": [_P, _P, _P, _I, _I, _I, _I, _P],
    "cf_copy_u8_to_f16": [_P, _P, _I, _P],
    "cf_pack_stem_weights": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "cf_conv_stem_lif_maxpool": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I,
                                 _I, _I, _I, _I, _I, _I, _I, _I, _I, c_double, c_double,
                                 c_double, c_int, c_int, _P],
    "cf_conv_direct_lif_maxpool": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I,
                                   _I, _I, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_linear_tokens": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "cf_conv_direct_avgpool_lif": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I,
                                   _I, _I, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_sparse_noalloc": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, c_int, _P,
                               c_double, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                               _I, _I, c_int, c_double, c_double, c_double, c_int, c_int, _P],
    "cf_conv_grouped_lif": [_P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I,
                            _I, _I, _I, _I, _I, _I, _I, c_double, c_double, c_double, c_int,
                            c_int, _P],
    "cf_conv_direct": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                       _I, _I, _I, c_int, c_double, c_double, c_double, c_int, c_int, _P],
    # argument blocks (ConvMfmaArgs / ConvHaloPairArgs below), by address
    "cf_conv_mfma_args": [_P],
    "cf_conv_halo_pair_args": [_P],
    "cf_conv_args_sizes": [_P],
}

_D = c_double
# The argument blocks of cf_conv_mfma_args / cf_conv_halo_pair_args
# (include/catfuse_amd.h: CfConvMfmaArgs, CfConvHaloPairArgs): every field
# 8 bytes, in the order of the entry points' parameters.
_CONV_MFMA_FIELDS = [
    ("x", _P), ("w_packed", _P), ("alpha", _P), ("beta", _P), ("v_in", _P), ("v_out", _P),
    ("out", _P), ("out_nhwc", _P), ("cp_out", _I), ("identity", _P), ("identity_nhwc", _P),
    ("cp_id", _I), ("identity_mode", _I), ("ag_mask", _P), ("tile_order", _P), ("nnz", _P),
    ("nz_out", _P), ("x_desc", _P), ("id_desc", _P), ("out_desc", _P), ("bias_info", _I),
    ("id_nnz", _P), ("numel", _I), ("sparse_threshold", _D), ("T", _I), ("B", _I), ("Cp", _I),
    ("Cout", _I), ("Coutp", _I), ("H", _I), ("W", _I), ("Ho", _I), ("Wo", _I), ("KH", _I),
    ("KW", _I), ("stride", _I), ("pad", _I), ("x_img_tstride", _I), ("tile_h", _I),
    ("tile_w", _I), ("group_size", _I), ("epilogue", _I), ("tau", _D), ("v_th", _D),
    ("v_reset", _D), ("hard_reset", _I), ("decay_input", _I), ("stream", _P)]
_PAIR_HALF = [("w", _P), ("alpha", _P), ("beta", _P), ("v_in", _P), ("v_out", _P), ("out", _P),
              ("cp_out", _I), ("nz", _P), ("desc", _P), ("bias_info", _I), ("Cout", _I),
              ("Coutp", _I), ("pad", _I)]
_CONV_HALO_PAIR_FIELDS = (
    [("x", _P), ("nnz", _P), ("x_desc", _P), ("numel", _I), ("T", _I), ("B", _I), ("Cp", _I),
     ("H", _I), ("W", _I), ("Ho", _I), ("Wo", _I)]
    + [(f + "_a", t) for f, t in _PAIR_HALF] + [(f + "_b", t) for f, t in _PAIR_HALF]
    + [("tau", _D), ("v_th", _D), ("v_reset", _D), ("hard_reset", _I), ("decay_input", _I),
       ("stream", _P)])


class ConvMfmaArgs(ctypes.Structure):
    _fields_ = _CONV_MFMA_FIELDS


class ConvHaloPairArgs(ctypes.Structure):
    _fields_ = _CONV_HALO_PAIR_FIELDS
_RESTYPES = {"cf_error_string": c_char_p}

_lib = None


class _Lib:
    def __init__(self, handle):
        self._h = handle
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, c_int)
            setattr(self, name, fn)


def library_path() -> str:
    return _LIB_PATH


def lib() -> _Lib:
    """Load (once) and return the bound library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"catfuse_amd HIP library not found at {_LIB_PATH}; build it with "
                "`python -m catfuse_amd.build` (hipcc --offload-arch=gfx950)")
        _check_fresh()
        _lib = _Lib(ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_LOCAL))
    return _lib


def _check_fresh() -> None:
    """Refuse a library built from other sources than the ones in the tree:
    its entry points may take other arguments than the signatures above."""
    from catfuse_amd import build
    try:
        with open(build.stamp_path()) as fh:
            built = fh.read().strip()
    except OSError:
        built = None
    if built != build.source_digest():
        raise RuntimeError(
            f"catfuse_amd HIP library at {_LIB_PATH} was not built from the current "
            "sources; rebuild it with `python -m catfuse_amd.build`")


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().cf_error_string(rc)
        msg = msg.decode() if isinstance(msg, bytes) else str(msg)
        raise RuntimeError(f"catfuse_amd {what} failed: hipError {rc} ({msg})")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None passes a null pointer).  A fused
    layer's output still held only as its NHWC copy is filled first."""
    if t is None:
        return None
    m = getattr(t, "cf_materialize", None)
    if m is not None:
        m()
    return t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device=None) -> int:
    """hipStream_t of torch's current stream on the tensor's device (the raw
    handle straight from torch's stream registry when it exposes one: no
    Stream object per launch)."""
    if _RAW_STREAM is not None and isinstance(device, torch.device) and device.index is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(t: torch.Tensor, name: str, dtype=torch.float32) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (catfuse_amd has no CPU path)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
