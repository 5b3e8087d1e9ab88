"""Loader for the native library and the host operator extension.

``import torch`` happens first on purpose: torch ships its own HIP runtime (soname
libamdhip64.so.7); loading it before libdtattn.so makes the kernels and torch's streams share one
runtime instance.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the native library, see module docstring)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libdtattn.so")

_host = None
_cabi = None


def _missing(what: str) -> ImportError:
    return ImportError(f"dtorch_amd: {what} is not built; run `python -m dtorch_amd.build` "
                       "(hipcc for gfx950 is required). There is no fallback path.")


def load():
    """Return the host operator extension module (``_dtattn_host``)."""
    global _host
    if _host is None:
        if not os.path.exists(LIB_PATH):
            raise _missing("libdtattn.so")
        try:
            from . import _dtattn_host as h
        except ImportError as e:  # pragma: no cover - depends on the build state
            raise _missing(f"the host extension ({e})") from e
        _host = h
    return _host


def cabi() -> ctypes.CDLL:
    """ctypes handle on libdtattn.so (the C ABI itself)."""
    global _cabi
    if _cabi is None:
        if not os.path.exists(LIB_PATH):
            raise _missing("libdtattn.so")
        _cabi = ctypes.CDLL(LIB_PATH)
    return _cabi


# ctypes mirrors of the C ABI's argument structs (include/dtattn.h), for callers that drive the library
# directly: the codes entry point of the fp8 path, the allocation-free decode, tests of the ABI itself.
class PrefillArgs(ctypes.Structure):
    """dtattn_prefill_args (ABI version 10, same layout as 8); `scale` starts as NaN, the ABI's "1/sqrt(D)"."""
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
                ("lse", ctypes.c_void_p),
                ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("Sq", ctypes.c_int64),
                ("Sk", ctypes.c_int64), ("D", ctypes.c_int64), ("Dv", ctypes.c_int64),
                ("q_stride", ctypes.c_int64 * 3), ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3),
                ("o_stride", ctypes.c_int64 * 3), ("lse_stride", ctypes.c_int64 * 2),
                ("dtype", ctypes.c_int32), ("o_dtype", ctypes.c_int32), ("scale", ctypes.c_float),
                ("causal", ctypes.c_int32), ("q_offset", ctypes.c_int64), ("k_offset", ctypes.c_int64),
                ("q_descale", ctypes.c_void_p), ("k_descale", ctypes.c_void_p), ("v_descale", ctypes.c_void_p),
                ("mask", ctypes.c_void_p), ("mask_stride", ctypes.c_int64 * 3),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t)]

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        if "scale" not in kw:
            self.scale = float("nan")


class DecodeArgs(ctypes.Structure):
    """dtattn_decode_args (ABI version 10, same layout as 8); `scale` starts as NaN, the ABI's "1/sqrt(D)"."""
    _fields_ = [("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
                ("lengths", ctypes.c_void_p), ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
                ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("S_max", ctypes.c_int64),
                ("D", ctypes.c_int64),
                ("q_stride", ctypes.c_int64 * 2), ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3),
                ("o_stride", ctypes.c_int64 * 2), ("lse_stride", ctypes.c_int64 * 1),
                ("dtype", ctypes.c_int32), ("scale", ctypes.c_float), ("chunk", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t)]

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        if "scale" not in kw:
            self.scale = float("nan")


def prefill_fp8_codes(q8, k8, v8, qd, kd, vd, out_dtype, causal=False, q_offset=0, k_offset=0, scale=None,
                      split=True):
    """Attention on e4m3fn codes with per-head descales (dtattn_prefill_fwd, dtype FP8_E4M3FN): the kernel of
    the native fp8 path on codes the caller quantized already.  q8/k8/v8 are contiguous float8_e4m3fn
    [B, H, S, D] device tensors, qd/kd/vd fp32 [B, H]; returns (O [B, Hq, Sq, D] in out_dtype, LSE fp32).
    With `split` the call gets the workspace dtattn_prefill_workspace_size() asks for (the tail split of
    non-causal grids, as the native path runs it); without, it runs unsplit."""
    import torch
    B, Hq, Sq, D = q8.shape
    Hkv, Sk = k8.shape[1], k8.shape[2]
    o = torch.empty(B, Hq, Sq, D, dtype=out_dtype, device=q8.device)
    lse = torch.empty(B, Hq, Sq, device=q8.device)
    a = PrefillArgs()
    a.q, a.k, a.v, a.o, a.lse = q8.data_ptr(), k8.data_ptr(), v8.data_ptr(), o.data_ptr(), lse.data_ptr()
    a.B, a.Hq, a.Hkv, a.Sq, a.Sk, a.D, a.Dv = B, Hq, Hkv, Sq, Sk, D, D
    for dst, t in ((a.q_stride, q8), (a.k_stride, k8), (a.v_stride, v8), (a.o_stride, o)):
        dst[0], dst[1], dst[2] = t.stride(0), t.stride(1), t.stride(2)
    a.lse_stride[0], a.lse_stride[1] = lse.stride(0), lse.stride(1)
    a.dtype, a.o_dtype = 2, 0 if out_dtype == torch.bfloat16 else 1
    a.scale = float("nan") if scale is None else float(scale)
    a.causal, a.q_offset, a.k_offset = int(causal), int(q_offset), int(k_offset)
    a.q_descale, a.k_descale, a.v_descale = qd.data_ptr(), kd.data_ptr(), vd.data_ptr()
    lib = cabi()
    ws = None
    if split:
        lib.dtattn_prefill_workspace_size.argtypes = [ctypes.c_void_p]
        lib.dtattn_prefill_workspace_size.restype = ctypes.c_size_t
        with torch.cuda.device(q8.device):
            nbytes = lib.dtattn_prefill_workspace_size(ctypes.byref(a))
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q8.device)  # the caching allocator aligns to 512 B
            a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    lib.dtattn_prefill_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.dtattn_last_error.restype = ctypes.c_char_p
    st = lib.dtattn_prefill_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(q8.device).cuda_stream))
    if st != 0:
        raise ValueError(f"dtattn_prefill_fwd failed ({st}): {lib.dtattn_last_error().decode()}")
    return o, lse
