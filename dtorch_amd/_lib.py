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
