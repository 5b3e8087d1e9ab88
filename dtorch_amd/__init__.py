"""MI355X-native attention operator for DTorch (SdpaOp), built on hand-written gfx950 HIP kernels.

The compute path is ``libdtattn.so`` (C ABI, ``include/dtattn.h``) driven by the C++ host operators in
``_dtattn_host`` (the SdpaOp contract).  There is no CPU or eager-PyTorch fallback: if the native
library is missing, importing :mod:`dtorch_amd.nn.functional` raises.
"""
__all__ = ["nn", "load"]

from ._lib import load  # noqa: E402
