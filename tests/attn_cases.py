"""Shared input generation and comparison helpers for the attention tests.

Inputs follow the measurement recipe: ``np.random.default_rng(seed).standard_normal`` drawn in the
order Q, K, V (then lengths), cast to bf16 with round-to-nearest-even; the oracle sees the
bf16-rounded values upcast, so a comparison isolates the kernel's own error.
"""
from __future__ import annotations

import numpy as np
import torch

O_TOL_BF16 = 2e-2   # max-abs on bf16 outputs
O_TOL_FP8 = 6e-2    # max-abs on bf16 outputs of the fp8 path
LSE_TOL = 1e-3      # |dLSE| / max(|LSE_ref|, 1)


def randn(rng, shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


def to_dev(x: np.ndarray, dtype=torch.bfloat16, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).to(device)


def rounded(x: np.ndarray, dtype=torch.bfloat16) -> np.ndarray:
    """The values a device tensor of `dtype` holds, as float64."""
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).double().numpy()


def max_abs(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


def lse_rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    fin = np.isfinite(b)
    if not np.array_equal(np.isfinite(a), fin):
        return float("inf")
    if not fin.any():
        return 0.0
    return float(np.max(np.abs(a[fin] - b[fin]) / np.maximum(np.abs(b[fin]), 1.0)))


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().double().numpy()


def cpu_path_full(q: np.ndarray, k: np.ndarray, v: np.ndarray, is_causal: bool, dtype=torch.bfloat16,
                  prerounded: bool = False):
    """DTorch's CPU path on every (batch, head) of a full-size case: libtorch's CPU flash attention in
    fp32 (the kernel SdpaOp::Compute reaches on a CPU mesh, with its LSE) on the values the device
    tensors hold (the `dtype`-rounded inputs, or `q, k, v` as given when `prerounded`).  GQA is spelled
    out with repeat_interleave, i.e. repeat_kv.  Returns float64 (O, LSE)."""
    from oracle import dtorch_cpu_path as cpu
    conv = (lambda x: torch.from_numpy(np.asarray(x, dtype=np.float32))) if prerounded else (
        lambda x: torch.from_numpy(rounded(x, dtype).astype(np.float32)))
    tq, tk, tv = conv(q), conv(k), conv(v)
    g = tq.shape[1] // tk.shape[1]
    if g > 1:
        tk, tv = tk.repeat_interleave(g, dim=1), tv.repeat_interleave(g, dim=1)
    o, lse = cpu.sdpa_with_lse(tq, tk, tv, is_causal=is_causal)
    return o.double().numpy(), lse.double().numpy()
