"""DTorch's CPU-mesh attention path: libtorch's scaled_dot_product_attention on CPU tensors.

Test infrastructure and the timed CPU baseline (bench.py's ``cpu_baseline`` leg); never a product
path.  On ``DeviceMesh('cpu', [0])`` with Replicate placement, SdpaOp::Compute runs exactly
``torch::scaled_dot_product_attention(q, k, v, mask, 0.0, isCausal, scale, enableGqa)``
(dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109) on the local CPU tensors.
The reference never exposes an LSE; for the LSE checks this module uses torch's CPU flash-attention
op, which returns ``(out, logsumexp)`` and is the kernel libtorch dispatches the CPU SDPA to.
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask=None, is_causal: bool = False,
         scale: Optional[float] = None, enable_gqa: bool = False) -> torch.Tensor:
    """The SdpaOp::Compute call on CPU tensors (scaled_dot_product_attention_op.cc:107-109)."""
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask, 0.0, is_causal, scale=scale,
                                                            enable_gqa=enable_gqa)


def sdpa_with_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool = False,
                  scale: Optional[float] = None):
    """(O, LSE) from libtorch's CPU flash-attention kernel (MHA shapes, no mask)."""
    out, lse = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu(q, k, v, 0.0, is_causal, scale=scale)
    return out, lse


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: Sequence[int],
           scale: Optional[float] = None) -> torch.Tensor:
    """Per-sequence loop over the true lengths, is_causal=False, enable_gqa=True (Lq = 1)."""
    outs = []
    for b in range(q.shape[0]):
        L = int(lengths[b])
        outs.append(sdpa(q[b:b + 1], k_cache[b:b + 1, :, :L], v_cache[b:b + 1, :, :L], scale=scale,
                         enable_gqa=True))
    return torch.cat(outs, 0)


def ring_step(q: torch.Tensor, k_chunks, v_chunks, q_chunk_index: int, scale: Optional[float] = None):
    """Blockwise ring step on CPU: the diagonal block with is_causal=True, earlier blocks full,
    per-block LSE from the CPU flash kernel, then a NumPy LSE merge."""
    hq = q.shape[1]
    os_, lses = [], []
    for c in range(q_chunk_index + 1):
        k = k_chunks[c].repeat_interleave(hq // k_chunks[c].shape[1], dim=1)
        v = v_chunks[c].repeat_interleave(hq // v_chunks[c].shape[1], dim=1)
        o, lse = sdpa_with_lse(q, k, v, is_causal=(c == q_chunk_index), scale=scale)
        os_.append(o.double().numpy())
        lses.append(lse.double().numpy())
    lse_stack = np.stack(lses)
    m = lse_stack.max(0)
    w = np.exp(lse_stack - m)
    s = w.sum(0)
    o = (w[..., None] * np.stack(os_)).sum(0) / s[..., None]
    return o, m + np.log(s)
