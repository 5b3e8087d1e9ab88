"""Python front end of the MI355X attention path.

Mirrors ``dtorch.nn.functional.scaled_dot_product_attention`` and ``SdpaOption``
(python/dtorch/nn/functional.py:169-238) on local torch device tensors: same signature, same
defaults, same validation; the call lands in the C++ ``SdpaOp`` host operator, whose ``Compute``
launches the gfx950 kernels through the dtattn C ABI on the current HIP stream.

New entry points (no reference counterpart, see the host operators):
``scaled_dot_product_attention_with_lse``, ``decode_attention``, ``lse_merge``,
``ring_attention_step`` and ``quantize_fp8_per_head``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import torch

from .._lib import load

_h = load()

_SAGE_TYPES = ("auto", "qk_int8_pv_fp8", "qk_int8_pv_fp16")


@dataclass
class SdpaOption:
    """Per-call attention options (python/dtorch/nn/functional.py:169-188).

    ``sage_attn_type`` keeps the reference's candidates ("", "auto", "qk_int8_pv_fp8",
    "qk_int8_pv_fp16") and adds ``"native_fp8"``: per-head absmax e4m3fn quantization of q/k/v and
    fp8 MFMA for both products, bf16 output.
    """

    # cp
    ulysess_cp_dim: Optional[Union[int, str]] = "ulysess_cp"
    ring_cp_dim: Optional[Union[int, str]] = "ring_cp"

    # candidate: "", "auto", "qk_int8_pv_fp8", "qk_int8_pv_fp16", "native_fp8"
    sage_attn_type: Optional[str] = None

    def check_valid(self):
        return self.sage_attn_type in (None, "", "native_fp8") + _SAGE_TYPES


def _param(is_causal: bool, scale: Optional[float], enable_gqa: bool, sdpa_option: SdpaOption):
    return _h.SdpaParam(bool(is_causal), None if scale is None else float(scale), bool(enable_gqa),
                        _h.SdpaOption(sdpa_option.sage_attn_type or ""))


def _check_option(query, sdpa_option: SdpaOption):
    assert sdpa_option.check_valid(), f"sdpa_option invalid: {sdpa_option}"
    if sdpa_option.sage_attn_type in _SAGE_TYPES:
        # python/dtorch/nn/functional.py:216-220
        try:
            import sageattention  # noqa: F401
        except ImportError:
            raise RuntimeError("Require sageattention, please install sageattention.")
    mesh = getattr(query, "device_mesh", None)
    if (isinstance(sdpa_option.ulysess_cp_dim, int) or isinstance(sdpa_option.ring_cp_dim, int) or
            (mesh is not None and (mesh.has_dim_name(sdpa_option.ulysess_cp_dim or "") or
                                   mesh.has_dim_name(sdpa_option.ring_cp_dim or "")))):
        raise NotImplementedError(
            "context parallelism across devices is not part of this single-GPU build; "
            "ring_attention_step() computes one device's share")


def scaled_dot_product_attention(
    query: torch.Tensor,  # N, Hq, L, E
    key: torch.Tensor,  # N, H, S, E
    value: torch.Tensor,  # N, H, S, E
    attn_mask=None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    scale: Optional[float] = None,
    enable_gqa=False,
    sdpa_option: SdpaOption = SdpaOption(),
) -> torch.Tensor:
    """O = softmax(scale Q K^T [causal, top-left]) V on the gfx950 kernels.

    ``dropout_p`` is accepted and ignored, as in the reference (neural_network.cc:147-154 drops it and
    SdpaOp::Compute passes 0.0).  ``attn_mask`` follows torch: broadcastable to [..., Hq, L, S], boolean
    (True keeps a key) or floating point (added to the scaled logits), applied together with ``is_causal``;
    not supported with ``native_fp8``.
    """
    _check_option(query, sdpa_option)
    op = _h.SdpaOp(_param(is_causal, scale, enable_gqa, sdpa_option))
    return op.compute([query, key, value, attn_mask])[0]


def scaled_dot_product_attention_with_lse(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    is_causal: bool = False,
    scale: Optional[float] = None,
    enable_gqa: bool = False,
    q_offset: int = 0,
    k_offset: int = 0,
    sdpa_option: SdpaOption = SdpaOption(),
    attn_mask: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE[..., Hq, L] fp32).  Causal rule: key j visible to query i iff j + k_offset <= i + q_offset.
    ``attn_mask`` as in scaled_dot_product_attention, applied together with the causal rule."""
    _check_option(query, sdpa_option)
    op = _h.SdpaWithLseOp(_param(is_causal, scale, enable_gqa, sdpa_option), int(q_offset), int(k_offset))
    o, lse = op.compute([query, key, value, attn_mask])
    return o, lse


def decode_attention(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor,
                     scale: Optional[float] = None, chunk: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Single-token attention per sequence over k_cache[b, :, :lengths[b]] (split-KV + LSE merge).

    query [B, Hq, 1, D]; caches [B, Hkv, S_max, D]; lengths int32 [B] on the device.
    Returns (O [B, Hq, 1, D], LSE [B, Hq] fp32).
    """
    op = _h.SdpaDecodeOp(None if scale is None else float(scale), int(chunk))
    o, lse = op.compute([query, k_cache, v_cache, lengths])
    return o, lse


def decode_attention_paged(query: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                           block_table: torch.Tensor, lengths: torch.Tensor, scale: Optional[float] = None,
                           chunk: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """decode_attention over a paged KV cache.

    query [B, Hq, 1, D]; k_pages / v_pages are page pools viewed as [num_pages, Hkv, page_size, D]
    (any strides with unit stride on D, so a [num_pages, page_size, Hkv, D] pool passed through
    .permute(0, 2, 1, 3) works without a copy); block_table int32 [B, max_pages] holds the page of
    each sequence's p-th block; lengths int32 [B].  page_size is a power of two >= 16.
    Returns (O [B, Hq, 1, D], LSE [B, Hq] fp32).
    """
    op = _h.SdpaDecodePagedOp(None if scale is None else float(scale), int(chunk))
    o, lse = op.compute([query, k_pages, v_pages, block_table, lengths])
    return o, lse


def kv_cache_append(k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor, k_new: torch.Tensor,
                    v_new: torch.Tensor) -> None:
    """Write n_new tokens per sequence into a [B, Hkv, S_max, D] cache, in place.

    k_new / v_new are [B, Hkv, n_new, D] (any strides with unit stride on D, e.g. a transposed projection
    output).  Token j of sequence b lands at position lengths[b] + j; positions at or past S_max are not
    written.  lengths (contiguous int32 [B]) then advances by n_new, saturating at S_max.
    """
    _h.KvCacheAppendOp().compute([k_cache, v_cache, lengths, k_new, v_new])


def kv_cache_append_paged(k_pages: torch.Tensor, v_pages: torch.Tensor, block_table: torch.Tensor,
                          lengths: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
    """kv_cache_append for the paged cache of decode_attention_paged; the block table must already name
    the pages of the positions being written."""
    _h.KvCacheAppendPagedOp().compute([k_pages, v_pages, block_table, lengths, k_new, v_new])


def lse_merge(outs: Sequence[torch.Tensor], lses: Sequence[torch.Tensor],
              out_dtype: Optional[torch.dtype] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merge partial attention blocks over the same queries by their LSE."""
    if len(outs) != len(lses) or not outs:
        raise ValueError("lse_merge needs matching, non-empty lists of outputs and LSEs")
    ins: List[Optional[torch.Tensor]] = []
    for o, l in zip(outs, lses):
        ins += [o, l]
    return tuple(_h.LseMergeOp(out_dtype).compute(ins))


def ring_attention_step(query: torch.Tensor, k_chunks: Sequence[torch.Tensor], v_chunks: Sequence[torch.Tensor],
                        q_chunk_index: int, scale: Optional[float] = None, enable_gqa: bool = True,
                        return_blocks: bool = False):
    """One device's share of causal ring attention over equal-length sequence chunks.

    The Q chunk has global chunk index ``q_chunk_index``; KV chunk c is visible in full when
    c < q_chunk_index, causally (diagonal, offsets equal) when c == q_chunk_index, and not at all
    after.  Each visible block yields (O_c, LSE_c) with global offsets; the blocks are then merged by
    LSE.  This is the per-step arithmetic a true ring needs (the reference all-gathers K/V instead:
    python/dtorch/nn/scaled_dot_product_attention_with_cp.py:87-101).
    """
    L = query.shape[-2]
    blocks = []
    for c in range(min(q_chunk_index + 1, len(k_chunks))):
        diag = c == q_chunk_index
        o, lse = scaled_dot_product_attention_with_lse(
            query, k_chunks[c], v_chunks[c], is_causal=diag, scale=scale, enable_gqa=enable_gqa,
            q_offset=q_chunk_index * L, k_offset=c * k_chunks[c].shape[-2])
        blocks.append((o, lse))
    o, lse = lse_merge([b[0] for b in blocks], [b[1] for b in blocks])
    if return_blocks:
        return o, lse, blocks
    return o, lse


def quantize_fp8_per_head(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-head absmax e4m3fn quantization: (codes float8_e4m3fn [..., H, S, D], descale fp32 [..., H])."""
    codes, desc = _h.Fp8QuantizeOp().compute([x])
    return codes, desc


def device_peaks(device: int = 0):
    """MI355X peak table (CU count x clock x CDNA4 per-CU MFMA rate; HBM 8 TB/s)."""
    return _h.get_device_peaks(device)
