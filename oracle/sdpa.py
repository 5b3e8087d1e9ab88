"""fp64 NumPy restatement of DTorch's attention operator and the new LSE / decode / merge paths.

Test infrastructure: imported only by tests, smoke() and bench.py's cpu_baseline leg.

Semantics restated (reference paths relative to the reference repository root):

* ``SdpaOp::Compute`` (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:97-122)
  calls ``torch::scaled_dot_product_attention(q, k, v, mask, dropout=0.0, isCausal, scale,
  enableGqa)``.  That is ``O = softmax(scale * Q K^T + mask) V`` with

  - ``scale`` None -> 1/sqrt(E) (python/dtorch/nn/functional.py:191-200 passes it through),
  - ``is_causal`` -> keep key j for query i iff j <= i (top-left aligned ``tril(ones(L, S))``),
  - a boolean ``attn_mask`` keeps True entries, a float mask is added to the logits,
  - ``enable_gqa`` -> query head h reads kv head h // (Hq / Hkv), identical to the Llama port's
    ``repeat_kv`` expand+reshape (python/dtorch/test/modules/llama.py:80-85),
  - dropout is forced to 0.0 (scaled_dot_product_attention_op.cc:107-109, neural_network.cc:147-154).

* The output shape is q's shape with the last axis replaced by v's, same dtype as q
  (scaled_dot_product_attention_op.cc:16-32).

The per-row LSE, split-KV decode and LSE merge have no counterpart in the reference; they are
defined by their closed forms (LSE_i = log sum_j exp(scale q_i.k_j) over unmasked j; merge
LSE = m + log sum_b exp(LSE_b - m), O = sum_b exp(LSE_b - LSE) O_b).  ``q_offset``/``k_offset``
generalise the causal alignment: key j is visible to query i iff ``j + k_offset <= i + q_offset``
(0, 0 is torch's top-left alignment).  A query row that sees no key gets O = 0 and LSE = -inf, so
that it is a no-op in a merge.  The KV-cache append (``kv_append``, ``kv_append_paged``) is a copy into
the positions after each sequence's length; tests pin it by round trips (a sequence appended in pieces
equals the sequence, and decode over the appended cache equals causal attention over the full one).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

LOG2E = 1.4426950408889634
FP8_E4M3_MAX = 448.0


def _as64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def visible_mask(L: int, S: int, is_causal: bool, q_offset: int = 0, k_offset: int = 0) -> np.ndarray:
    """Boolean [L, S] keep-mask of the causal rule (torch's top-left alignment at offsets 0, 0).

    Restates ``tril(ones(L, S))`` of torch's causal SDPA, which SdpaOp::Compute reaches through
    scaled_dot_product_attention_op.cc:107-109, generalised by explicit offsets.
    """
    if not is_causal:
        return np.ones((L, S), dtype=bool)
    i = np.arange(L)[:, None] + q_offset
    j = np.arange(S)[None, :] + k_offset
    return j <= i


def expand_kv_heads(x: np.ndarray, hq: int) -> np.ndarray:
    """GQA head mapping: kv head h // (Hq/Hkv) serves query head h.

    Same as ``repeat_kv`` (python/dtorch/test/modules/llama.py:80-85): expand on a new axis after
    the head axis, then reshape, so each kv head is repeated for a contiguous group of query heads.
    """
    hkv = x.shape[-3]
    if hkv == hq:
        return x
    if hq % hkv != 0:
        raise ValueError(f"Hq={hq} is not a multiple of Hkv={hkv}")
    return np.repeat(x, hq // hkv, axis=-3)


def sdpa_fwd(
    q,
    k,
    v,
    attn_mask=None,
    is_causal: bool = False,
    scale: Optional[float] = None,
    enable_gqa: bool = False,
    q_offset: int = 0,
    k_offset: int = 0,
) -> Tuple[np.ndarray, np.ndarray]:
    """O and natural-log LSE of scaled dot-product attention, in float64.

    Follows SdpaOp::Compute (scaled_dot_product_attention_op.cc:97-122) and torch's SDPA contract
    described in the module docstring.  q: [..., Hq, L, E], k: [..., Hkv, S, E],
    v: [..., Hkv, S, Ev].  Returns O [..., Hq, L, Ev] and LSE [..., Hq, L].
    """
    q, k, v = _as64(q), _as64(k), _as64(v)
    hq, L, E = q.shape[-3:]
    S = k.shape[-2]
    if k.shape[-3] != hq or v.shape[-3] != hq:
        if not enable_gqa:
            raise ValueError("query and key/value head counts differ but enable_gqa is False")
        k = expand_kv_heads(k, hq)
        v = expand_kv_heads(v, hq)
    if scale is None:
        scale = 1.0 / math.sqrt(E)
    logits = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    keep = np.broadcast_to(visible_mask(L, S, is_causal, q_offset, k_offset), logits.shape)
    if attn_mask is not None:
        m = np.asarray(attn_mask)
        if m.dtype == bool:
            keep = keep & np.broadcast_to(m, logits.shape)
        else:
            logits = logits + m.astype(np.float64)
    logits = np.where(keep, logits, -np.inf)
    mx = np.max(logits, axis=-1, keepdims=True, initial=-np.inf)  # an empty key set is fully masked
    mx_safe = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(logits - mx_safe)
    l = np.sum(p, axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        o = np.where(l > 0, np.matmul(p, v) / np.where(l > 0, l, 1.0), 0.0)
        lse = np.where(l[..., 0] > 0, mx_safe[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)), -np.inf)
    return o, lse


def decode(q, k_cache, v_cache, lengths, scale: Optional[float] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Single-token decode over a padded per-sequence KV cache.

    New path (no reference function).  Defined as SdpaOp::Compute's arithmetic
    (scaled_dot_product_attention_op.cc:107-109) with Lq = 1, is_causal = False, GQA enabled,
    restricted to each sequence's true length: q [B, Hq, 1, D], caches [B, Hkv, S_max, D],
    lengths [B].  Rows past lengths[b] are never read.
    """
    q = _as64(q)
    B = q.shape[0]
    outs, lses = [], []
    for b in range(B):
        L = int(lengths[b])
        o, lse = sdpa_fwd(q[b], k_cache[b, :, :L], v_cache[b, :, :L], scale=scale, enable_gqa=True)
        outs.append(o)
        lses.append(lse)
    return np.stack(outs), np.stack(lses)


def gather_pages(pages, block_table, lengths, max_len: Optional[int] = None) -> np.ndarray:
    """Contiguous [B, Hkv, S, D] cache rebuilt from a paged one: token t of sequence b is row
    t % page_size of page block_table[b, t // page_size] in pages [num_pages, Hkv, page_size, D].
    Rows at or past lengths[b] are left zero and never looked up."""
    pages = np.asarray(pages)
    _, hkv, ps, d = pages.shape
    B = len(lengths)
    S = int(max_len if max_len is not None else max(int(x) for x in lengths))
    out = np.zeros((B, hkv, S, d), dtype=pages.dtype)
    for b in range(B):
        for t in range(int(lengths[b])):
            out[b, :, t] = pages[int(block_table[b][t // ps]), :, t % ps]
    return out


def decode_paged(q, k_pages, v_pages, block_table, lengths, scale: Optional[float] = None):
    """Single-token decode over a paged KV cache: ``decode`` on the cache that ``gather_pages``
    rebuilds (new path, no reference function)."""
    kc = gather_pages(k_pages, block_table, lengths)
    vc = gather_pages(v_pages, block_table, lengths)
    return decode(q, kc, vc, lengths, scale=scale)


def kv_append(cache, lengths, new):
    """KV-cache append (new path, no reference function: the reference keeps no cache,
    python/dtorch/test/modules/llama.py:126-156).  cache [B, H, S_max, D] and lengths [B] are updated in
    place: token j of sequence b goes to position max(lengths[b], 0) + j unless that is >= S_max, then
    lengths[b] = min(max(lengths[b], 0) + n_new, S_max).  new is [B, H, n_new, D]."""
    s_max = cache.shape[2]
    n_new = new.shape[2]
    for b in range(cache.shape[0]):
        t0 = max(int(lengths[b]), 0)
        n = max(0, min(n_new, s_max - t0))
        cache[b, :, t0:t0 + n] = new[b, :, :n]
        lengths[b] = min(t0 + n_new, s_max)


def kv_append_paged(pages, block_table, lengths, new):
    """kv_append for a paged cache: position t of sequence b is row t % page_size of page
    block_table[b, t // page_size] in pages [num_pages, H, page_size, D]; the capacity is
    max_pages * page_size.  A token whose table entry is not a page of the pool (below 0 or at least
    num_pages: an unassigned slot) is dropped, and the length advances as for a written one.  pages and
    lengths are updated in place."""
    num_pages, _, ps, _ = pages.shape
    cap = block_table.shape[1] * ps
    n_new = new.shape[2]
    for b in range(block_table.shape[0]):
        t0 = max(int(lengths[b]), 0)
        for j in range(n_new):
            t = t0 + j
            if t >= cap:
                break
            page = int(block_table[b, t // ps])
            if 0 <= page < num_pages:
                pages[page, :, t % ps] = new[b, :, j]
        lengths[b] = min(t0 + n_new, cap)


def lse_merge(os: Sequence[np.ndarray], lses: Sequence[np.ndarray]) -> Tuple[np.ndarray, np.ndarray]:
    """Merge partial attention blocks by their log-sum-exp (closed form, no reference function).

    With m = max_b LSE_b: LSE = m + log sum_b exp(LSE_b - m), O = sum_b exp(LSE_b - LSE) O_b.
    A block whose LSE is -inf contributes nothing; rows where every block is -inf give O = 0,
    LSE = -inf.
    """
    lse_stack = np.stack([_as64(x) for x in lses])
    o_stack = np.stack([_as64(x) for x in os])
    m = np.max(lse_stack, axis=0)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    w = np.exp(lse_stack - m_safe)
    s = np.sum(w, axis=0)
    with np.errstate(divide="ignore"):
        lse = np.where(s > 0, m_safe + np.log(np.where(s > 0, s, 1.0)), -np.inf)
    wn = np.where(s > 0, w / np.where(s > 0, s, 1.0), 0.0)
    o = np.sum(wn[..., None] * o_stack, axis=0)
    return o, lse


def ring_step(q, k_chunks, v_chunks, q_chunk_index: int, scale: Optional[float] = None, enable_gqa: bool = True):
    """One device's share of causal ring attention: per-block O + LSE, then the LSE merge.

    The reference's "ring" all-gathers K/V and runs one local SDPA
    (python/dtorch/nn/scaled_dot_product_attention_with_cp.py:87-101); this is the blockwise form
    of the same result.  The Q chunk has global index ``q_chunk_index``; KV chunk c < index is fully
    visible, c == index is the causal diagonal (Lq == Lk, top-left), chunks after it are skipped.
    Returns (per-block list of (O_b, LSE_b), merged O, merged LSE).
    """
    blocks = []
    for c in range(len(k_chunks)):
        if c > q_chunk_index:
            continue
        o, lse = sdpa_fwd(q, k_chunks[c], v_chunks[c], is_causal=(c == q_chunk_index), scale=scale,
                          enable_gqa=enable_gqa)
        blocks.append((o, lse))
    o, lse = lse_merge([b[0] for b in blocks], [b[1] for b in blocks])
    return blocks, o, lse


# ---------------------------------------------------------------------------------------------
# OCP fp8 e4m3fn (1 sign, 4 exponent bits, bias 7, 3 mantissa bits, no infinities, 0x7f/0xff NaN,
# max finite 448).  Replaces the reference's third-party quantized branch
# (dtorch/external/sage_attn/sage_attn_adapter.cc:28-158), which has no fp8 e4m3fn path of its own.
# ---------------------------------------------------------------------------------------------

def e4m3fn_encode(x) -> np.ndarray:
    """Round float32 values to e4m3fn codes (uint8), round-to-nearest-even, saturating to +-448.

    Finite values above 448 in magnitude saturate (the quantizer never produces NaN for finite
    input); NaN maps to 0x7f.  Subnormals have step 2^-9.
    """
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    a = np.abs(x)
    nan = np.isnan(a)
    a = np.where(nan, 0.0, np.minimum(a, FP8_E4M3_MAX))
    # exponent of the fp8 grid that contains a: normals have e >= -6, below that the subnormal step
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.clip(e, -6, 8)
    step = np.exp2(e - 3)
    # np.round is round-half-to-even, which is RNE on the scaled mantissa (exact in float64)
    q = np.round(a / step) * step
    q = np.minimum(q, FP8_E4M3_MAX)
    # re-derive exponent after rounding (mantissa overflow bumps the exponent)
    with np.errstate(divide="ignore"):
        e2 = np.floor(np.log2(np.where(q > 0, q, 1.0)))
    normal = q >= 2.0 ** -6
    exp_field = np.where(normal, e2 + 7, 0).astype(np.int64)
    mant = np.where(normal, q / np.exp2(e2) - 1.0, q / 2.0 ** -9) * np.where(normal, 8, 1)
    mant = np.rint(mant).astype(np.int64)
    code = (exp_field << 3) | mant
    code = np.where(q == 0, 0, code)
    out = sign | code.astype(np.uint8)
    out = np.where(nan, np.uint8(0x7F), out).astype(np.uint8)
    return out


def e4m3fn_decode(codes) -> np.ndarray:
    """Decode e4m3fn codes (uint8) to float64."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return s * val


def fp8_quantize_per_head(x) -> Tuple[np.ndarray, np.ndarray]:
    """Per-head absmax quantization to e4m3fn, as the fp8 prefill path defines it.

    x: [B, H, S, D] (any float dtype; computed in float32 like the kernel).  For each (b, h):
    ``amax = max|x|``; ``inv = float32(448 / amax)`` (amax == 0 -> inv = 1); codes =
    e4m3fn(float32(x * inv)); ``descale = float32(amax / 448)`` (amax == 0 -> 1).  Returns
    (codes uint8 [B, H, S, D], descale float32 [B, H]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=(-2, -1)).astype(np.float32)
    safe = amax > 0
    inv = np.where(safe, np.float32(FP8_E4M3_MAX) / np.where(safe, amax, np.float32(1)), np.float32(1)).astype(np.float32)
    descale = np.where(safe, amax / np.float32(FP8_E4M3_MAX), np.float32(1)).astype(np.float32)
    y = (x * inv[..., None, None]).astype(np.float32)
    return e4m3fn_encode(y), descale


def fp8_dequantize_per_head(codes, descale) -> np.ndarray:
    return e4m3fn_decode(codes) * np.asarray(descale, dtype=np.float64)[..., None, None]


# ---------------------------------------------------------------------------------------------
# Cost models
# ---------------------------------------------------------------------------------------------

def reference_cost_flops(q_shape, k_shape, v_shape) -> int:
    """SdpaOp::GetOperatorCost: 2 * batch * qHeads * seqQ * seqKv * (headDim + Ev), mask ignored.

    Restates scaled_dot_product_attention_op.cc:68-95; pinned by
    dtorch/tests/test_operator_cost.cc:171-183 (Q [2,8,16,64], K/V [2,8,20,64] -> 1,310,720).
    """
    batch = int(np.prod(q_shape[:-3])) if len(q_shape) > 3 else 1
    hq, sq, d = q_shape[-3:]
    skv = k_shape[-2]
    ev = v_shape[-1]
    return 2 * batch * hq * sq * skv * (d + ev)


def causal_pairs(L: int, S: int, q_offset: int = 0, k_offset: int = 0) -> int:
    """Number of visible (query, key) pairs under the causal rule (diagonal included)."""
    i = np.arange(L, dtype=np.int64) + q_offset - k_offset
    return int(np.sum(np.clip(i + 1, 0, S)))


def algorithmic_flops(B, Hq, L, S, D, Dv, is_causal, q_offset=0, k_offset=0) -> int:
    """Useful FLOPs: 2 * (D + Dv) per visible (query, key) pair per (batch, query head)."""
    pairs = causal_pairs(L, S, q_offset, k_offset) if is_causal else L * S
    return 2 * (D + Dv) * B * Hq * pairs
