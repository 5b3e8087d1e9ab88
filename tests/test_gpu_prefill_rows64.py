"""GPU parity of the 64-rows-per-wave prefill (head dim 128, no mask, no padding) against the fp64 oracle.

Two layouts take these calls: grouped-query calls with groups of 4k heads and a positive scale run the
persistent kernel whose 4 waves are 4 query heads over the same rows (work items dealt to XCDs when
B*Hkv is a multiple of 8, several items per workgroup when there are more items than CUs); the rest run
64 consecutive rows per wave.  Both are checked here on the shapes where their bookkeeping differs: ragged
Sq and Sk, causal offsets of either sign (rows that see no key: O = 0, LSE = -inf), item counts below and
above the CU count, strided layouts, and a negative scale (which takes the rows layout).  Bar: max-abs 2e-2
on O, LSE |d| / max(|ref|, 1) <= 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _check(B, Hq, Hkv, Sq, Sk, causal, dtype=torch.bfloat16, seed=0, q_offset=0, k_offset=0, scale=None,
           rows=None):
    rng = np.random.default_rng(seed)
    q, k, v = randn(rng, (B, Hq, Sq, 128)), randn(rng, (B, Hkv, Sk, 128)), randn(rng, (B, Hkv, Sk, 128))
    o, lse = _F().scaled_dot_product_attention_with_lse(
        to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), is_causal=causal, enable_gqa=Hq != Hkv,
        q_offset=q_offset, k_offset=k_offset, scale=scale)
    torch.cuda.synchronize()
    o, lse = host(o), host(lse)
    rq = rounded(q, dtype)
    if rows is not None:  # a row subset: the causal rule becomes an explicit mask over those rows
        rq, o, lse = rq[:, :, rows], o[:, :, rows], lse[:, :, rows]
    if rows is not None and causal:
        qi = np.asarray(rows)[:, None] + q_offset
        kj = np.arange(Sk)[None, :] + k_offset
        mask = kj <= qi
        ro, rl = orc.sdpa_fwd(rq, rounded(k, dtype), rounded(v, dtype), attn_mask=mask, enable_gqa=Hq != Hkv,
                              scale=scale)
    else:
        ro, rl = orc.sdpa_fwd(rq, rounded(k, dtype), rounded(v, dtype), is_causal=causal, enable_gqa=Hq != Hkv,
                              q_offset=q_offset, k_offset=k_offset, scale=scale)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL
    return o, lse, rl


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,causal,dtype", [
    (1, 4, 1, 700, 700, True, torch.bfloat16),     # GQA 4, one kv head (no XCD map), ragged
    (2, 8, 2, 333, 901, False, torch.bfloat16),    # GQA 4, Sq != Sk
    (1, 8, 1, 260, 260, True, torch.float16),      # GQA 8: two 4-head subgroups per kv head, fp16
    (2, 32, 4, 200, 200, True, torch.bfloat16),    # B*Hkv = 8: items dealt to XCDs, fewer items than CUs
    (4, 32, 8, 1000, 1000, True, torch.float16),   # XCD map, more items than CUs (several per workgroup)
    (1, 4, 4, 300, 500, True, torch.bfloat16),     # MHA: rows layout, causal
    (2, 6, 6, 190, 190, False, torch.float16),     # MHA: rows layout, non-causal
    (1, 6, 3, 129, 129, True, torch.bfloat16),     # GQA 2: rows layout
])
def test_rows64_layouts(B, Hq, Hkv, Sq, Sk, causal, dtype):
    _check(B, Hq, Hkv, Sq, Sk, causal, dtype, seed=Sq + Hq)


@pytest.mark.parametrize("q_offset,k_offset", [(300, 0), (0, 150), (37, 5)])
def test_rows64_gqa_causal_offsets(q_offset, k_offset):
    # j + k_offset <= i + q_offset; with k_offset > q_offset the first rows see no key at all
    o, lse, rl = _check(1, 8, 2, 257, 555, True, seed=q_offset + k_offset, q_offset=q_offset, k_offset=k_offset)
    hidden = np.isneginf(rl)
    assert np.array_equal(np.isneginf(lse), hidden)
    assert np.all(o[np.broadcast_to(hidden[..., None], o.shape)] == 0)


def test_rows64_negative_scale_takes_the_rows_layout():
    # a negative scale runs as |scale| on negated q: the persistent layout loads q untransformed, so this call
    # goes to the rows layout; both must agree with the oracle
    _check(1, 8, 2, 300, 300, True, seed=9, scale=-0.05)
    _check(1, 8, 2, 300, 300, False, seed=10, scale=0.2)


def test_rows64_without_lse_and_single_row():
    F = _F()
    rng = np.random.default_rng(11)
    q, k, v = randn(rng, (2, 8, 1, 128)), randn(rng, (2, 2, 77, 128)), randn(rng, (2, 2, 77, 128))
    o = F.scaled_dot_product_attention(to_dev(q), to_dev(k), to_dev(v), enable_gqa=True)
    o2, _ = F.scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), enable_gqa=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    ro, _ = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), enable_gqa=True)
    assert max_abs(host(o), ro) <= O_TOL_BF16


def test_rows64_strided_bshd_layout():
    # [B, S, H, D] storage viewed as [B, H, S, D]: row pitches of H*D elements
    rng = np.random.default_rng(12)
    B, Hq, Hkv, S = 2, 8, 2, 400
    qs, ks, vs = randn(rng, (B, S, Hq, 128)), randn(rng, (B, S, Hkv, 128)), randn(rng, (B, S, Hkv, 128))
    tq, tk, tv = (to_dev(x).transpose(1, 2) for x in (qs, ks, vs))
    o, lse = _F().scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=True, enable_gqa=True)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(*(rounded(x).transpose(0, 2, 1, 3) for x in (qs, ks, vs)), is_causal=True,
                          enable_gqa=True)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


def test_rows64_gqa_long_context_sampled_rows():
    # 8 items per CU-slot on the persistent grid: every 64-row item's first and last row of each head
    S = 4096
    rows = np.sort(np.concatenate([np.arange(0, S, 64), np.arange(63, S, 64)]))
    _check(2, 16, 4, S, S, True, seed=13, rows=rows)
