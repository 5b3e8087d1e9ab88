"""Seeded random configurations of the prefill against the fp64 oracle.

Each case draws a dtype (bf16, fp16, fp32), a head dim (64, 128, and 256 / 512 for the 16-bit types), GQA
group, batch, ragged Sq and Sk, causal flag with causal offsets, and sometimes an attention mask, from a
fixed seed, so the set is the same on every run.  Bars: max-abs 2e-2 (bf16/fp16) or 1e-5 (fp32) on O,
LSE |d| / max(|ref|, 1) <= 1e-3 (1e-5 for fp32), on rows that see at least one key.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _draw(i):
    rng = np.random.default_rng(1000 + i)
    dtype = DTYPES[rng.integers(0, 3)]
    D = [64, 128][i % 2] if dtype == torch.float32 else [64, 128, 256, 512][i % 4]
    Hkv = int(rng.integers(1, 4))
    group = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 3))
    Sq = int(rng.integers(1, 400))
    Sk = int(rng.integers(1, 400))
    causal = bool(rng.integers(0, 2))
    q_off = int(rng.integers(0, 200)) if causal and rng.random() < 0.4 else 0
    masked = rng.random() < 0.3
    return rng, dtype, D, Hkv, group, B, Sq, Sk, causal, q_off, masked


@pytest.mark.parametrize("i", range(32))
def test_random_prefill_config(i):
    rng, dtype, D, Hkv, group, B, Sq, Sk, causal, q_off, masked = _draw(i)
    Hq = Hkv * group
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    mask = None
    if masked:
        mask = rng.random((Sq, Sk)) < 0.7
    import dtorch_amd.nn.functional as F
    o, lse = F.scaled_dot_product_attention_with_lse(
        to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), is_causal=causal, enable_gqa=group > 1,
        q_offset=q_off, attn_mask=None if mask is None else torch.from_numpy(mask).cuda())
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), attn_mask=mask, is_causal=causal,
                          enable_gqa=group > 1, q_offset=q_off)
    o, lse = host(o), host(lse)
    seen = np.isfinite(rl)  # rows with at least one visible key
    hidden = ~seen
    assert np.all(o[hidden] == 0), (dtype, D, causal, masked)
    assert np.all(np.isneginf(lse[hidden]))
    tol_o = 1e-5 if dtype == torch.float32 else O_TOL_BF16
    tol_l = 1e-5 if dtype == torch.float32 else LSE_TOL
    if seen.any():
        assert max_abs(o[seen], ro[seen]) <= tol_o, (dtype, D, B, Hq, Hkv, Sq, Sk, causal, q_off, masked)
        assert lse_rel(lse[seen], rl[seen]) <= tol_l, (dtype, D, B, Hq, Hkv, Sq, Sk, causal, q_off, masked)
