"""Seeded random sweep at medium sizes against the fp64 oracle on sampled rows.

The small-shape sweep (test_gpu_random_sweep.py) stays below 300 keys; these cases draw 64-4000 query rows
and 64-6000 keys, so they reach the persistent grouped-query kernel with several items per workgroup, the
stream-K form (non-causal calls whose items leave CUs idle, with the workspace the operator passes), the
key blocks of the wide heads and the ragged last tiles of long rows.  Each case checks the first and last
row and 24 random rows of every (batch, head): the causal rule over a row subset becomes an explicit mask,
as in tests/test_gpu_prefill_rows64.py.  Bars: max-abs 2e-2 on O, LSE |d| / max(|ref|, 1) <= 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(64))
def test_prefill_random_medium(seed):
    rng = np.random.default_rng(5000 + seed)
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(2))]
    D = int(rng.choice([128, 128, 128, 64, 256, 512]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    Hq = Hkv * int(rng.choice([1, 2, 3, 4, 8]))
    while Hq > 32:
        Hq //= 2
        Hkv = max(1, Hkv // 2)
        if Hq % Hkv:
            Hq = Hkv
    B = int(rng.integers(1, 4)) if Hq <= 8 else 1
    Sq, Sk = int(rng.integers(64, 4001)), int(rng.integers(64, 6001))
    causal = bool(rng.random() < 0.5)
    q_off = int(rng.integers(0, Sk)) if causal and rng.random() < 0.3 else 0
    print(f"medium seed={seed}: {dtype} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} causal={causal} "
          f"q_offset={q_off}", flush=True)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    import dtorch_amd.nn.functional as F
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                     is_causal=causal, enable_gqa=Hq != Hkv, q_offset=q_off)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, Sq - 1], rng.integers(0, Sq, 24)]))
    o, lse = host(o)[:, :, rows], host(lse)[:, :, rows]
    rq = rounded(q, dtype)[:, :, rows]
    if causal:
        mask = np.arange(Sk)[None, :] <= (rows[:, None] + q_off)
        ro, rl = orc.sdpa_fwd(rq, rounded(k, dtype), rounded(v, dtype), attn_mask=mask, enable_gqa=Hq != Hkv)
    else:
        ro, rl = orc.sdpa_fwd(rq, rounded(k, dtype), rounded(v, dtype), enable_gqa=Hq != Hkv)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL
