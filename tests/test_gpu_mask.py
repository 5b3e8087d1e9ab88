"""GPU parity of the masked prefill (attn_mask) against the oracle."""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _run(q, k, v, mask_dev, mask_ref, causal=False, dtype=torch.bfloat16, scale=None):
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                     is_causal=causal, enable_gqa=True, scale=scale,
                                                     attn_mask=mask_dev)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), attn_mask=mask_ref,
                          is_causal=causal, enable_gqa=True, scale=scale)
    return host(o), host(lse), ro, rl


def test_bool_mask_broadcast_gqa_ragged():
    rng = np.random.default_rng(51)
    B, Hq, Hkv, L, S, D = 2, 8, 2, 200, 333, 128
    q, k, v = randn(rng, (B, Hq, L, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    keep = rng.random((L, S)) < 0.5
    keep[np.arange(L), rng.integers(0, S, size=L)] = True  # every row keeps some key
    o, lse, ro, rl = _run(q, k, v, torch.from_numpy(keep).cuda(), keep)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_hf_additive_mask_with_causal():
    # HF-style padding mask [B, 1, L, S]: 0 where visible, the dtype minimum on padded keys, plus is_causal
    rng = np.random.default_rng(52)
    B, H, L, D = 3, 4, 160, 128
    q, k, v = randn(rng, (B, H, L, D)), randn(rng, (B, H, L, D)), randn(rng, (B, H, L, D))
    pad = np.array([0, 37, 100])  # leading padded keys per sequence (left padding)
    m = np.zeros((B, 1, L, L), dtype=np.float32)
    for b in range(B):
        m[b, :, :, :pad[b]] = torch.finfo(torch.bfloat16).min
    tm = torch.from_numpy(m).to(torch.bfloat16).cuda()
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), is_causal=True,
                                                     attn_mask=tm)
    torch.cuda.synchronize()
    o, lse = host(o), host(lse)
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), attn_mask=m.astype(np.float64), is_causal=True)
    # rows whose every visible key is padded (row i < pad[b]) are fully hidden: the kernels give O = 0 and
    # LSE = -inf there (torch would spread them over the padded keys); compare the others
    for b in range(B):
        rows = slice(pad[b], L)
        assert max_abs(o[b, :, rows], ro[b, :, rows]) <= O_TOL_BF16, b
        assert lse_rel(lse[b, :, rows], rl[b, :, rows]) <= LSE_TOL, b
        assert np.all(o[b, :, :pad[b]] == 0) and np.all(np.isneginf(lse[b, :, :pad[b]])), b


def test_clip_style_causal_additive_mask_d64_odd_pitch():
    # CLIP text: 77 tokens, a causal mask passed as an additive float mask (row pitch 77 -> padded copy)
    rng = np.random.default_rng(53)
    B, H, L, D = 2, 8, 77, 64
    q, k, v = randn(rng, (B, H, L, D)), randn(rng, (B, H, L, D)), randn(rng, (B, H, L, D))
    m = np.triu(np.full((L, L), -np.inf, dtype=np.float32), k=1)[None, None]
    o, lse, ro, rl = _run(q, k, v, torch.from_numpy(m).expand(B, 1, L, L).cuda(), m)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_fp16_per_head_bias_fp32():
    rng = np.random.default_rng(54)
    B, H, L, S, D = 1, 4, 96, 130, 128
    q, k, v = randn(rng, (B, H, L, D)), randn(rng, (B, H, S, D)), randn(rng, (B, H, S, D))
    bias = (rng.standard_normal((1, H, L, S)) * 2).astype(np.float32)
    o, lse, ro, rl = _run(q, k, v, torch.from_numpy(bias).cuda(), bias.astype(np.float64), dtype=torch.float16,
                          scale=0.05)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_fully_masked_rows_and_errors():
    rng = np.random.default_rng(55)
    B, H, L, S, D = 1, 2, 64, 64, 128
    q, k, v = randn(rng, (B, H, L, D)), randn(rng, (B, H, S, D)), randn(rng, (B, H, S, D))
    keep = np.ones((L, S), dtype=bool)
    keep[5] = False
    o, lse, ro, rl = _run(q, k, v, torch.from_numpy(keep).cuda(), keep)
    assert np.all(o[:, :, 5] == 0) and np.all(np.isneginf(lse[:, :, 5]))
    assert max_abs(o, ro) <= O_TOL_BF16
    F = _F()
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    with pytest.raises(ValueError, match="broadcast"):
        F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.ones(3, S, dtype=torch.bool, device="cuda"))
    with pytest.raises(ValueError, match="native_fp8"):
        F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(keep).cuda(),
                                       sdpa_option=F.SdpaOption(sage_attn_type="native_fp8"))
