"""Long contexts: a 64K-token causal GQA prefill and a 128K-token decode against the oracle.

At these lengths the index arithmetic of the kernels runs over its whole range (tile offsets into
64K-row slabs, split grids of 512 chunks per sequence).  The oracle is evaluated on sampled query rows:
row i of a causal prefill is the oracle's causal attention of q[i:i+1] with q_offset = i over all keys,
the same visibility rule the kernels apply.  Tolerances as for every bf16 case: max-abs 2e-2 on O,
LSE |d| / max(|ref|, 1) <= 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, rounded

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def test_prefill_causal_gqa_64k_sampled_rows():
    B, Hq, Hkv, S, D = 1, 8, 1, 65536, 128
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(B, Hq, S, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(torch.bfloat16)
    o, lse = _F().scaled_dot_product_attention_with_lse(q, k, v, is_causal=True, enable_gqa=True)
    torch.cuda.synchronize()
    kh, vh = host(k), host(v)
    rows = [0, 1, 63, 64, 127, 128, 4095, 32768, 40000, 65407, 65408, 65535]
    for i in rows:
        ro, rl = orc.sdpa_fwd(host(q[:, :, i:i + 1]), kh[:, :, :i + 1], vh[:, :, :i + 1], is_causal=True,
                              enable_gqa=True, q_offset=i)
        assert max_abs(host(o[:, :, i:i + 1]), ro) <= O_TOL_BF16, i
        assert lse_rel(host(lse[:, :, i:i + 1]), rl) <= LSE_TOL, i


def test_decode_128k_context():
    rng = np.random.default_rng(8)
    B, Hq, Hkv, Smax, D = 2, 8, 1, 131072, 128
    q = rng.standard_normal((B, Hq, 1, D), dtype=np.float32)
    g = torch.Generator(device="cuda").manual_seed(9)
    kc = torch.randn(B, Hkv, Smax, D, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, Smax, D, device="cuda", generator=g).to(torch.bfloat16)
    lengths = np.array([131072, 70001], dtype=np.int32)
    kc[1, :, 70001:] = float("nan")  # padding is never read
    vc[1, :, 70001:] = float("nan")
    o, lse = _F().decode_attention(torch.from_numpy(rounded(q)).to(torch.bfloat16).cuda(), kc, vc,
                                   torch.from_numpy(lengths).cuda())
    torch.cuda.synchronize()
    ro, rl = orc.decode(rounded(q), np.nan_to_num(host(kc)), np.nan_to_num(host(vc)), lengths)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl[..., 0]) <= LSE_TOL
