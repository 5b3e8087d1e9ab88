"""The DTorch integration adapter on the GPU (integration/tree/dtorch/external/dtattn/dtattn_adapter.cc, the file
the integration patch adds to a DTorch tree; built in-tree as tests/integration_adapter/_adapter_check).

Its argument fills are held against the product path (the host operators, which drive the same kernels:
bit-identical results) and, where it reshapes the call itself (head dims padded to a multiple of 8, a rank-5
batch, a broadcast boolean mask), against the oracle at the usual tolerances.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _A():
    import dtorch_amd  # noqa: F401  (loads torch's HIP runtime first)
    from tests.integration_adapter import _adapter_check as A
    return A


def _F():
    import dtorch_amd.nn.functional as F
    return F


def test_sdpa_branch_equals_the_product_path():
    A, F = _A(), _F()
    rng = np.random.default_rng(71)
    q, k, v = (to_dev(randn(rng, (2, h, 300, 128))) for h in (8, 2, 2))
    print("adapter: causal GQA 2x8/2x300x128 bf16", flush=True)
    o = A.sdpa(q, k, v, None, True, None, True, "")
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    mask = torch.from_numpy(rng.random((300, 300)) < 0.6).cuda()
    o = A.sdpa(q, k, v, mask, False, 0.07, True, "")
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=0.07, enable_gqa=True)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    opt = F.SdpaOption(sage_attn_type="native_fp8")
    o = A.sdpa(q, k, v, None, False, None, True, "native_fp8")
    ref = F.scaled_dot_product_attention(q, k, v, enable_gqa=True, sdpa_option=opt)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    with pytest.raises(ValueError, match="sage attention type"):
        A.sdpa(q, k, v, None, False, None, True, "qk_int8_pv_fp16")


def test_ring_block_decode_and_merge_equal_the_product_path():
    A, F = _A(), _F()
    rng = np.random.default_rng(72)
    q = to_dev(randn(rng, (1, 8, 256, 128)))
    kc = [to_dev(randn(rng, (1, 2, 256, 128))) for _ in range(2)]
    vc = [to_dev(randn(rng, (1, 2, 256, 128))) for _ in range(2)]
    blocks, ref_blocks = [], []
    for c in range(2):
        blocks.append(A.sdpa_with_lse(q, kc[c], vc[c], None, c == 1, None, True, 256, c * 256))
        ref_blocks.append(F.scaled_dot_product_attention_with_lse(q, kc[c], vc[c], is_causal=c == 1, enable_gqa=True,
                                                                  q_offset=256, k_offset=c * 256))
    torch.cuda.synchronize()
    for (o, l), (ro, rl) in zip(blocks, ref_blocks):
        assert torch.equal(o, ro) and torch.equal(l, rl)
    o, l = A.lse_merge([b[0] for b in blocks], [b[1] for b in blocks], None)
    ro, rl = F.lse_merge([b[0] for b in ref_blocks], [b[1] for b in ref_blocks])
    torch.cuda.synchronize()
    assert torch.equal(o, ro) and torch.equal(l, rl)
    o32, _ = A.lse_merge([b[0] for b in blocks], [b[1] for b in blocks], torch.float32)
    assert o32.dtype == torch.float32
    B, S = 6, 2000
    qd = to_dev(randn(rng, (B, 32, 1, 128)))
    kd, vd = (to_dev(randn(rng, (B, 8, S, 128))) for _ in range(2))
    lengths = torch.tensor([1, 17, 500, 2000, 1999, 0], dtype=torch.int32, device="cuda")
    o, l = A.decode(qd, kd, vd, lengths, None, 0)
    ro, rl = F.decode_attention(qd, kd, vd, lengths)
    torch.cuda.synchronize()
    assert torch.equal(o, ro) and torch.equal(l, rl)


@pytest.mark.parametrize("D,Dv", [(100, 100), (72, 40), (20, 136)])
def test_padded_head_dims_rank5_and_broadcast_mask_against_the_oracle(D, Dv):
    # head dims that are not multiples of 8 are zero-padded by the adapter (scale stays 1/sqrt(real D)); a rank-5
    # batch folds into B; a boolean mask [Sq, Sk] broadcasts over batch and heads
    A = _A()
    rng = np.random.default_rng(73 + D)
    q, k = randn(rng, (2, 1, 4, 96, D)), randn(rng, (2, 1, 2, 130, D))
    v = randn(rng, (2, 1, 2, 130, Dv))
    keep = rng.random((96, 130)) < 0.7
    keep[:, 0] = True
    o, lse = A.sdpa_with_lse(to_dev(q), to_dev(k), to_dev(v), torch.from_numpy(keep).cuda(), False, None, True, 0, 0)
    torch.cuda.synchronize()
    assert o.shape == (2, 1, 4, 96, Dv) and lse.shape == (2, 1, 4, 96)
    ro, rl = orc.sdpa_fwd(rounded(q).reshape(2, 4, 96, D), rounded(k).reshape(2, 2, 130, D),
                          rounded(v).reshape(2, 2, 130, Dv), attn_mask=keep, enable_gqa=True)
    assert max_abs(host(o).reshape(2, 4, 96, Dv), ro) <= O_TOL_BF16
    assert lse_rel(host(lse).reshape(2, 4, 96), rl) <= LSE_TOL
