"""GPU parity of the wide-head prefill (D = 256, 512) against the fp64 oracle.

The reference's diffusers ports reach D = 512 through the VAE mid-block attention: one head of
block_out_channels[-1] = 512 dimensions over the latent's pixels, non-causal
(python/dtorch/applications/huggingface/diffusers/models/unets/unet_2d_blocks.py:126-140,
autoencoders/vae.py:62-68).  Same bar as every bf16/fp16 case: max-abs 2e-2 on O, LSE |d| / max(|ref|, 1)
<= 1e-3.
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


def _case(B, Hq, Hkv, Sq, Sk, D, causal, dtype=torch.bfloat16, seed=0, q_offset=0, k_offset=0, mask=None):
    rng = np.random.default_rng(seed)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    o, lse = _F().scaled_dot_product_attention_with_lse(
        to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), is_causal=causal, enable_gqa=Hq != Hkv,
        q_offset=q_offset, k_offset=k_offset, attn_mask=None if mask is None else torch.from_numpy(mask).cuda())
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), attn_mask=mask,
                          is_causal=causal, enable_gqa=Hq != Hkv, q_offset=q_offset, k_offset=k_offset)
    return host(o), host(lse), ro, rl


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 1, 1, 1024, 1024, 512, False),   # the VAE attention's shape, at 32x32 latent pixels
    (2, 2, 2, 100, 333, 512, False),     # ragged tails
    (1, 4, 2, 300, 300, 512, True),      # causal, GQA 2
    (1, 8, 1, 130, 200, 256, True),      # D = 256, GQA 8, Sq < Sk
    (2, 3, 3, 257, 64, 256, False),      # Sq > Sk
    (1, 2, 2, 1, 500, 512, False),       # one query row
])
def test_prefill_wide(B, Hq, Hkv, Sq, Sk, D, causal):
    o, lse, ro, rl = _case(B, Hq, Hkv, Sq, Sk, D, causal)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_prefill_wide_fp16_offsets_and_mask():
    o, lse, ro, rl = _case(1, 2, 2, 96, 200, 512, True, dtype=torch.float16, seed=3, q_offset=100)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL
    rng = np.random.default_rng(4)
    keep = rng.random((160, 160)) < 0.6
    keep[np.arange(160), np.arange(160)] = True
    o, lse, ro, rl = _case(1, 2, 2, 160, 160, 256, False, seed=5, mask=keep)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_vae_attention_16k_pixels_sampled_rows():
    # 128x128 latent pixels (a 1024x1024 image), one head of 512, non-causal.  Rows checked: the first and the
    # last row of every 64-row workgroup (512 of the 16,384), which covers each workgroup's two row groups and
    # every position of the grid
    B, H, S, D = 1, 1, 16384, 512
    g = torch.Generator(device="cuda").manual_seed(12)
    q, k, v = (torch.randn(B, H, S, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    o, lse = _F().scaled_dot_product_attention_with_lse(q, k, v)
    torch.cuda.synchronize()
    rows = np.sort(np.concatenate([np.arange(0, S, 64), np.arange(63, S, 64)]))
    ro, rl = orc.sdpa_fwd(host(q[:, :, rows]), host(k), host(v))
    assert max_abs(host(o[:, :, rows]), ro) <= O_TOL_BF16
    assert lse_rel(host(lse[:, :, rows]), rl) <= LSE_TOL


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal,q_offset,dtype", [
    (1, 1, 1, 4096, 4096, 512, False, 0, torch.bfloat16),   # the 64x64-latent VAE attention: 4 key blocks
    (1, 2, 2, 1024, 1024, 512, True, 0, torch.bfloat16),    # causal key blocks with their offsets
    (1, 4, 1, 700, 1500, 256, True, 800, torch.float16),    # GQA 4, causal with a query offset
    (1, 1, 1, 333, 2000, 320, False, 0, torch.bfloat16),    # padded head dim in key blocks
    (2, 4, 4, 2048, 2048, 512, False, 0, torch.bfloat16),   # a full grid: no split
    (1, 2, 1, 500, 1001, 512, False, 0, torch.float16),     # fp16, GQA 2, a ragged tail in the last block
    (2, 8, 4, 1000, 1001, 512, False, 0, torch.bfloat16),   # a full grid, ragged keys and queries
])
def test_prefill_wide_key_blocks(B, Hq, Hkv, Sq, Sk, D, causal, q_offset, dtype):
    # Grids smaller than the CU count run the keys as several blocks merged by LSE; every row and the LSE
    # must match the single-pass oracle.
    o, lse, ro, rl = _case(B, Hq, Hkv, Sq, Sk, D, causal, dtype=dtype, seed=Sq + D, q_offset=q_offset)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_prefill_wide_key_blocks_with_mask_and_sdpa_op():
    rng = np.random.default_rng(77)
    keep = rng.random((512, 1800)) < 0.5
    keep[:, 1799] = True
    o, lse, ro, rl = _case(1, 2, 2, 512, 1800, 512, False, seed=78, mask=keep)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL
    # the one-output SdpaOp takes the same split (no LSE output requested)
    q, k, v = (torch.randn(1, 1, 512, 512, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    o1 = _F().scaled_dot_product_attention(q, k, v, is_causal=True)
    o2, _ = _F().scaled_dot_product_attention_with_lse(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    ro, _ = orc.sdpa_fwd(host(q), host(k), host(v), is_causal=True)
    assert max_abs(host(o1), ro) <= O_TOL_BF16
