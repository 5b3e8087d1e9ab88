"""GPU parity of the software-pipelined head-dim-512 prefill (non-causal, no mask, no padding) against the fp64
oracle, and bit-identity with the unpipelined wide kernel.

Non-causal head-dim-512 calls without mask or padding (the VAE mid-block attention of the reference's diffusers
ports, python/dtorch/applications/huggingface/diffusers/models/unets/unet_2d_blocks.py:126-140) run
prefill_wide512_kernel, whose tile loop is one inline-asm program.  The cases cover its bookkeeping: a single
key and a single tile, ragged key tails (the last tile's mask), query counts that leave a workgroup partly
empty, GQA, key blocks (grids of at most half the CUs split their keys), fp16, strided layouts and a negative
scale (which takes the unpipelined kernel).  An all-zero additive mask sends the same inputs to the
unpipelined kernel, whose arithmetic the program restates element for element: the two outputs must be equal
bit for bit.  Bar otherwise: max-abs 2e-2 on O, LSE |d| / max(|ref|, 1) <= 1e-3.
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


def _inputs(B, Hq, Hkv, Sq, Sk, seed):
    rng = np.random.default_rng(seed)
    return randn(rng, (B, Hq, Sq, 512)), randn(rng, (B, Hkv, Sk, 512)), randn(rng, (B, Hkv, Sk, 512))


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,dtype", [
    (1, 1, 1, 100, 1, torch.bfloat16),      # one key
    (1, 1, 1, 70, 32, torch.bfloat16),      # one whole tile
    (1, 2, 2, 1000, 777, torch.bfloat16),   # ragged tail, Sq not a multiple of 64
    (2, 4, 2, 130, 1000, torch.bfloat16),   # GQA 2, key blocks (a grid of 24 workgroups)
    (1, 1, 1, 4096, 4096, torch.bfloat16),  # key blocks of whole tiles
    (1, 2, 1, 300, 65, torch.float16),      # fp16, GQA, a tail of one key
    (3, 1, 1, 64, 2000, torch.float16),     # fp16, one workgroup per batch, many tiles
])
def test_wide512_against_oracle(B, Hq, Hkv, Sq, Sk, dtype):
    q, k, v = _inputs(B, Hq, Hkv, Sq, Sk, seed=Sq + Sk)
    o, lse = _F().scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                        enable_gqa=Hq != Hkv)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), enable_gqa=Hq != Hkv)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,dtype", [
    (1, 2, 2, 333, 500, torch.bfloat16),
    (1, 1, 1, 2048, 2048, torch.bfloat16),  # key blocks
    (2, 2, 1, 200, 97, torch.float16),
])
def test_wide512_equals_unpipelined_kernel(B, Hq, Hkv, Sq, Sk, dtype):
    q, k, v = (to_dev(x, dtype) for x in _inputs(B, Hq, Hkv, Sq, Sk, seed=7 + Sq))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(q, k, v, enable_gqa=Hq != Hkv)
    zero = torch.zeros(Sq, Sk, device=q.device, dtype=torch.float32)  # routes to prefill_wide_kernel
    o2, lse2 = F.scaled_dot_product_attention_with_lse(q, k, v, attn_mask=zero, enable_gqa=Hq != Hkv)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.equal(lse, lse2)


def test_wide512_strided_layout_and_negative_scale():
    rng = np.random.default_rng(21)
    B, H, S = 2, 2, 300
    qs, ks, vs = (randn(rng, (B, S, H, 512)) for _ in range(3))
    tq, tk, tv = (to_dev(x).transpose(1, 2) for x in (qs, ks, vs))  # [B, S, H, D] storage
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv)
    torch.cuda.synchronize()
    rq, rk, rv = (rounded(x).transpose(0, 2, 1, 3) for x in (qs, ks, vs))
    ro, rl = orc.sdpa_fwd(rq, rk, rv)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL
    # a negative scale runs the unpipelined kernel (it loads q through the sign transform)
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv, scale=-0.03)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rq, rk, rv, scale=-0.03)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


def test_wide512_key_offsets_past_31_bits_take_the_unpipelined_kernel():
    # K and V rows 2 MiB apart (two views of one 2.1 GB buffer): (Sk + 64) * pitch >= 2^31, so a tile's byte
    # offset no longer fits the program's 32-bit scalar arithmetic and the call must take prefill_wide_kernel,
    # whose outputs equal the pipelined kernel's on contiguous copies of the same K and V bit for bit
    rng = np.random.default_rng(23)
    Sq, Sk, pitch = 128, 1000, 1 << 20
    assert (Sk + 64) * pitch * 2 >= 1 << 31
    q, k, v = randn(rng, (1, 1, Sq, 512)), randn(rng, (1, 1, Sk, 512)), randn(rng, (1, 1, Sk, 512))
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    buf = torch.zeros(Sk * pitch, dtype=torch.bfloat16, device=tq.device)
    sk = torch.as_strided(buf, (1, 1, Sk, 512), (0, 0, pitch, 1), 0)
    sv = torch.as_strided(buf, (1, 1, Sk, 512), (0, 0, pitch, 1), 512)
    sk.copy_(tk)
    sv.copy_(tv)
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(tq, sk, sv)
    o2, lse2 = F.scaled_dot_product_attention_with_lse(tq, tk, tv)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.equal(lse, lse2)
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v))
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL
    del buf, sk, sv


def test_wide512_vae_16k_sampled_rows():
    # the VAE shape itself (128 x 128 latent pixels): the first and last row of every 64-row workgroup
    rng = np.random.default_rng(22)
    S = 16384
    q, k, v = (randn(rng, (1, 1, S, 512)) for _ in range(3))
    o, lse = _F().scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    rows = np.sort(np.concatenate([np.arange(0, S, 64), np.arange(63, S, 64)]))
    ro, rl = orc.sdpa_fwd(rounded(q)[:, :, rows], rounded(k), rounded(v))
    assert max_abs(host(o)[:, :, rows], ro) <= O_TOL_BF16
    assert lse_rel(host(lse)[:, :, rows], rl) <= LSE_TOL
