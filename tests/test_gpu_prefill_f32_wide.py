"""GPU parity of the fp32 prefill at kernel head dims 256 and 512 (the wide fp32 kernel) against the fp64 oracle.

The diffusers VAE attention is one head of 512 (python/dtorch/applications/huggingface/diffusers/models/unets/
unet_2d_blocks.py:126-140); a port that runs the VAE in fp32 reaches SdpaOp::Compute with fp32 tensors of that
head dim, which libtorch takes (scaled_dot_product_attention_op.cc:107-109).  Same bars as the fp32 kernel of
head dims up to 128: max |O - O_ref| <= 1e-5 and LSE |d| / max(|ref|, 1) <= 1e-5 on the same fp32 inputs.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import host, lse_rel, max_abs, randn

pytestmark = pytest.mark.gpu

O_TOL_F32 = 1e-5
LSE_TOL_F32 = 1e-5


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _qkv(seed, B, Hq, Hkv, Sq, Sk, D, Dv=None):
    rng = np.random.default_rng(seed)
    return (randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, Dv or D)))


def _run(q, k, v, causal=False, scale=None, q_offset=0, k_offset=0, mask_dev=None, mask_ref=None):
    Hq, Hkv = q.shape[1], k.shape[1]
    print(f"fp32 wide: q {q.shape} k {k.shape} v {v.shape} causal={causal} mask={mask_ref is not None}", flush=True)
    o, lse = _F().scaled_dot_product_attention_with_lse(
        _dev(q), _dev(k), _dev(v), is_causal=causal, scale=scale, enable_gqa=Hq != Hkv, q_offset=q_offset,
        k_offset=k_offset, attn_mask=mask_dev)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and o.shape == q.shape[:3] + (v.shape[3],)
    ro, rl = orc.sdpa_fwd(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), attn_mask=mask_ref,
                          is_causal=causal, scale=scale, enable_gqa=Hq != Hkv, q_offset=q_offset, k_offset=k_offset)
    return host(o), host(lse), ro, rl


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 2, 2, 128, 128, 256, False),
    (2, 4, 1, 200, 200, 256, True),     # GQA 4, ragged tail
    (1, 2, 2, 300, 40, 256, True),      # Sq > Sk: rows past the keys see all of them
    (1, 1, 1, 1, 300, 512, False),      # one query row
    (1, 2, 1, 77, 333, 512, False),     # GQA 2, ragged query and key tails
    (1, 2, 2, 17, 333, 512, True),      # Sq < Sk, bottom-right causal
    (1, 1, 1, 1000, 1000, 512, True),   # many tiles: the running max moves and rescales
])
def test_prefill_f32_wide_shapes(B, Hq, Hkv, Sq, Sk, D, causal):
    q, k, v = _qkv(20 + Sq + D, B, Hq, Hkv, Sq, Sk, D)
    o, lse, ro, rl = _run(q, k, v, causal=causal)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_vae_attention_fp32_1024_pixels():
    # the VAE mid-block attention at a 32x32 latent: one head of 512 over 1024 pixels, non-causal, fp32
    q, k, v = _qkv(31, 1, 1, 1, 1024, 1024, 512)
    o, lse, ro, rl = _run(q, k, v)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32
    # and against libtorch's fp32 CPU SDPA, the call DTorch makes on a CPU mesh
    cpu = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(x) for x in (q, k, v)))
    assert max_abs(o, cpu.double().numpy()) <= O_TOL_F32


@pytest.mark.parametrize("D,Dv,causal", [(300, 300, False), (200, 136, True), (512, 264, False), (132, 132, True)])
def test_prefill_f32_wide_padded_head_dims(D, Dv, causal):
    # real head dims below the kernel's 256 / 512 (multiples of 4, D and Dv apart): zero columns, the scale of
    # the real D, the output cut back to Dv
    q, k, v = _qkv(40 + D + Dv, 1, 2, 1, 150, 170, D, Dv)
    o, lse, ro, rl = _run(q, k, v, causal=causal)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


@pytest.mark.parametrize("kind", ["bool_key_padding", "float_bias"])
def test_prefill_f32_wide_masks(kind):
    B, H, S, D = 2, 2, 130, 512
    q, k, v = _qkv(50, B, H, H, S, S, D)
    rng = np.random.default_rng(51)
    if kind == "bool_key_padding":
        keep = np.ones((B, 1, 1, S), dtype=bool)
        keep[0, ..., 100:] = False
        keep[1, ..., 7] = False
        mask_dev, mask_ref = torch.from_numpy(keep).cuda(), keep
    else:
        bias = (rng.standard_normal((1, H, S, S)) * 2).astype(np.float32)
        mask_dev, mask_ref = _dev(bias), bias.astype(np.float64)
    o, lse, ro, rl = _run(q, k, v, causal=True, mask_dev=mask_dev, mask_ref=mask_ref)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_wide_ring_block_offsets_and_scale():
    # a ring block with global causal offsets (key j visible to query i iff j + k_off <= i + q_off) and an
    # explicit scale
    q, k, v = _qkv(60, 1, 2, 2, 96, 96, 256)
    o, lse, ro, rl = _run(q, k, v, causal=True, scale=0.07, q_offset=96, k_offset=48)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_wide_empty_and_single_key():
    # no keys: O = 0 and LSE = -inf (the rows see nothing); one key: O = v, LSE = the one score
    F = _F()
    q = _dev(np.ones((1, 2, 40, 512), dtype=np.float32))
    k0 = torch.zeros(1, 2, 0, 512, dtype=torch.float32, device="cuda")
    o, lse = F.scaled_dot_product_attention_with_lse(q, k0, k0)
    torch.cuda.synchronize()
    assert o.shape == (1, 2, 40, 512) and bool((o == 0).all()) and bool(torch.isneginf(lse).all())
    q, k, v = _qkv(70, 1, 2, 2, 40, 1, 256)
    o, lse, ro, rl = _run(q, k, v)
    assert max_abs(o, ro) <= O_TOL_F32 and lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_wide_fully_masked_rows():
    # rows whose mask hides every key get O = 0 and LSE = -inf, as in every other kernel
    B, H, S, D = 1, 2, 70, 512
    q, k, v = _qkv(80, B, H, H, S, S, D)
    keep = np.ones((B, 1, S, S), dtype=bool)
    keep[0, 0, 5] = False
    keep[0, 0, 66] = False
    o, lse, ro, rl = _run(q, k, v, mask_dev=torch.from_numpy(keep).cuda(), mask_ref=keep)
    assert np.all(o[0, :, 5] == 0) and np.all(np.isneginf(lse[0, :, 5]))
    ok = ~np.isneginf(rl)
    assert max_abs(o, ro) <= O_TOL_F32 and lse_rel(lse[ok], rl[ok]) <= LSE_TOL_F32
