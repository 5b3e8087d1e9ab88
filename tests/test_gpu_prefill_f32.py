"""GPU parity of the fp32 prefill (fp32 matrix cores, fp32 softmax and P) against the fp64 oracle.

fp32 tensors reach SdpaOp::Compute whenever a model runs in fp32: the reference's own Llama test
(python/dtorch/test/modules/test_llama.py:26-64) runs its GPU path in fp32 and compares the whole model
with transformers at 1e-4.  Bar here, on the same fp32 inputs as the fp64 oracle: max |O - O_ref| <= 1e-5
and LSE |d| / max(|ref|, 1) <= 1e-5.  The smallest configuration (B1 H8 S512 D64, causal, fp32) is also
compared with libtorch's fp32 CPU SDPA, the call DTorch makes on a CPU mesh.
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


def _run(q, k, v, causal=False, scale=None, q_offset=0, k_offset=0, mask_dev=None, mask_ref=None):
    Hq, Hkv = q.shape[1], k.shape[1]
    o, lse = _F().scaled_dot_product_attention_with_lse(
        _dev(q), _dev(k), _dev(v), is_causal=causal, scale=scale, enable_gqa=Hq != Hkv, q_offset=q_offset,
        k_offset=k_offset, attn_mask=mask_dev)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    ro, rl = orc.sdpa_fwd(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), attn_mask=mask_ref,
                          is_causal=causal, scale=scale, enable_gqa=Hq != Hkv, q_offset=q_offset, k_offset=k_offset)
    return host(o), host(lse), ro, rl


def _qkv(seed, B, Hq, Hkv, Sq, Sk, D):
    rng = np.random.default_rng(seed)
    return randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))


def test_cpu_runnable_config_fp32_matches_libtorch_cpu():
    # B1 H8 S512 D64, causal, fp32 throughout
    q, k, v = _qkv(0, 1, 8, 8, 512, 512, 64)
    o, lse, ro, rl = _run(q, k, v, causal=True)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    cpu = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    assert max_abs(o, cpu.double().numpy()) <= O_TOL_F32


def test_llama_test_shape_fp32():
    # the reference Llama test's attention: batch 2, 16 tokens, 8 heads of 128, causal
    q, k, v = _qkv(1, 2, 8, 8, 16, 16, 128)
    o, lse, ro, rl = _run(q, k, v, causal=True)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 2, 2, 128, 128, 128, False),
    (2, 4, 1, 200, 200, 128, True),     # GQA 4, ragged tail
    (1, 8, 2, 1, 300, 128, False),      # one query row
    (1, 2, 2, 17, 333, 128, True),      # Sq < Sk, top-left causal
    (1, 2, 2, 300, 40, 128, True),      # Sq > Sk: rows past the keys see all of them
    (2, 6, 3, 130, 130, 64, True),      # D = 64
    (1, 3, 3, 257, 511, 64, False),
    (1, 4, 4, 1000, 1000, 128, True),   # many tiles: the running max moves and rescales
])
def test_prefill_f32_shapes(B, Hq, Hkv, Sq, Sk, D, causal):
    q, k, v = _qkv(10 + Sq, B, Hq, Hkv, Sq, Sk, D)
    o, lse, ro, rl = _run(q, k, v, causal=causal)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_offsets_scale_and_growing_logits():
    q, k, v = _qkv(5, 1, 4, 2, 100, 260, 128)
    k[:, :, 200:] *= 4.0  # later keys raise the row max by far more than the lazy-rescale threshold
    o, lse, ro, rl = _run(q, k, v, causal=True, scale=0.2, q_offset=160, k_offset=0)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_strided_bshd_view():
    # q/k/v handed over as [B, S, H, D] storage viewed as [B, H, S, D] (no copy)
    rng = np.random.default_rng(6)
    B, H, S, D = 2, 4, 150, 128
    x = [randn(rng, (B, S, H, D)) for _ in range(3)]
    tq, tk, tv = (torch.from_numpy(a).cuda().transpose(1, 2) for a in x)
    o = _F().scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    torch.cuda.synchronize()
    ro, _ = orc.sdpa_fwd(*(a.transpose(0, 2, 1, 3).astype(np.float64) for a in x), is_causal=True)
    assert max_abs(host(o), ro) <= O_TOL_F32


def test_prefill_f32_masks():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, L, S, D = 2, 8, 2, 200, 333, 128
    q, k, v = randn(rng, (B, Hq, L, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    keep = rng.random((L, S)) < 0.5
    keep[np.arange(L), rng.integers(0, S, size=L)] = True
    keep[7] = False  # a fully hidden row: O = 0, LSE = -inf
    o, lse, ro, rl = _run(q, k, v, mask_dev=torch.from_numpy(keep).cuda(), mask_ref=keep)
    assert np.all(o[:, :, 7] == 0) and np.all(np.isneginf(lse[:, :, 7]))
    rows = np.ones(L, dtype=bool)
    rows[7] = False
    assert max_abs(o[:, :, rows], ro[:, :, rows]) <= O_TOL_F32
    assert lse_rel(lse[:, :, rows], rl[:, :, rows]) <= LSE_TOL_F32
    # a float per-head bias with is_causal, D = 64
    q, k, v = _qkv(8, 1, 4, 4, 96, 96, 64)
    bias = (rng.standard_normal((1, 4, 96, 96)) * 2).astype(np.float32)
    o, lse, ro, rl = _run(q, k, v, causal=True, mask_dev=torch.from_numpy(bias).cuda(),
                          mask_ref=bias.astype(np.float64))
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_ring_step_fp32():
    # 4 chunks of 256 tokens, rank 2: diagonal block causal, two earlier blocks full, merged by LSE
    rng = np.random.default_rng(9)
    C, H, D = 256, 4, 128
    q_all, k_all, v_all = (randn(rng, (1, H, 4 * C, D)) for _ in range(3))
    idx = 2
    kch = [_dev(k_all[:, :, c * C:(c + 1) * C]) for c in range(4)]
    vch = [_dev(v_all[:, :, c * C:(c + 1) * C]) for c in range(4)]
    o, lse = _F().ring_attention_step(_dev(q_all[:, :, idx * C:(idx + 1) * C]), kch, vch, idx)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    ro, rl = orc.sdpa_fwd(q_all.astype(np.float64), k_all.astype(np.float64), v_all.astype(np.float64),
                          is_causal=True)
    rows = slice(idx * C, (idx + 1) * C)
    assert max_abs(host(o), ro[:, :, rows]) <= O_TOL_F32
    assert lse_rel(host(lse), rl[:, :, rows]) <= LSE_TOL_F32


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,Dv,causal", [
    (2, 8, 2, 150, 150, 96, 96, True),     # 96 -> kernel 128, GQA 4
    (1, 4, 4, 130, 257, 80, 80, False),    # 80 -> 128, ragged key tail
    (1, 2, 2, 100, 100, 32, 32, True),     # 32 -> 64
    (1, 2, 1, 70, 90, 100, 128, True),     # D 100, Dv 128 at 128
    (1, 2, 2, 90, 90, 128, 44, False),     # Dv < D at 128
    (1, 3, 3, 33, 40, 4, 4, False),        # the smallest fp32 head dim (one 16-byte chunk)
    (1, 2, 2, 65, 64, 60, 36, True),       # both below 64, Sq > Sk
])
def test_prefill_f32_padded_head_dims(B, Hq, Hkv, Sq, Sk, D, Dv, causal):
    # fp32 takes any D and Dv that are multiples of 4 up to 128: the kernel runs at 64 or 128 and
    # reads the columns past the real dims as zeros; O takes v's last axis
    # (scaled_dot_product_attention_op.cc:26-29).
    rng = np.random.default_rng(D * 1000 + Dv)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, Dv))
    o, lse, ro, rl = _run(q, k, v, causal=causal)
    assert o.shape == (B, Hq, Sq, Dv)
    assert max_abs(o, ro) <= O_TOL_F32
    assert lse_rel(lse, rl) <= LSE_TOL_F32


def test_prefill_f32_padded_columns_past_the_row_are_never_read():
    # head-sliced views of wider fp32 rows whose columns past D / Dv hold NaN, with a mask and causal
    # offsets: a padded load that touched them would poison the scores or O
    rng = np.random.default_rng(44)
    B, H, Sq, Sk, D, Dv = 2, 4, 70, 100, 92, 52
    q, k, v = randn(rng, (B, H, Sq, D)), randn(rng, (B, H, Sk, D)), randn(rng, (B, H, Sk, Dv))
    wide = []
    for x in (q, k, v):
        w = np.full(x.shape[:-1] + (128,), np.nan, dtype=np.float32)
        w[..., :x.shape[-1]] = x
        wide.append(torch.from_numpy(w).cuda()[..., :x.shape[-1]])
    keep = rng.random((Sq, Sk)) < 0.6
    keep[:, 0] = True
    o, lse = _F().scaled_dot_product_attention_with_lse(*wide, is_causal=True, q_offset=30,
                                                        attn_mask=torch.from_numpy(keep).cuda())
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), attn_mask=keep,
                          is_causal=True, q_offset=30)
    assert max_abs(host(o), ro) <= O_TOL_F32
    assert lse_rel(host(lse), rl) <= LSE_TOL_F32
