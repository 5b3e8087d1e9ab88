"""GPU parity of the prefill / per-block kernel against the fp64 oracle.

Tolerances (stated by the task): max-abs <= 2e-2 on bf16/fp16 outputs, LSE |d|/max(|ref|, 1) <= 1e-3.
Full-size configurations are checked on every (batch, head) and every query row against DTorch's
CPU path (libtorch's fp32 CPU flash attention on the same bf16 values).
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, cpu_path_full, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _run_case(B, Hq, Hkv, Sq, Sk, D, causal, dtype=torch.bfloat16, seed=0, q_offset=0, k_offset=0, scale=None):
    rng = np.random.default_rng(seed)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                     is_causal=causal, scale=scale, enable_gqa=Hq != Hkv,
                                                     q_offset=q_offset, k_offset=k_offset)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), is_causal=causal, scale=scale,
                          enable_gqa=Hq != Hkv, q_offset=q_offset, k_offset=k_offset)
    return host(o), host(lse), ro, rl


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 2, 2, 128, 128, 128, False),
    (1, 2, 2, 128, 128, 128, True),
    (2, 4, 1, 200, 200, 128, True),     # GQA 4, ragged tail
    (1, 8, 2, 1, 300, 128, False),      # one query row
    (1, 2, 2, 17, 333, 128, True),      # Sq < Sk, top-left causal
    (1, 2, 2, 300, 40, 128, True),      # Sq > Sk
    (2, 6, 3, 130, 130, 64, True),      # D = 64
    (1, 3, 3, 257, 511, 64, False),
    (1, 8, 1, 64, 64, 128, True),       # GQA 8
])
def test_prefill_small(B, Hq, Hkv, Sq, Sk, D, causal):
    o, lse, ro, rl = _run_case(B, Hq, Hkv, Sq, Sk, D, causal)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_prefill_fp16():
    o, lse, ro, rl = _run_case(2, 4, 2, 190, 190, 128, True, dtype=torch.float16, seed=3)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_prefill_explicit_scale_and_offsets():
    o, lse, ro, rl = _run_case(1, 4, 2, 100, 260, 128, True, seed=4, q_offset=160, k_offset=0, scale=0.05)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_prefill_fully_masked_rows():
    # rows whose every key is in the future see nothing: O = 0, LSE = -inf
    o, lse, ro, rl = _run_case(1, 2, 2, 96, 96, 128, True, seed=5, q_offset=0, k_offset=50)
    assert np.all(o[..., :50, :] == 0) and np.all(np.isneginf(lse[..., :50]))
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_config1_causal_mha_d64():
    # B=1, H=8 (MHA), S=512, D=64, causal, N(0,1) seed 0, scale 1/sqrt(64); GPU runs in bf16
    rng = np.random.default_rng(0)
    q, k, v = (randn(rng, (1, 8, 512, 64)) for _ in range(3))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), is_causal=True)
    # against the fp32 CPU path on the original fp32 inputs (what DTorch computes on a CPU mesh)
    from oracle import dtorch_cpu_path as cpu
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ref_o, ref_l = cpu.sdpa_with_lse(tq, tk, tv, is_causal=True)
    assert max_abs(host(o), ref_o.double().numpy()) <= O_TOL_BF16 * 2  # includes bf16 input rounding
    # and against the oracle on the bf16-rounded inputs (kernel error only)
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=True)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


def test_sdpa_op_contract_and_strides():
    # SdpaOp.compute({q, k, v, None}) -> [O]; non-contiguous (B, S, H, D)-major inputs
    rng = np.random.default_rng(6)
    B, H, S, D = 2, 4, 96, 128
    q, k, v = (randn(rng, (B, S, H, D)) for _ in range(3))
    tq, tk, tv = (to_dev(x).transpose(1, 2) for x in (q, k, v))
    assert not tq.is_contiguous()
    F = _F()
    o = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    assert o.shape == (B, H, S, D) and o.dtype == torch.bfloat16
    ro, _ = orc.sdpa_fwd(*(rounded(x).transpose(0, 2, 1, 3) for x in (q, k, v)), is_causal=True)
    assert max_abs(host(o), ro) <= O_TOL_BF16


def test_reference_operator_test_shape_fp16_gqa_flag():
    # python/dtorch/test/operators/test_scaled_dot_product_attention.py:23-36: fp16 torch.rand
    # [32, 32, 128, 64], enable_gqa=True with equal head counts, non-causal
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.rand(32, 32, 128, 64, generator=g, dtype=torch.float32).half() for _ in range(3))
    F = _F()
    o = F.scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), enable_gqa=True)
    ro, _ = orc.sdpa_fwd(q.double().numpy(), k.double().numpy(), v.double().numpy())
    assert max_abs(host(o), ro) <= 2e-3 * 4  # fp16 output, values in [0, 1]


def test_joint_attention_concat_shape():
    # test_scaled_dot_product_attention.py:73-162: image (512) + text (128) tokens, non-causal
    g = torch.Generator().manual_seed(1)
    parts = [torch.rand(2, 8, n, 64, generator=g).half() for n in (512, 128) for _ in range(3)]
    q = torch.cat([parts[0], parts[3]], 2)
    k = torch.cat([parts[1], parts[4]], 2)
    v = torch.cat([parts[2], parts[5]], 2)
    F = _F()
    o = F.scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda())
    ro, _ = orc.sdpa_fwd(q.double().numpy(), k.double().numpy(), v.double().numpy())
    assert max_abs(host(o), ro) <= 8e-3


def test_deterministic():
    rng = np.random.default_rng(7)
    q, k, v = (to_dev(randn(rng, (1, 4, 300, 128))) for _ in range(3))
    F = _F()
    o1, l1 = F.scaled_dot_product_attention_with_lse(q, k, v, is_causal=True)
    o2, l2 = F.scaled_dot_product_attention_with_lse(q, k, v, is_causal=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_config2_llama_prefill_full_size():
    # B=4, Hq=32, Hkv=8, S=2048, D=128, causal, bf16, seed 0; every (b, h) and row against the CPU path
    rng = np.random.default_rng(0)
    q = randn(rng, (4, 32, 2048, 128))
    k = randn(rng, (4, 8, 2048, 128))
    v = randn(rng, (4, 8, 2048, 128))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), is_causal=True, enable_gqa=True)
    torch.cuda.synchronize()
    ro, rl = cpu_path_full(q, k, v, True)
    err, lerr = max_abs(host(o), ro), lse_rel(host(lse), rl)
    print(f"C2 full size: max-abs {err:.3e}, LSE rel {lerr:.3e}")
    assert err <= O_TOL_BF16
    assert lerr <= LSE_TOL


def test_config5a_mmdit_joint_full_size():
    # B=1, H=24, S=4608 (4096 image + 512 text), D=128, non-causal, bf16, seed 0; every head and row
    rng = np.random.default_rng(0)
    q, k, v = (randn(rng, (1, 24, 4608, 128)) for _ in range(3))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    ro, rl = cpu_path_full(q, k, v, False)
    err, lerr = max_abs(host(o), ro), lse_rel(host(lse), rl)
    print(f"C5a full size: max-abs {err:.3e}, LSE rel {lerr:.3e}")
    assert err <= O_TOL_BF16
    assert lerr <= LSE_TOL


def test_prefill_empty_key_set():
    # Sk = 0: every row is fully masked (O = 0, LSE = -inf), with and without causal masking
    F = _F()
    q = torch.randn(1, 4, 70, 128, device="cuda", dtype=torch.bfloat16)
    kv = torch.empty(1, 2, 0, 128, device="cuda", dtype=torch.bfloat16)
    for causal in (False, True):
        o, lse = F.scaled_dot_product_attention_with_lse(q, kv, kv, is_causal=causal, enable_gqa=True)
        torch.cuda.synchronize()
        assert o.shape == q.shape and lse.shape == (1, 4, 70)
        assert bool((o == 0).all()) and bool(torch.isneginf(lse).all())
