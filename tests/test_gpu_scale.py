"""GPU parity at softmax scales of zero and below, which torch::scaled_dot_product_attention accepts
(scaled_dot_product_attention_op.cc:107-109 forwards SdpaParam's std::optional<double> scale): logits =
scale * q.k (+ mask).  The kernels run |scale| on negated q, or scale 1 on zeroed q for scale 0; each case
is checked against the oracle at the same scale, and the negated-q identity is checked bit for bit."""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, O_TOL_FP8, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("scale", [-0.2, 0.0, -1.0 / np.sqrt(128)])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_nonpositive_scale(dtype, scale, causal):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, S, D = 2, 4, 2, 150, 128
    q, k, v = randn(rng, (B, Hq, S, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    o, lse = _F().scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                        is_causal=causal, scale=scale, enable_gqa=True)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), is_causal=causal, scale=scale,
                          enable_gqa=True)
    tol = 1e-5 if dtype == torch.float32 else O_TOL_BF16
    assert max_abs(host(o), ro) <= tol
    assert lse_rel(host(lse), rl) <= (1e-5 if dtype == torch.float32 else LSE_TOL)


def test_negative_scale_is_positive_scale_on_negated_q():
    rng = np.random.default_rng(8)
    q, k, v = randn(rng, (1, 8, 200, 128)), randn(rng, (1, 2, 200, 128)), randn(rng, (1, 2, 200, 128))
    tq, tk, tv = (to_dev(x) for x in (q, k, v))
    F = _F()
    a = F.scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=True, scale=-0.1, enable_gqa=True)
    b = F.scaled_dot_product_attention_with_lse(-tq, tk, tv, is_causal=True, scale=0.1, enable_gqa=True)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("mask_kind", ["bool", "additive"])
def test_zero_scale_with_mask_gives_the_mask_alone(mask_kind):
    rng = np.random.default_rng(9)
    B, Hq, Hkv, L, S, D = 1, 4, 4, 96, 130, 64
    q, k, v = randn(rng, (B, Hq, L, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    if mask_kind == "bool":
        m = rng.random((L, S)) < 0.6
        m[:, 0] = True
        mdev = torch.from_numpy(m).cuda()
    else:
        m = (rng.standard_normal((B, Hq, L, S)) * 2).astype(np.float32)
        mdev = torch.from_numpy(m).cuda()
    o, lse = _F().scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), scale=0.0, attn_mask=mdev)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), attn_mask=m, scale=0.0)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


@pytest.mark.parametrize("D,causal", [(256, True), (512, False), (96, True)])
def test_wide_and_padded_heads_negative_scale(D, causal):
    rng = np.random.default_rng(10 + D)
    B, Hq, Hkv, S = 1, 2, 1, 100
    q, k, v = randn(rng, (B, Hq, S, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    o, lse = _F().scaled_dot_product_attention_with_lse(to_dev(q), to_dev(k), to_dev(v), is_causal=causal,
                                                        scale=-0.05, enable_gqa=True)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=causal, scale=-0.05, enable_gqa=True)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("scale", [-0.15, 0.0])
def test_decode_nonpositive_scale(dtype, scale):
    rng = np.random.default_rng(11)
    B, Hq, Hkv, Smax, D = 3, 8, 2, 700, 128
    lengths = np.array([0, 385, 700], dtype=np.int32)
    q = randn(rng, (B, Hq, 1, D))
    kc, vc = randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    o, lse = _F().decode_attention(to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype),
                                   torch.from_numpy(lengths).cuda(), scale=scale)
    torch.cuda.synchronize()
    ro, rl = orc.decode(rounded(q, dtype), rounded(kc, dtype), rounded(vc, dtype), lengths, scale=scale)
    tol = 1e-5 if dtype == torch.float32 else O_TOL_BF16
    assert max_abs(host(o), ro) <= tol
    assert lse_rel(host(lse), rl[..., 0]) <= (1e-5 if dtype == torch.float32 else LSE_TOL)


def test_paged_decode_negative_scale_matches_contiguous():
    rng = np.random.default_rng(12)
    B, Hq, Hkv, D, ps, npages = 2, 4, 2, 128, 16, 40
    lengths = np.array([100, 257], dtype=np.int32)
    pages_k, pages_v = randn(rng, (npages, Hkv, ps, D)), randn(rng, (npages, Hkv, ps, D))
    table = rng.permutation(npages)[:2 * 17].reshape(2, 17).astype(np.int32)
    q = randn(rng, (B, Hq, 1, D))
    F = _F()
    o, lse = F.decode_attention_paged(to_dev(q), to_dev(pages_k), to_dev(pages_v), torch.from_numpy(table).cuda(),
                                      torch.from_numpy(lengths).cuda(), scale=-0.1)
    torch.cuda.synchronize()
    kc = orc.gather_pages(rounded(pages_k), table, lengths)
    vc = orc.gather_pages(rounded(pages_v), table, lengths)
    ro, rl = orc.decode(rounded(q), kc, vc, lengths, scale=-0.1)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl[..., 0]) <= LSE_TOL


def test_native_fp8_negative_and_zero_scale():
    rng = np.random.default_rng(13)
    q, k, v = randn(rng, (1, 4, 256, 128)), randn(rng, (1, 2, 256, 128)), randn(rng, (1, 2, 256, 128))
    tq, tk, tv = (to_dev(x) for x in (q, k, v))
    F = _F()
    opt = F.SdpaOption(sage_attn_type="native_fp8")
    a = F.scaled_dot_product_attention_with_lse(tq, tk, tv, scale=-0.08, enable_gqa=True, sdpa_option=opt)
    b = F.scaled_dot_product_attention_with_lse(-tq, tk, tv, scale=0.08, enable_gqa=True, sdpa_option=opt)
    z = F.scaled_dot_product_attention_with_lse(tq, tk, tv, scale=0.0, enable_gqa=True, sdpa_option=opt)
    torch.cuda.synchronize()
    # per-head e4m3 rounding is symmetric, so negating q commutes with the quantization
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), scale=-0.08, enable_gqa=True)
    assert max_abs(host(a[0]), ro) <= O_TOL_FP8
    # scale 0: every logit is 0, the output is the mean of V's e4m3-rounded rows
    rz, rlz = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), scale=0.0, enable_gqa=True)
    assert max_abs(host(z[0]), rz) <= O_TOL_FP8
    assert lse_rel(host(z[1]), rlz) <= LSE_TOL


def test_infinite_scale_raises():
    t = torch.zeros(1, 2, 8, 64, device="cuda", dtype=torch.bfloat16)
    F = _F()
    with pytest.raises(ValueError, match="finite"):
        F.scaled_dot_product_attention(t, t, t, scale=float("inf"))
    with pytest.raises(ValueError, match="finite"):
        F.decode_attention(t[:, :, :1], t, t, torch.ones(1, dtype=torch.int32, device="cuda"), scale=float("-inf"))
