"""Seeded random sweep of every kernel family against the fp64 oracle.

Each case draws its shapes, dtype and options from its own seed and prints them before the call, so a
failure names a reproducible case.  Bars as in the per-kernel tests: 16-bit outputs max-abs 2e-2 and LSE
|d| / max(|ref|, 1) <= 1e-3; fp32 1e-5 on both; native fp8 against exact attention on the per-head
dequantized inputs, 6e-2 and 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, O_TOL_FP8, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _tols(dtype):
    return (1e-5, 1e-5) if dtype == "fp32" else (O_TOL_BF16, LSE_TOL)


@pytest.mark.parametrize("seed", range(120))
def test_prefill_random(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
    step = 4 if dtype == "fp32" else 8
    # the kernel head dim (64, 128, 256, 512) first, so that each kernel family draws as many cases; then
    # the real head dims inside it, the value head dim at most as wide
    band = int(rng.choice([64, 128, 256, 512]))
    lo = 0 if band == 64 else band // 2
    D = int(rng.integers(lo // step + 1, band // step + 1)) * step
    Dv = D if rng.random() < 0.6 else int(rng.integers(1, band // step + 1)) * step
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 3, 4]))
    B = int(rng.integers(1, 3))
    Sq, Sk = int(rng.integers(1, 300)), int(rng.integers(1, 300))
    causal = bool(rng.random() < 0.5)
    scale = None if rng.random() < 0.7 else float(rng.uniform(0.02, 0.2))
    q_off = int(rng.integers(0, 200)) if causal and rng.random() < 0.3 else 0
    k_off = int(rng.integers(0, 100)) if causal and rng.random() < 0.2 else 0
    mask, kind = None, "none"
    r = rng.random()
    if r < 0.15:
        mask, kind = rng.random((B, 1, Sq, Sk)) < 0.7, "bool"
    elif r < 0.25:
        mask, kind = (rng.standard_normal((Sq, Sk)) * 2).astype(np.float32), "bias"
    print(f"prefill seed={seed}: {dtype} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} Dv={Dv} causal={causal} "
          f"offsets=({q_off},{k_off}) scale={scale} mask={kind}", flush=True)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, Dv))
    t = DTYPES[dtype]
    o, lse = _F().scaled_dot_product_attention_with_lse(
        to_dev(q, t), to_dev(k, t), to_dev(v, t), is_causal=causal, scale=scale, enable_gqa=Hq != Hkv,
        q_offset=q_off, k_offset=k_off, attn_mask=None if mask is None else torch.from_numpy(mask).cuda())
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, Sq, Dv) and o.dtype == t
    ro, rl = orc.sdpa_fwd(rounded(q, t), rounded(k, t), rounded(v, t), attn_mask=mask, is_causal=causal,
                          scale=scale, enable_gqa=Hq != Hkv, q_offset=q_off, k_offset=k_off)
    to, tl = _tols(dtype)
    assert max_abs(host(o), ro) <= to
    assert lse_rel(host(lse), rl) <= tl


@pytest.mark.parametrize("seed", range(40))
def test_decode_random(seed):
    rng = np.random.default_rng(2000 + seed)
    dtype = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
    step = 4 if dtype == "fp32" else 8
    D = int(rng.integers(1, 128 // step + 1)) * step
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 9))
    Smax = int(rng.integers(1, 2000))
    lengths = rng.integers(0, Smax + 1, size=B).astype(np.int32)
    chunk = int(rng.choice([0, 128, 256, 384, 512]))
    print(f"decode seed={seed}: {dtype} B={B} Hq={Hq} Hkv={Hkv} S_max={Smax} D={D} chunk={chunk} "
          f"lengths={lengths.tolist()}", flush=True)
    q, kc, vc = randn(rng, (B, Hq, 1, D)), randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    t = DTYPES[dtype]
    o, lse = _F().decode_attention(to_dev(q, t), to_dev(kc, t), to_dev(vc, t), torch.from_numpy(lengths).cuda(),
                                   chunk=chunk)
    torch.cuda.synchronize()
    ro, rl = orc.decode(rounded(q, t), rounded(kc, t), rounded(vc, t), lengths)
    to, tl = _tols(dtype)
    assert max_abs(host(o), ro) <= to
    assert lse_rel(host(lse), rl[..., 0]) <= tl


@pytest.mark.parametrize("seed", range(30))
def test_decode_paged_random(seed):
    rng = np.random.default_rng(3000 + seed)
    dtype = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
    step = 4 if dtype == "fp32" else 8
    D = int(rng.integers(1, 128 // step + 1)) * step
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 4]))
    B = int(rng.integers(1, 6))
    ps = int(rng.choice([16, 32, 64, 128]))
    max_pages = int(rng.integers(1, 24))
    lengths = rng.integers(0, max_pages * ps + 1, size=B).astype(np.int32)
    num_pages = B * max_pages + int(rng.integers(0, 8))
    table = rng.permutation(num_pages)[:B * max_pages].reshape(B, max_pages).astype(np.int32)
    print(f"paged decode seed={seed}: {dtype} B={B} Hq={Hq} Hkv={Hkv} D={D} page={ps} pages/seq={max_pages} "
          f"pool={num_pages} lengths={lengths.tolist()}", flush=True)
    q = randn(rng, (B, Hq, 1, D))
    kp, vp = randn(rng, (num_pages, Hkv, ps, D)), randn(rng, (num_pages, Hkv, ps, D))
    t = DTYPES[dtype]
    o, lse = _F().decode_attention_paged(to_dev(q, t), to_dev(kp, t), to_dev(vp, t), torch.from_numpy(table).cuda(),
                                         torch.from_numpy(lengths).cuda())
    torch.cuda.synchronize()
    ro, rl = orc.decode_paged(rounded(q, t), rounded(kp, t), rounded(vp, t), table, lengths)
    to, tl = _tols(dtype)
    assert max_abs(host(o), ro) <= to
    assert lse_rel(host(lse), rl[..., 0]) <= tl


@pytest.mark.parametrize("seed", range(30))
def test_merge_random(seed):
    rng = np.random.default_rng(4000 + seed)
    dtype = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
    n = int(rng.integers(1, 9))
    B, H, S = int(rng.integers(1, 3)), int(rng.integers(1, 5)), int(rng.integers(1, 600))
    D = int(rng.integers(1, 33)) * 8
    print(f"merge seed={seed}: {dtype} n={n} B={B} H={H} S={S} D={D}", flush=True)
    os_ = [randn(rng, (B, H, S, D)) for _ in range(n)]
    ls_ = [randn(rng, (B, H, S)).astype(np.float32) * 3 for _ in range(n)]
    if n > 1 and rng.random() < 0.5:
        ls_[int(rng.integers(n))][..., : S // 2] = -np.inf  # a block that saw no key for half the rows
    t = DTYPES[dtype]
    o, lse = _F().lse_merge([to_dev(x, t) for x in os_], [torch.from_numpy(x).cuda() for x in ls_])
    torch.cuda.synchronize()
    ro, rl = orc.lse_merge([rounded(x, t) for x in os_], [x.astype(np.float64) for x in ls_])
    to = 1e-5 if dtype == "fp32" else O_TOL_BF16
    assert max_abs(host(o), ro) <= to
    assert lse_rel(host(lse), rl) <= 1e-6


@pytest.mark.parametrize("seed", range(30))
def test_native_fp8_random(seed):
    rng = np.random.default_rng(5000 + seed)
    dtype = ["bf16", "fp16"][int(rng.integers(2))]
    D = int(rng.choice([64, 128])) if rng.random() < 0.6 else int(rng.integers(1, 17)) * 8
    Hkv = int(rng.choice([1, 2]))
    Hq = Hkv * int(rng.choice([1, 2, 4]))
    B = int(rng.integers(1, 3))
    Sq, Sk = int(rng.integers(1, 400)), int(rng.integers(1, 400))
    causal = bool(rng.random() < 0.5)
    print(f"native fp8 seed={seed}: {dtype} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} causal={causal}", flush=True)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    t = DTYPES[dtype]
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, t), to_dev(k, t), to_dev(v, t), is_causal=causal,
                                                     enable_gqa=Hq != Hkv,
                                                     sdpa_option=F.SdpaOption(sage_attn_type="native_fp8"))
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, Sq, D) and o.dtype == t
    deq = [orc.fp8_dequantize_per_head(*orc.fp8_quantize_per_head(rounded(x, t).astype(np.float32))) for x in (q, k, v)]
    ro, rl = orc.sdpa_fwd(*deq, is_causal=causal, enable_gqa=Hq != Hkv)
    # rows with few keys keep e4m3 P's 2^-4 relative error: the fp8 path's bar
    assert max_abs(host(o), ro) <= O_TOL_FP8
    assert lse_rel(host(lse), rl) <= 1e-3
