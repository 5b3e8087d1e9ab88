"""GPU parity of prefill at head dims other than 64/128/256/512, and with Dv != D.

The reference hands any head dims to libtorch (scaled_dot_product_attention_op.cc:107-109) and gives the
output v's last axis (:26-29).  Here bf16/fp16 take any D and Dv that are multiples of 8 up to 512: the
kernels run at the next of 64/128/256/512 and read the columns past the real dims as zeros.  Each case
is checked against the fp64 oracle on the same rounded inputs at the task's bars (max-abs 2e-2 on O,
LSE 1e-3 relative).
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


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,Dv,causal,dtype", [
    (2, 4, 2, 200, 200, 96, 96, True, torch.bfloat16),     # 96 -> kernel 128
    (1, 4, 4, 130, 257, 80, 80, False, torch.float16),     # 80 -> 128, ragged
    (1, 2, 2, 100, 100, 32, 32, True, torch.bfloat16),     # 32 -> 64
    (2, 8, 2, 150, 150, 72, 72, True, torch.bfloat16),     # 72 -> 128, GQA 4
    (1, 4, 1, 120, 300, 192, 128, True, torch.bfloat16),   # Q/K 192, V 128 -> 256 (wide kernel)
    (1, 2, 2, 90, 90, 128, 64, False, torch.bfloat16),     # Dv < D at 128
    (1, 2, 2, 90, 90, 64, 128, True, torch.float16),       # Dv > D at 128
    (1, 2, 1, 70, 70, 160, 160, False, torch.bfloat16),    # 160 -> 256
    (1, 1, 1, 64, 130, 320, 320, True, torch.bfloat16),    # 320 -> 512
    (1, 2, 2, 64, 64, 512, 256, False, torch.float16),     # Dv < D at 512
    (1, 3, 3, 33, 40, 8, 8, False, torch.bfloat16),        # the smallest head dim
])
def test_prefill_head_dims(B, Hq, Hkv, Sq, Sk, D, Dv, causal, dtype):
    rng = np.random.default_rng(D * 1000 + Dv)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, Dv))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                     is_causal=causal, enable_gqa=Hq != Hkv)
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, Sq, Dv) and o.dtype == dtype
    ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), is_causal=causal,
                          enable_gqa=Hq != Hkv)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


def test_head_dim_96_with_mask_offsets_and_strides():
    # a boolean mask, causal offsets and [B, S, H, D]-major views on a padded head dim
    rng = np.random.default_rng(96)
    B, H, Sq, Sk, D = 2, 4, 100, 120, 96
    q, k, v = randn(rng, (B, Sq, H, D)), randn(rng, (B, Sk, H, D)), randn(rng, (B, Sk, H, D))
    mask = rng.random((Sq, Sk)) > 0.3
    mask[:, 0] = True
    F = _F()
    tq, tk, tv = (to_dev(x).transpose(1, 2) for x in (q, k, v))
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=True, q_offset=20, k_offset=0,
                                                     attn_mask=torch.from_numpy(mask).cuda())
    torch.cuda.synchronize()
    rq, rk, rv = (rounded(x).transpose(0, 2, 1, 3) for x in (q, k, v))
    ro, rl = orc.sdpa_fwd(rq, rk, rv, attn_mask=mask, is_causal=True, q_offset=20, k_offset=0)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL


def test_sdpa_op_output_takes_v_head_dim():
    # SdpaOp::InferOutputMetaInfo and Compute: O has q's shape with v's last axis, in q's dtype
    rng = np.random.default_rng(7)
    q, k, v = randn(rng, (1, 8, 64, 192)), randn(rng, (1, 8, 80, 192)), randn(rng, (1, 8, 80, 128))
    F = _F()
    o = F.scaled_dot_product_attention(to_dev(q), to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    assert o.shape == (1, 8, 64, 128) and o.dtype == torch.bfloat16
    ro, _ = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v))
    assert max_abs(host(o), ro) <= O_TOL_BF16


def test_unsupported_head_dims_raise():
    # head dims above 512 have no kernel in any dtype; they raise rather than fall back
    F = _F()
    y = torch.zeros(1, 2, 16, 520, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="head dim"):
        F.scaled_dot_product_attention(y, y, y)
    w = torch.zeros(1, 1, 16, 520, dtype=torch.bfloat16, device="cuda")  # 16-bit: up to 512
    with pytest.raises(ValueError, match="head dim"):
        F.scaled_dot_product_attention(w, w, w)


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,Dv,causal,dtype,opt", [
    (2, 8, 2, 190, 190, 100, 100, True, torch.bfloat16, ""),     # 100 -> 104 (kernel 128), GQA 4
    (1, 4, 4, 77, 129, 36, 36, False, torch.float16, ""),        # 36 -> 40 (kernel 64)
    (1, 2, 2, 64, 100, 100, 52, True, torch.bfloat16, ""),       # D and Dv padded apart
    (1, 2, 1, 70, 90, 300, 300, False, torch.bfloat16, ""),      # 300 -> 304 (wide kernel 512)
    (1, 4, 2, 66, 66, 66, 66, True, torch.float32, ""),          # fp32: 66 -> 68 (kernel 128)
    (1, 2, 1, 70, 90, 300, 300, False, torch.float32, ""),       # fp32: 300 (wide fp32 kernel 512)
    (1, 2, 2, 64, 100, 136, 100, True, torch.float32, ""),       # fp32: 136 / 100 (wide fp32 kernel 256)
    (1, 4, 2, 128, 128, 100, 100, False, torch.bfloat16, "native_fp8"),  # 100 -> 104 -> 128 on the fp8 kernel
])
def test_head_dims_off_the_kernel_grid_are_zero_padded(B, Hq, Hkv, Sq, Sk, D, Dv, causal, dtype, opt):
    # libtorch takes any head dim (scaled_dot_product_attention_op.cc:107-109); the host operator pads q, k on D
    # and v on Dv with zero columns to the kernels' multiple (8, or 4 for fp32), keeps the scale of the real D and
    # cuts the output back to Dv
    rng = np.random.default_rng(D * 100 + Dv + Sk)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, Dv))
    F = _F()
    print(f"padded head dims: D={D} Dv={Dv} {dtype} {opt or 'native'}", flush=True)
    o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                     is_causal=causal, enable_gqa=Hq != Hkv,
                                                     sdpa_option=F.SdpaOption(sage_attn_type=opt or None))
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, Sq, Dv) and o.dtype == dtype and o.is_contiguous()
    if opt == "native_fp8":
        # against exact attention on the dequantized inputs (per-head e4m3fn of the real columns: the zero
        # padding changes no absmax), which leaves the kernel's own error, at the fp8 kernel bars
        deq = [orc.fp8_dequantize_per_head(*orc.fp8_quantize_per_head(rounded(x, dtype).astype(np.float32)))
               for x in (q, k, v)]
        ro, rl = orc.sdpa_fwd(*deq, is_causal=causal, enable_gqa=Hq != Hkv, scale=1.0 / np.sqrt(D))
    else:
        ro, rl = orc.sdpa_fwd(rounded(q, dtype), rounded(k, dtype), rounded(v, dtype), is_causal=causal,
                              enable_gqa=Hq != Hkv)
    if dtype == torch.float32:
        assert max_abs(host(o), ro) <= 1e-4 and lse_rel(host(lse), rl) <= 1e-5
    elif opt == "native_fp8":
        assert max_abs(host(o), ro) <= 3e-2 and lse_rel(host(lse), rl) <= 1e-3
    else:
        assert max_abs(host(o), ro) <= O_TOL_BF16 and lse_rel(host(lse), rl) <= LSE_TOL
    # the explicit scale of the real D gives the same bits as the default
    o2, _ = F.scaled_dot_product_attention_with_lse(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype),
                                                    is_causal=causal, enable_gqa=Hq != Hkv, scale=1.0 / np.sqrt(D),
                                                    sdpa_option=F.SdpaOption(sage_attn_type=opt or None))
    torch.cuda.synchronize()
    assert torch.equal(o, o2)


def _decode(B, Hq, Hkv, Smax, D, lengths, dtype, seed, chunk=0):
    rng = np.random.default_rng(seed)
    q, kc, vc = randn(rng, (B, Hq, 1, D)), randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    lengths = np.asarray(lengths, dtype=np.int32)
    tk, tv = to_dev(kc, dtype), to_dev(vc, dtype)
    for b, L in enumerate(lengths):  # rows past the length are never read
        tk[b, :, L:] = float("nan")
        tv[b, :, L:] = float("nan")
    F = _F()
    o, lse = F.decode_attention(to_dev(q, dtype), tk, tv, torch.from_numpy(lengths).cuda(), chunk=chunk)
    torch.cuda.synchronize()
    assert o.shape == (B, Hq, 1, D)
    return q, kc, vc, lengths, host(o), host(lse)


@pytest.mark.parametrize("D,dtype,Hq,Hkv,chunk", [
    (96, torch.bfloat16, 32, 8, 0),
    (80, torch.float16, 8, 2, 0),
    (32, torch.bfloat16, 4, 4, 256),
    (48, torch.float32, 8, 4, 0),     # fp32 rows: multiples of 4 elements
    (100, torch.float32, 6, 2, 384),
    (120, torch.bfloat16, 16, 2, 128),  # 8 heads per kv head
])
def test_decode_head_dims(D, dtype, Hq, Hkv, chunk):
    lengths = [0, 383, 384, 385, 900]
    q, kc, vc, lengths, o, lse = _decode(len(lengths), Hq, Hkv, 900, D, lengths, dtype, D, chunk)
    nz = lengths > 0
    assert np.all(o[~nz] == 0) and np.all(np.isneginf(lse[~nz]))
    ro, rl = orc.decode(rounded(q[nz], dtype), rounded(kc[nz], dtype), rounded(vc[nz], dtype), lengths[nz])
    tol = 1e-5 if dtype == torch.float32 else O_TOL_BF16
    assert max_abs(o[nz], ro) <= tol
    assert lse_rel(lse[nz], rl[..., 0]) <= (1e-5 if dtype == torch.float32 else LSE_TOL)


def test_paged_decode_and_kv_cache_loop_head_dim_96():
    # the KV-cache loop at a padded head dim: a 37-token prefill then single-token decode steps reproduce
    # the causal rows of the full sequence, for the padded and the paged cache
    from dtorch_amd.nn.kv_cache import KVCache, PagedKVCache
    rng = np.random.default_rng(960)
    B, Hq, Hkv, D, P, N = 2, 8, 2, 96, 37, 12
    q, k, v = randn(rng, (B, Hq, P + N, D)), randn(rng, (B, Hkv, P + N, D)), randn(rng, (B, Hkv, P + N, D))
    ro, _ = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=True, enable_gqa=True)
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    for cache in (KVCache(B, Hkv, 128, D), PagedKVCache(B, Hkv, 16, 16, 8, D)):
        out = cache.prefill(tq[:, :, :P], tk[:, :, :P], tv[:, :, :P])
        assert max_abs(host(out), ro[:, :, :P]) <= O_TOL_BF16
        for i in range(P, P + N):
            o1 = cache.decode(tq[:, :, i:i + 1], tk[:, :, i:i + 1], tv[:, :, i:i + 1])
            assert max_abs(host(o1), ro[:, :, i:i + 1]) <= O_TOL_BF16, (type(cache).__name__, i)


@pytest.mark.parametrize("D,n,dtype", [(96, 3, torch.bfloat16), (256, 2, torch.float16), (200, 4, torch.bfloat16),
                                       (512, 5, torch.float32), (8, 2, torch.bfloat16)])
def test_lse_merge_head_dims(D, n, dtype):
    rng = np.random.default_rng(D + n)
    B, H, S = 2, 3, 77
    os_ = [randn(rng, (B, H, S, D)) for _ in range(n)]
    ls = [randn(rng, (B, H, S)) * 3 for _ in range(n)]
    ls[0][0, 0, :5] = -np.inf  # a block that saw no key on some rows
    F = _F()
    o, lse = F.lse_merge([to_dev(x, dtype) for x in os_], [torch.from_numpy(x.astype(np.float32)).cuda() for x in ls])
    torch.cuda.synchronize()
    ro, rl = orc.lse_merge([rounded(x, dtype) for x in os_], [x.astype(np.float32).astype(np.float64) for x in ls])
    tol = 1e-5 if dtype == torch.float32 else O_TOL_BF16  # 16-bit outputs: their own rounding of |O| <~ 3
    assert max_abs(host(o), ro) <= tol
    assert lse_rel(host(lse), rl) <= 1e-5


@pytest.mark.parametrize("D,Dv,Sk", [(96, 96, 200), (96, 64, 130), (192, 128, 100), (40, 40, 77)])
def test_padded_columns_and_rows_past_the_end_are_never_read(D, Dv, Sk):
    # K and V are column slices of wider buffers whose extra columns, and the rows after the last key of
    # every head, hold NaN: a read of either would turn the output into NaN
    rng = np.random.default_rng(D + Dv + Sk)
    B, H, Sq, W = 2, 2, 70, 256
    q, k, v = randn(rng, (B, H, Sq, D)), randn(rng, (B, H, Sk, D)), randn(rng, (B, H, Sk, Dv))
    kb = torch.full((B, H, Sk + 1, W), float("nan"), dtype=torch.bfloat16, device="cuda")
    vb = torch.full((B, H, Sk + 1, W), float("nan"), dtype=torch.bfloat16, device="cuda")
    kb[:, :, :Sk, :D] = to_dev(k)
    vb[:, :, :Sk, :Dv] = to_dev(v)
    tk, tv = kb[:, :, :Sk, :D], vb[:, :, :Sk, :Dv]
    F = _F()
    for causal in (False, True):
        o, lse = F.scaled_dot_product_attention_with_lse(to_dev(q), tk, tv, is_causal=causal)
        torch.cuda.synchronize()
        ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=causal)
        assert max_abs(host(o), ro) <= O_TOL_BF16, causal
        assert lse_rel(host(lse), rl) <= LSE_TOL, causal
    # decode over the same caches (D = Dv only): padded chunks and rows past the length unread
    if D == Dv and D <= 128:
        lengths = torch.tensor([Sk, Sk // 2], dtype=torch.int32, device="cuda")
        q1 = to_dev(q[:, :, :1])
        o, lse = F.decode_attention(q1, kb[:, :, :, :D], vb[:, :, :, :D], lengths)
        torch.cuda.synchronize()
        ro, rl = orc.decode(rounded(q[:, :, :1]), rounded(k), rounded(v), [Sk, Sk // 2])
        assert max_abs(host(o), ro) <= O_TOL_BF16
        assert lse_rel(host(lse), rl[..., 0]) <= LSE_TOL
