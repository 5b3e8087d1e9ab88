"""GPU parity of the fp32 decode (contiguous and paged), the fp32 KV-cache append and an fp32 decode loop.

Same bar as the fp32 prefill: max |O - O_ref| <= 1e-5 and LSE |d| / max(|ref|, 1) <= 1e-5 against the fp64
oracle on the same fp32 inputs; the append is bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import host, lse_rel, max_abs, randn
from tests.test_gpu_decode_merge import _gather_dev, _paged_pool

pytestmark = pytest.mark.gpu

O_TOL_F32 = 1e-5
LSE_TOL_F32 = 1e-5


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("B,Hq,Hkv,Smax,D,lengths,chunk", [
    (3, 32, 8, 1024, 128, [1, 256, 1024], 0),
    (4, 8, 8, 600, 128, [255, 257, 511, 600], 0),     # MHA, chunk boundaries
    (2, 16, 2, 700, 128, [700, 129], 128),             # GQA 8, 8-head workgroups
    (2, 64, 8, 600, 128, [600, 0], 0),                 # two 4-head workgroups per kv head; an empty sequence
    (2, 12, 2, 300, 128, [300, 77], 512),              # GQA 6 -> subgroups of 2
    (2, 8, 4, 520, 64, [519, 3], 256),                 # D = 64
    (3, 8, 2, 1000, 128, [383, 385, 1000], 384),       # 384-token splits: three 32-token sub-blocks per wave
])
def test_decode_fp32(B, Hq, Hkv, Smax, D, lengths, chunk):
    rng = np.random.default_rng(70 + Smax)
    q, kc, vc = randn(rng, (B, Hq, 1, D)), randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    lengths = np.asarray(lengths, dtype=np.int32)
    tk, tv = _dev(kc), _dev(vc)
    for b, L in enumerate(lengths):  # padding rows must never be read
        tk[b, :, L:] = float("nan")
        tv[b, :, L:] = float("nan")
    o, lse = _F().decode_attention(_dev(q), tk, tv, torch.from_numpy(lengths).cuda(), chunk=chunk)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    o, lse = host(o), host(lse)
    for b in np.flatnonzero(lengths == 0):
        assert np.all(o[b] == 0) and np.all(np.isneginf(lse[b]))
    nz = np.flatnonzero(lengths > 0)
    ro, rl = orc.decode(q[nz].astype(np.float64), kc[nz].astype(np.float64), vc[nz].astype(np.float64), lengths[nz])
    assert max_abs(o[nz], ro) <= O_TOL_F32
    assert lse_rel(lse[nz], rl[..., 0]) <= LSE_TOL_F32


@pytest.mark.parametrize("token_major", [False, True])
def test_decode_paged_fp32(token_major):
    rng = np.random.default_rng(80 + token_major)
    lengths = np.array([333, 40, 1, 700], dtype=np.int32)
    B, Hq, Hkv, D, ps = 4, 16, 4, 128, 16
    q = randn(rng, (B, Hq, 1, D))
    kp, vp, tk, tv, bt, max_pages = _paged_pool(rng, lengths, Hkv, D, ps, token_major=token_major,
                                                dtype=torch.float32)
    F = _F()
    tq, tl, tb = _dev(q), torch.from_numpy(lengths).cuda(), torch.from_numpy(bt).cuda()
    o, lse = F.decode_attention_paged(tq, tk, tv, tb, tl)
    torch.cuda.synchronize()
    ro, rl = orc.decode_paged(q.astype(np.float64), np.nan_to_num(kp).astype(np.float64),
                              np.nan_to_num(vp).astype(np.float64), bt, lengths)
    assert max_abs(host(o), ro) <= O_TOL_F32
    assert lse_rel(host(lse), rl[..., 0]) <= LSE_TOL_F32
    # the paged kernel's arithmetic is the contiguous one's over the gathered cache
    S = max_pages * ps
    co, cl = F.decode_attention(tq, _gather_dev(tk, bt, lengths, S), _gather_dev(tv, bt, lengths, S), tl)
    torch.cuda.synchronize()
    assert torch.equal(o, co) and torch.equal(lse, cl)


def test_kv_append_fp32_bit_exact():
    rng = np.random.default_rng(90)
    B, Hkv, S_max, D, n = 3, 2, 50, 64, 4
    kc, vc = _dev(randn(rng, (B, Hkv, S_max, D))), _dev(randn(rng, (B, Hkv, S_max, D)))
    lengths = np.array([0, 20, 48], dtype=np.int32)  # 48: two of the four tokens fall past S_max
    kn = _dev(randn(rng, (B, n, Hkv, D))).transpose(1, 2)
    vn = _dev(randn(rng, (B, n, Hkv, D))).transpose(1, 2)
    bits = lambda t: t.detach().contiguous().view(torch.int32).cpu().numpy()
    ref_k, ref_v = bits(kc), bits(vc)
    lk, lv = lengths.astype(np.int64), lengths.astype(np.int64)
    orc.kv_append(ref_k, lk, bits(kn))
    orc.kv_append(ref_v, lv, bits(vn))
    tl = torch.from_numpy(lengths).cuda()
    _F().kv_cache_append(kc, vc, tl, kn, vn)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc), ref_k) and np.array_equal(bits(vc), ref_v)
    assert np.array_equal(tl.cpu().numpy(), lk)


@pytest.mark.parametrize("paged", [False, True])
def test_decode_loop_fp32_equals_causal_attention(paged):
    from dtorch_amd.nn.kv_cache import KVCache, PagedKVCache
    rng = np.random.default_rng(95 + paged)
    B, Hq, Hkv, D, L0, steps = 2, 8, 2, 128, 29, 20
    T = L0 + steps
    q, k, v = randn(rng, (B, Hq, T, D)), randn(rng, (B, Hkv, T, D)), randn(rng, (B, Hkv, T, D))
    ro, _ = orc.sdpa_fwd(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), is_causal=True,
                         enable_gqa=True)
    tq, tk, tv = _dev(q), _dev(k), _dev(v)
    if paged:
        cache = PagedKVCache(B, Hkv, num_pages=8, page_size=16, max_pages=4, head_dim=D, dtype=torch.float32)
    else:
        cache = KVCache(B, Hkv, max_len=T, head_dim=D, dtype=torch.float32)
    out = cache.prefill(tq[:, :, :L0], tk[:, :, :L0], tv[:, :, :L0])
    torch.cuda.synchronize()
    assert max_abs(host(out), ro[:, :, :L0]) <= O_TOL_F32
    for j in range(L0, T):
        s = slice(j, j + 1)
        o = cache.decode(tq[:, :, s], tk[:, :, s], tv[:, :, s])
        torch.cuda.synchronize()
        assert max_abs(host(o), ro[:, :, s]) <= O_TOL_F32, j
