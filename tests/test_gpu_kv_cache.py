"""GPU parity of the KV-cache append and of a decode loop over the cache against the oracle."""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_kv_append_contiguous(dtype, D):
    rng = np.random.default_rng(41)
    B, Hkv, S_max, n = 4, 2, 100, 3
    kc, vc = to_dev(randn(rng, (B, Hkv, S_max, D)), dtype), to_dev(randn(rng, (B, Hkv, S_max, D)), dtype)
    lengths = np.array([0, 50, 99, -2], dtype=np.int32)  # 99: two of the three tokens fall past S_max
    # the projection's natural layout [B, n, Hkv, D], handed over transposed
    kn = to_dev(randn(rng, (B, n, Hkv, D)), dtype).transpose(1, 2)
    vn = to_dev(randn(rng, (B, n, Hkv, D)), dtype).transpose(1, 2)
    ref_k, ref_v = _bits(kc), _bits(vc)
    ref_lk, ref_lv = lengths.astype(np.int64), lengths.astype(np.int64)
    orc.kv_append(ref_k, ref_lk, _bits(kn.contiguous()))
    orc.kv_append(ref_v, ref_lv, _bits(vn.contiguous()))
    tl = torch.from_numpy(lengths).cuda()
    _F().kv_cache_append(kc, vc, tl, kn, vn)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kc), ref_k)
    assert np.array_equal(_bits(vc), ref_v)
    assert np.array_equal(tl.cpu().numpy(), ref_lk)


def test_kv_append_paged():
    rng = np.random.default_rng(42)
    B, Hkv, D, ps, max_pages, n = 3, 2, 128, 16, 4, 5
    P = B * max_pages + 3
    table = rng.permutation(P)[:B * max_pages].reshape(B, max_pages).astype(np.int32)
    kp, vp = to_dev(randn(rng, (P, Hkv, ps, D))), to_dev(randn(rng, (P, Hkv, ps, D)))
    lengths = np.array([0, 14, 61], dtype=np.int32)  # crosses a page boundary; runs past the capacity
    kn, vn = to_dev(randn(rng, (B, Hkv, n, D))), to_dev(randn(rng, (B, Hkv, n, D)))
    ref_k, ref_v = _bits(kp), _bits(vp)
    lk, lv = lengths.astype(np.int64), lengths.astype(np.int64)
    orc.kv_append_paged(ref_k, table, lk, _bits(kn))
    orc.kv_append_paged(ref_v, table, lv, _bits(vn))
    tl = torch.from_numpy(lengths).cuda()
    _F().kv_cache_append_paged(kp, vp, torch.from_numpy(table).cuda(), tl, kn, vn)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kp), ref_k)
    assert np.array_equal(_bits(vp), ref_v)
    assert np.array_equal(tl.cpu().numpy(), lk)


@pytest.mark.parametrize("paged", [False, True])
def test_decode_loop_equals_causal_attention(paged):
    # prefill L0 prompt tokens, then decode one token at a time: every output row equals the causal
    # attention row of the full sequence (the reference's Llama port recomputes exactly that each step)
    from dtorch_amd.nn.kv_cache import KVCache, PagedKVCache
    rng = np.random.default_rng(43 + paged)
    B, Hq, Hkv, D, L0, steps = 2, 8, 2, 128, 37, 24
    T = L0 + steps
    q, k, v = randn(rng, (B, Hq, T, D)), randn(rng, (B, Hkv, T, D)), randn(rng, (B, Hkv, T, D))
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=True, enable_gqa=True)
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    if paged:
        cache = PagedKVCache(B, Hkv, num_pages=16, page_size=16, max_pages=5, head_dim=D)
    else:
        cache = KVCache(B, Hkv, max_len=T, head_dim=D)
    out = cache.prefill(tq[:, :, :L0], tk[:, :, :L0], tv[:, :, :L0])
    torch.cuda.synchronize()
    assert max_abs(host(out), ro[:, :, :L0]) <= O_TOL_BF16
    for j in range(L0, T):
        s = slice(j, j + 1)
        o = cache.decode(tq[:, :, s], tk[:, :, s], tv[:, :, s])
        torch.cuda.synchronize()
        assert max_abs(host(o), ro[:, :, s]) <= O_TOL_BF16, j
    assert np.array_equal(cache.lengths.cpu().numpy(), np.full(B, T))


@pytest.mark.parametrize("paged", [False, True])
def test_decode_covers_the_longest_sequence_not_the_capacity(paged):
    # A cache far larger than its sequences: decode runs over a view up to the longest one (the split grid
    # follows S_max), and must equal the call over the whole cache bit for bit.
    from dtorch_amd.nn.kv_cache import KVCache, PagedKVCache
    F = _F()
    rng = np.random.default_rng(44 + paged)
    B, Hq, Hkv, D, L0 = 3, 8, 2, 128, 700
    q, k, v = randn(rng, (B, Hq, L0 + 3, D)), randn(rng, (B, Hkv, L0 + 3, D)), randn(rng, (B, Hkv, L0 + 3, D))
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    if paged:
        cache = PagedKVCache(B, Hkv, num_pages=B * 200, page_size=16, max_pages=200, head_dim=D)
    else:
        cache = KVCache(B, Hkv, max_len=16384, head_dim=D)
    cache.prefill(tq[:, :, :L0], tk[:, :, :L0], tv[:, :, :L0])
    for j in range(L0, L0 + 3):
        s = slice(j, j + 1)
        o = cache.decode(tq[:, :, s], tk[:, :, s], tv[:, :, s])
        if paged:
            assert cache._span_pages() == (j + 1 + 15) // 16 < 200
            full = F.decode_attention_paged(tq[:, :, s], cache.k, cache.v, cache.block_table, cache.lengths)[0]
        else:
            assert cache._span() == j + 1 < cache.capacity
            full = F.decode_attention(tq[:, :, s], cache.k, cache.v, cache.lengths)[0]
        torch.cuda.synchronize()
        assert torch.equal(o, full), j


def test_kv_cache_capacity_is_checked_on_the_host():
    from dtorch_amd.nn.kv_cache import KVCache, PagedKVCache
    cache = KVCache(1, 1, max_len=4, head_dim=64)
    x = torch.zeros(1, 1, 3, 64, dtype=torch.bfloat16, device="cuda")
    cache.append(x, x)
    with pytest.raises(ValueError, match="full"):
        cache.append(x, x)
    paged = PagedKVCache(1, 1, num_pages=1, page_size=16, max_pages=4, head_dim=64)
    y = torch.zeros(1, 1, 17, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="pages"):
        paged.append(y, y)


def test_kv_append_paged_drops_tokens_without_a_page():
    # A block-table entry that names no page of the pool (an unassigned -1 slot, or a corrupt id at or past
    # num_pages) drops the token: no page changes, the length still advances.  A clamp into the pool would
    # write another sequence's cache.
    rng = np.random.default_rng(47)
    B, Hkv, D, ps, max_pages, n = 3, 2, 64, 16, 3, 6
    P = 7
    table = np.array([[4, -1, -1], [1, 9, 2], [0, 5, 3]], dtype=np.int32)  # 9 >= num_pages
    kp, vp = to_dev(randn(rng, (P, Hkv, ps, D))), to_dev(randn(rng, (P, Hkv, ps, D)))
    lengths = np.array([13, 13, 13], dtype=np.int32)  # tokens 13..18: the last three cross into slot 1
    kn, vn = to_dev(randn(rng, (B, Hkv, n, D))), to_dev(randn(rng, (B, Hkv, n, D)))
    before_k, before_v = _bits(kp), _bits(vp)
    ref_k, ref_v = before_k.copy(), before_v.copy()
    lk, lv = lengths.astype(np.int64), lengths.astype(np.int64)
    orc.kv_append_paged(ref_k, table, lk, _bits(kn))
    orc.kv_append_paged(ref_v, table, lv, _bits(vn))
    tl = torch.from_numpy(lengths).cuda()
    _F().kv_cache_append_paged(kp, vp, torch.from_numpy(table).cuda(), tl, kn, vn)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kp), ref_k) and np.array_equal(_bits(vp), ref_v)
    assert np.array_equal(tl.cpu().numpy(), np.full(B, 19))
    # only rows 13..15 of the pages in slot 0 changed; page 6 (never named) and the pages of slot 1 of
    # sequences 1 and 2 (their tokens 16..18 went to pages 9 -> dropped, and 5) are checked explicitly
    changed = np.nonzero(np.any(_bits(kp) != before_k, axis=(1, 2, 3)))[0].tolist()
    assert changed == [0, 1, 4, 5]
    assert np.array_equal(_bits(kp)[6], before_k[6])


def test_paged_graph_replays_past_assigned_pages_write_nothing_else():
    # A decode step captured in a HIP graph and replayed past a sequence's assigned pages: the tokens past
    # them meet table slots of -1 and are dropped, every page that no sequence owns stays bit-identical, the
    # owned pages equal the oracle's append, and sync_lengths() reports the overrun.
    from dtorch_amd.nn.kv_cache import PagedKVCache
    rng = np.random.default_rng(48)
    B, Hq, Hkv, D, ps, L0, replays = 2, 8, 2, 64, 16, 20, 15
    cache = PagedKVCache(B, Hkv, num_pages=8, page_size=ps, max_pages=4, head_dim=D)
    cache.k.copy_(to_dev(randn(rng, tuple(cache.k.shape))))
    cache.v.copy_(to_dev(randn(rng, tuple(cache.v.shape))))
    q, k, v = (to_dev(randn(rng, (B, h, L0, D))) for h in (Hq, Hkv, Hkv))
    cache.prefill(q, k, v)  # two pages per sequence; slots 2 and 3 stay -1
    torch.cuda.synchronize()
    table = cache.block_table.cpu().numpy()
    assert np.array_equal(table[:, 2:], np.full((B, 2), -1))
    owned = set(table[table >= 0].tolist())
    before_k, before_v = _bits(cache.k), _bits(cache.v)
    sq, sk, sv = (to_dev(randn(rng, (B, h, 1, D))) for h in (Hq, Hkv, Hkv))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cache.decode(sq, sk, sv)
    torch.cuda.synchronize()
    ref_k, ref_v = before_k.copy(), before_v.copy()
    lk = np.full(B, L0, dtype=np.int64)
    lv = lk.copy()
    for _ in range(replays):  # lengths 20 -> 35; positions 32..34 fall in slot 2
        graph.replay()
        torch.cuda.synchronize()  # eager work between replays
        orc.kv_append_paged(ref_k, table, lk, _bits(sk))
        orc.kv_append_paged(ref_v, table, lv, _bits(sv))
    assert np.array_equal(_bits(cache.k), ref_k) and np.array_equal(_bits(cache.v), ref_v)
    for pg in range(cache.k.shape[0]):
        if pg not in owned:
            assert np.array_equal(_bits(cache.k)[pg], before_k[pg]), pg
            assert np.array_equal(_bits(cache.v)[pg], before_v[pg]), pg
    assert np.array_equal(cache.lengths.cpu().numpy(), np.full(B, L0 + replays))
    with pytest.raises(RuntimeError, match="past the assigned pages"):
        cache.sync_lengths()
