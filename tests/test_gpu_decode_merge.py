"""GPU parity of split-KV decode, the LSE merge and the ring-attention step against the oracle."""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _decode_case(B, Hq, Hkv, Smax, D, lengths, chunk=0, dtype=torch.bfloat16, seed=0, nan_pad=True):
    rng = np.random.default_rng(seed)
    q = randn(rng, (B, Hq, 1, D))
    kc = randn(rng, (B, Hkv, Smax, D))
    vc = randn(rng, (B, Hkv, Smax, D))
    lengths = np.asarray(lengths, dtype=np.int32)
    tk, tv = to_dev(kc, dtype), to_dev(vc, dtype)
    if nan_pad:  # padding rows must never be read
        for b, L in enumerate(lengths):
            tk[b, :, L:] = float("nan")
            tv[b, :, L:] = float("nan")
    F = _F()
    o, lse = F.decode_attention(to_dev(q, dtype), tk, tv, torch.from_numpy(lengths).cuda(), chunk=chunk)
    torch.cuda.synchronize()
    ro, rl = orc.decode(rounded(q, dtype), rounded(kc, dtype), rounded(vc, dtype), lengths)
    return host(o), host(lse), ro, rl[..., 0]


@pytest.mark.parametrize("B,Hq,Hkv,Smax,D,lengths,chunk", [
    (3, 32, 8, 1024, 128, [1, 256, 1024], 0),
    (4, 8, 8, 600, 128, [255, 257, 511, 600], 0),    # MHA, chunk boundaries
    (2, 16, 2, 700, 128, [700, 129], 128),            # GQA 8
    (2, 64, 8, 600, 128, [600, 257], 0),              # GQA 8 with Hkv 8: two 4-head workgroups per kv head
    (2, 12, 2, 300, 128, [300, 77], 0),               # GQA 6 -> subgroups of 2
    (2, 8, 4, 520, 64, [519, 3], 512),                # D = 64, chunk 512
    (4, 32, 8, 1200, 128, [383, 384, 385, 1200], 0),  # default 384-token splits: boundaries
    (2, 8, 4, 800, 64, [769, 384], 384),              # D = 64, chunk 384
])
def test_decode_small(B, Hq, Hkv, Smax, D, lengths, chunk):
    o, lse, ro, rl = _decode_case(B, Hq, Hkv, Smax, D, lengths, chunk)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_decode_fp16():
    o, lse, ro, rl = _decode_case(2, 8, 2, 400, 128, [400, 33], dtype=torch.float16, seed=2)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_decode_split_invariance_and_prefill_equality():
    rng = np.random.default_rng(3)
    B, Hq, Hkv, Smax, D = 2, 8, 2, 900, 128
    q, kc, vc = to_dev(randn(rng, (B, Hq, 1, D))), to_dev(randn(rng, (B, Hkv, Smax, D))), to_dev(
        randn(rng, (B, Hkv, Smax, D)))
    lengths = torch.tensor([900, 450], dtype=torch.int32, device="cuda")
    F = _F()
    outs = [F.decode_attention(q, kc, vc, lengths, chunk=c) for c in (128, 256, 384, 512)]
    for o, l in outs[1:]:
        assert max_abs(host(o), host(outs[0][0])) <= O_TOL_BF16
        assert lse_rel(host(l), host(outs[0][1])) <= LSE_TOL
    for b in range(B):
        L = int(lengths[b])
        po, pl = F.scaled_dot_product_attention_with_lse(q[b:b + 1], kc[b:b + 1, :, :L], vc[b:b + 1, :, :L],
                                                         enable_gqa=True)
        assert max_abs(host(outs[1][0][b:b + 1]), host(po)) <= O_TOL_BF16
        assert lse_rel(host(outs[1][1][b:b + 1]), host(pl)[..., 0]) <= LSE_TOL
    with pytest.raises(ValueError, match="chunk"):
        F.decode_attention(q, kc, vc, lengths, chunk=64)


def test_config3_decode_full_size():
    # B=64, Hq=32, Hkv=8, D=128, cache padded to 8192, lengths ~ U[512, 8192] drawn after Q, K, V
    rng = np.random.default_rng(0)
    B, Hq, Hkv, Smax, D = 64, 32, 8, 8192, 128
    q = randn(rng, (B, Hq, 1, D))
    kc = randn(rng, (B, Hkv, Smax, D))
    vc = randn(rng, (B, Hkv, Smax, D))
    lengths = rng.integers(512, 8192, size=B, endpoint=True).astype(np.int32)
    tk, tv = to_dev(kc), to_dev(vc)
    del kc, vc
    # rows at or past each sequence's length hold NaN: a kernel that read one would put NaN in O or LSE
    pad = torch.arange(Smax, device="cuda")[None, :] >= torch.from_numpy(lengths).cuda().long()[:, None]
    tk.masked_fill_(pad[:, None, :, None], float("nan"))
    tv.masked_fill_(pad[:, None, :, None], float("nan"))
    F = _F()
    o, lse = F.decode_attention(to_dev(q), tk, tv, torch.from_numpy(lengths).cuda())
    torch.cuda.synchronize()
    o, lse = host(o), host(lse)
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    kb = tk.float().cpu().numpy()
    vb = tv.float().cpu().numpy()
    ro, rl = orc.decode(rounded(q), kb, vb, lengths)
    rl = rl[..., 0]
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


# --------------------------------------------------------------------------- merge

@pytest.mark.parametrize("n,dtype", [(1, torch.bfloat16), (2, torch.bfloat16), (3, torch.float32),
                                     (4, torch.bfloat16), (16, torch.float16)])
def test_merge_random_blocks(n, dtype):
    rng = np.random.default_rng(n)
    B, H, S, D = 2, 4, 77, 128
    os_ = [randn(rng, (B, H, S, D)) for _ in range(n)]
    ls_ = [randn(rng, (B, H, S)) * 3 for _ in range(n)]
    F = _F()
    o, lse = F.lse_merge([to_dev(x, dtype) for x in os_], [torch.from_numpy(x).cuda() for x in ls_])
    ro, rl = orc.lse_merge([rounded(x, dtype) for x in os_], ls_)
    tol = 1e-5 if dtype == torch.float32 else O_TOL_BF16
    assert max_abs(host(o), ro) <= tol
    assert lse_rel(host(lse), rl) <= 1e-6


def test_merge_identity_and_neg_inf_block():
    rng = np.random.default_rng(9)
    o0 = to_dev(randn(rng, (1, 2, 64, 128)))
    l0 = torch.from_numpy(randn(rng, (1, 2, 64))).cuda()
    F = _F()
    o, l = F.lse_merge([o0], [l0])
    assert torch.equal(o, o0)
    assert torch.allclose(l, l0, atol=1e-6, rtol=0)
    junk = torch.full_like(o0, float("nan"))
    o2, l2 = F.lse_merge([o0, junk], [l0, torch.full_like(l0, float("-inf"))])
    assert torch.equal(o2, o0)
    assert torch.allclose(l2, l0, atol=1e-6, rtol=0)


def test_merge_of_kv_splits_equals_single_pass():
    rng = np.random.default_rng(10)
    q, k, v = to_dev(randn(rng, (1, 4, 200, 128))), to_dev(randn(rng, (1, 4, 700, 128))), to_dev(
        randn(rng, (1, 4, 700, 128)))
    F = _F()
    ref_o, ref_l = F.scaled_dot_product_attention_with_lse(q, k, v)
    cuts = [0, 64, 300, 301, 700]
    parts = [F.scaled_dot_product_attention_with_lse(q, k[:, :, a:b].contiguous(), v[:, :, a:b].contiguous())
             for a, b in zip(cuts[:-1], cuts[1:])]
    o, l = F.lse_merge([p[0] for p in parts], [p[1] for p in parts])
    assert max_abs(host(o), host(ref_o)) <= O_TOL_BF16
    assert lse_rel(host(l), host(ref_l)) <= LSE_TOL


# --------------------------------------------------------------------------- ring step

def test_ring_step_small_all_ranks():
    rng = np.random.default_rng(11)
    n, C, Hq, Hkv, D = 4, 96, 8, 2, 128
    q_all = randn(rng, (1, Hq, n * C, D))
    k_all = randn(rng, (1, Hkv, n * C, D))
    v_all = randn(rng, (1, Hkv, n * C, D))
    ro, rl = orc.sdpa_fwd(rounded(q_all), rounded(k_all), rounded(v_all), is_causal=True, enable_gqa=True)
    F = _F()
    kch = [to_dev(k_all[:, :, i * C:(i + 1) * C]) for i in range(n)]
    vch = [to_dev(v_all[:, :, i * C:(i + 1) * C]) for i in range(n)]
    for idx in range(n):
        o, l = F.ring_attention_step(to_dev(q_all[:, :, idx * C:(idx + 1) * C]), kch, vch, idx)
        assert max_abs(host(o), ro[:, :, idx * C:(idx + 1) * C]) <= O_TOL_BF16
        assert lse_rel(host(l), rl[:, :, idx * C:(idx + 1) * C]) <= LSE_TOL


def test_config4_ring_step_full_size():
    # Q chunk of 4096 tokens (global chunk 3) against 4 KV chunks of 4096: 1 causal diagonal + 3 full,
    # Hq=32, Hkv=8, D=128, B=1, bf16; every head and row against DTorch's CPU path for the same step
    # (libtorch's fp32 CPU flash attention per block, then the LSE merge), and sampled rows against the
    # single pass over all 16384 keys (which pins the block offsets independently of the merge).
    rng = np.random.default_rng(0)
    C, Hq, Hkv, D = 4096, 32, 8, 128
    q = randn(rng, (1, Hq, C, D))
    k = [randn(rng, (1, Hkv, C, D)) for _ in range(4)]
    v = [randn(rng, (1, Hkv, C, D)) for _ in range(4)]
    F = _F()
    o, l, blocks = F.ring_attention_step(to_dev(q), [to_dev(x) for x in k], [to_dev(x) for x in v], 3,
                                         return_blocks=True)
    torch.cuda.synchronize()
    assert len(blocks) == 4
    from oracle import dtorch_cpu_path as cpu
    f32 = lambda x: torch.from_numpy(rounded(x).astype(np.float32))
    ro, rl = cpu.ring_step(f32(q), [f32(x) for x in k], [f32(x) for x in v], 3)
    ho, hl = host(o), host(l)
    err, lerr = max_abs(ho, ro), lse_rel(hl, rl)
    print(f"C4 full size: max-abs {err:.3e}, LSE rel {lerr:.3e}")
    assert err <= O_TOL_BF16
    assert lerr <= LSE_TOL
    k_all = np.concatenate(k, axis=2)
    v_all = np.concatenate(v, axis=2)
    rows = np.r_[0:64, 2000:2064, 4032:4096]
    for h in (0, 17, 31):
        hk = h // 4
        qs = rounded(q[0, h, rows])[None]
        # global query position = 3*C + row; keys 0..16383 under the causal rule
        sro, srl = _causal_rows(qs[0], rounded(k_all[0, hk]), rounded(v_all[0, hk]), 3 * C + rows)
        assert max_abs(ho[0, h, rows], sro) <= O_TOL_BF16, h
        assert lse_rel(hl[0, h, rows], srl) <= LSE_TOL, h


def _causal_rows(q, k, v, qpos):
    scale = 1 / np.sqrt(q.shape[-1])
    logits = (q @ k.T) * scale
    keep = np.arange(k.shape[0])[None, :] <= qpos[:, None]
    logits = np.where(keep, logits, -np.inf)
    m = logits.max(-1, keepdims=True)
    p = np.exp(logits - m)
    s = p.sum(-1, keepdims=True)
    return (p @ v) / s, (m + np.log(s))[:, 0]


def test_decode_zero_length_sequences():
    # lengths of 0 (and lengths clamped to S_max) are defined: an empty sequence gives O = 0, LSE = -inf;
    # the other sequences of the batch are unaffected
    rng = np.random.default_rng(9)
    B, Hq, Hkv, Smax, D = 4, 8, 2, 300, 128
    q, kc, vc = randn(rng, (B, Hq, 1, D)), randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    lengths = np.array([0, 300, 0, 130], dtype=np.int32)
    F = _F()
    o, lse = F.decode_attention(to_dev(q), to_dev(kc), to_dev(vc), torch.from_numpy(lengths).cuda())
    torch.cuda.synchronize()
    o, lse = host(o), host(lse)
    for b in (0, 2):
        assert np.all(o[b] == 0) and np.all(np.isneginf(lse[b])), b
    ro, rl = orc.decode(rounded(q[[1, 3]]), rounded(kc[[1, 3]]), rounded(vc[[1, 3]]), lengths[[1, 3]])
    assert max_abs(o[[1, 3]], ro) <= O_TOL_BF16
    assert lse_rel(lse[[1, 3]], rl[..., 0]) <= LSE_TOL


# --------------------------------------------------------------------------- paged decode

def _paged_pool(rng, lengths, Hkv, D, ps, spare_pages=3, token_major=False, dtype=torch.bfloat16):
    """A page pool holding each sequence's tokens on randomly chosen pages, NaN on the pages no
    sequence uses, and a block table whose unused slots hold an id far outside the pool."""
    need = [(int(L) + ps - 1) // ps for L in lengths]
    P = sum(need) + spare_pages
    max_pages = max(max(need), 1) + 1
    perm = rng.permutation(P)
    bt = np.full((len(lengths), max_pages), 1 << 30, dtype=np.int32)
    used, off = set(), 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[off:off + n]
        used.update(int(x) for x in perm[off:off + n])
        off += n
    kp = randn(rng, (P, Hkv, ps, D))
    vp = randn(rng, (P, Hkv, ps, D))
    free = [p for p in range(P) if p not in used]
    kp[free] = np.nan
    vp[free] = np.nan
    # rows past the end of the last page of each sequence are never read either
    for b, L in enumerate(lengths):
        if int(L) % ps:
            last = bt[b, need[b] - 1]
            kp[last, :, int(L) % ps:] = np.nan
            vp[last, :, int(L) % ps:] = np.nan
    if token_major:  # pool stored [P, ps, Hkv, D], handed over as a permuted view
        tk = to_dev(kp.transpose(0, 2, 1, 3), dtype).permute(0, 2, 1, 3)
        tv = to_dev(vp.transpose(0, 2, 1, 3), dtype).permute(0, 2, 1, 3)
    else:
        tk, tv = to_dev(kp, dtype), to_dev(vp, dtype)
    return kp, vp, tk, tv, bt, max_pages


def _gather_dev(pool, bt, lengths, S):
    """Contiguous [B, Hkv, S, D] device cache with the paged cache's tokens, zeros elsewhere."""
    B = len(lengths)
    out = torch.zeros((B, pool.shape[1], S, pool.shape[3]), dtype=pool.dtype, device=pool.device)
    ps = pool.shape[2]
    for b in range(B):
        L = int(lengths[b])
        if L == 0:
            continue
        t = torch.arange(L, device=pool.device)
        pages = torch.from_numpy(bt[b]).to(pool.device).long()[t // ps]
        out[b, :, :L] = pool[pages, :, t % ps].permute(1, 0, 2)
    return out


@pytest.mark.parametrize("ps,B,Hq,Hkv,D,lengths,chunk,token_major", [
    (16, 3, 32, 8, 128, [1, 250, 513], 0, False),
    (64, 4, 8, 8, 128, [64, 65, 300, 0], 0, False),      # MHA, page-aligned and empty sequences
    (128, 2, 16, 2, 128, [700, 129], 256, True),         # GQA 8, token-major pool
    (256, 2, 12, 2, 128, [1000, 77], 512, False),        # GQA 6
    (16, 2, 8, 4, 64, [519, 3], 128, True),              # D = 64
    (32, 2, 64, 8, 128, [600, 40], 0, False),            # GQA 8 with Hkv 8
])
def test_decode_paged_small(ps, B, Hq, Hkv, D, lengths, chunk, token_major):
    rng = np.random.default_rng(ps + B)
    q = randn(rng, (B, Hq, 1, D))
    lengths = np.asarray(lengths, dtype=np.int32)
    kp, vp, tk, tv, bt, max_pages = _paged_pool(rng, lengths, Hkv, D, ps, token_major=token_major)
    F = _F()
    tq, tl = to_dev(q), torch.from_numpy(lengths).cuda()
    o, lse = F.decode_attention_paged(tq, tk, tv, torch.from_numpy(bt).cuda(), tl, chunk=chunk)
    torch.cuda.synchronize()
    ho, hl = host(o), host(lse)
    for b in np.flatnonzero(lengths == 0):
        assert np.all(ho[b] == 0) and np.all(np.isneginf(hl[b])), b
    nz = np.flatnonzero(lengths > 0)
    ro, rl = orc.decode_paged(rounded(q[nz]), rounded(np.nan_to_num(kp)), rounded(np.nan_to_num(vp)),
                              bt[nz], lengths[nz])
    assert max_abs(ho[nz], ro) <= O_TOL_BF16
    assert lse_rel(hl[nz], rl[..., 0]) <= LSE_TOL
    # same arithmetic as the contiguous decode over the gathered cache of S_max = max_pages * page_size
    S = max_pages * ps
    co, cl = F.decode_attention(tq, _gather_dev(tk, bt, lengths, S), _gather_dev(tv, bt, lengths, S), tl,
                                chunk=chunk)
    torch.cuda.synchronize()
    assert torch.equal(o, co)
    assert torch.equal(lse, cl)


def test_decode_paged_fp16_and_errors():
    rng = np.random.default_rng(21)
    lengths = np.array([333, 40], dtype=np.int32)
    q = randn(rng, (2, 8, 1, 128))
    kp, vp, tk, tv, bt, _ = _paged_pool(rng, lengths, 2, 128, 32, dtype=torch.float16)
    F = _F()
    tb, tl = torch.from_numpy(bt).cuda(), torch.from_numpy(lengths).cuda()
    o, lse = F.decode_attention_paged(to_dev(q, torch.float16), tk, tv, tb, tl)
    torch.cuda.synchronize()
    ro, rl = orc.decode_paged(rounded(q, torch.float16), rounded(np.nan_to_num(kp), torch.float16),
                              rounded(np.nan_to_num(vp), torch.float16), bt, lengths)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl[..., 0]) <= LSE_TOL
    with pytest.raises(ValueError, match="page"):  # page size 24 is not a power of two
        F.decode_attention_paged(to_dev(q, torch.float16), tk[:, :, :24], tv[:, :, :24], tb, tl)
    with pytest.raises(ValueError):
        F.decode_attention_paged(to_dev(q, torch.float16), tk, tv, tb.long(), tl)


def test_decode_paged_16_token_pages_fp16():
    # 16-token pages of fp16 rows take the path that loads each wave's page ids up front: the sequences'
    # last chunks read table slots past their last page (an id far outside the pool) and rows past their
    # end (NaN), which must not reach the result; bit-identical to the contiguous decode
    rng = np.random.default_rng(23)
    lengths = np.array([1, 383, 384, 385, 1500, 0, 770], dtype=np.int32)
    B, Hq, Hkv, D, ps = len(lengths), 16, 4, 128, 16
    q = randn(rng, (B, Hq, 1, D))
    kp, vp, tk, tv, bt, max_pages = _paged_pool(rng, lengths, Hkv, D, ps, dtype=torch.float16)
    F = _F()
    tq, tl = to_dev(q, torch.float16), torch.from_numpy(lengths).cuda()
    o, lse = F.decode_attention_paged(tq, tk, tv, torch.from_numpy(bt).cuda(), tl)
    S = max_pages * ps
    co, cl = F.decode_attention(tq, _gather_dev(tk, bt, lengths, S), _gather_dev(tv, bt, lengths, S), tl)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    assert torch.equal(o, co) and torch.equal(lse, cl)
    nz = np.flatnonzero(lengths > 0)
    ro, rl = orc.decode_paged(rounded(q[nz], torch.float16), rounded(np.nan_to_num(kp), torch.float16),
                              rounded(np.nan_to_num(vp), torch.float16), bt[nz], lengths[nz])
    assert max_abs(host(o)[nz], ro) <= O_TOL_BF16
    assert lse_rel(host(lse)[nz], rl[..., 0]) <= LSE_TOL


def test_config3_decode_paged_full_size():
    # the full-size decode workload (B=64, Hq=32, Hkv=8, D=128, lengths ~ U[512, 8192]) in 16-token
    # pages scattered over the pool: bit-identical to the contiguous decode over the gathered cache,
    # and sampled sequences against the oracle
    rng = np.random.default_rng(5)
    B, Hq, Hkv, D, ps = 64, 32, 8, 128, 16
    lengths = rng.integers(512, 8192, size=B, endpoint=True).astype(np.int32)
    need = (lengths + ps - 1) // ps
    P = int(need.sum())
    max_pages = int(need.max())
    perm = rng.permutation(P).astype(np.int32)
    bt = np.zeros((B, max_pages), dtype=np.int32)
    off = 0
    for b in range(B):
        bt[b, :need[b]] = perm[off:off + need[b]]
        off += need[b]
    g = torch.Generator(device="cuda").manual_seed(5)
    tk = torch.randn((P, Hkv, ps, D), generator=g, device="cuda").to(torch.bfloat16)
    tv = torch.randn((P, Hkv, ps, D), generator=g, device="cuda").to(torch.bfloat16)
    tq = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    tb, tl = torch.from_numpy(bt).cuda(), torch.from_numpy(lengths).cuda()
    F = _F()
    o, lse = F.decode_attention_paged(tq, tk, tv, tb, tl)
    S = max_pages * ps
    kc, vc = _gather_dev(tk, bt, lengths, S), _gather_dev(tv, bt, lengths, S)
    co, cl = F.decode_attention(tq, kc, vc, tl)
    torch.cuda.synchronize()
    assert torch.equal(o, co)
    assert torch.equal(lse, cl)
    pick = [0, int(np.argmax(lengths)), int(np.argmin(lengths)), B - 1]
    ro, rl = orc.decode(host(tq[pick]), host(kc[pick]), host(vc[pick]), lengths[pick])
    assert max_abs(host(o[pick]), ro) <= O_TOL_BF16
    assert lse_rel(host(lse[pick]), rl[..., 0]) <= LSE_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Hq,Hkv", [(8, 4), (16, 4)])   # groups of 2 and 4 heads per kv head
def test_decode_d64_default_splits(dtype, Hq, Hkv):
    # D = 64 with chunk = 0 takes the 384-token default splits (96 tokens per wave): lengths on both
    # sides of a split boundary and an empty sequence, contiguous and paged
    lengths = np.array([383, 384, 385, 0, 1000], dtype=np.int32)
    B, D, Smax = len(lengths), 64, 1024
    o, lse, ro, rl = _decode_case(B, Hq, Hkv, Smax, D, lengths, chunk=0, dtype=dtype, seed=Hq + Hkv)
    nz = lengths > 0
    assert np.all(o[~nz] == 0) and np.all(np.isneginf(lse[~nz]))
    assert max_abs(o[nz], ro[nz]) <= O_TOL_BF16
    assert lse_rel(lse[nz], rl[nz]) <= LSE_TOL
    rng = np.random.default_rng(Hq)
    q = randn(rng, (B, Hq, 1, D))
    kp, vp, tk, tv, bt, max_pages = _paged_pool(rng, lengths, Hkv, D, 16, dtype=dtype)
    F = _F()
    tq, tl = to_dev(q, dtype), torch.from_numpy(lengths).cuda()
    po, pl = F.decode_attention_paged(tq, tk, tv, torch.from_numpy(bt).cuda(), tl, chunk=0)
    torch.cuda.synchronize()
    hpo, hpl = host(po), host(pl)
    assert np.all(hpo[~nz] == 0) and np.all(np.isneginf(hpl[~nz]))
    idx = np.flatnonzero(nz)
    pro, prl = orc.decode_paged(rounded(q[idx], dtype), rounded(np.nan_to_num(kp), dtype),
                                rounded(np.nan_to_num(vp), dtype), bt[idx], lengths[idx])
    assert max_abs(hpo[idx], pro) <= O_TOL_BF16
    assert lse_rel(hpl[idx], prl[..., 0]) <= LSE_TOL
    S = max_pages * 16
    co, cl = F.decode_attention(tq, _gather_dev(tk, bt, lengths, S), _gather_dev(tv, bt, lengths, S), tl, chunk=0)
    torch.cuda.synchronize()
    assert torch.equal(po, co) and torch.equal(pl, cl)


def test_decode_paged_pool_past_4gb_takes_the_64bit_path():
    # Page offsets of a kv head that do not fit 32 bits run the 64-bit flat loads; pools below that run
    # 32-bit buffer offsets.  Both must give the bits of the contiguous kernel over the gathered cache.
    # One 4.3 GB allocation holds K and V interleaved by page ([pages, 2, Hkv, ps, D]), so each pool's page
    # stride is 16 KB and its span passes 4 GB; only the pages in the block table are written.
    B, Hq, Hkv, ps, D = 2, 8, 2, 16, 128
    num_pages = (1 << 32) // (2 * Hkv * ps * D * 2) + 2
    pool = torch.empty(num_pages, 2, Hkv, ps, D, dtype=torch.bfloat16, device="cuda")
    rng = np.random.default_rng(31)
    lengths = np.array([300, 517], dtype=np.int32)
    maxp = 33
    used = np.concatenate([np.arange(3), rng.choice(np.arange(3, num_pages), size=2 * maxp - 3, replace=False)])
    bt = used.reshape(B, maxp).astype(np.int32)
    bt[1, -1] = num_pages - 1  # the last page of the pool, past 4 GB
    vals = torch.randn(len(used), 2, Hkv, ps, D, device="cuda").to(torch.bfloat16)
    pool[torch.from_numpy(bt.reshape(-1).astype(np.int64)).cuda()] = vals
    kp, vp = pool[:, 0], pool[:, 1]
    q = torch.randn(B, Hq, 1, D, device="cuda").to(torch.bfloat16)
    tb, tl = torch.from_numpy(bt).cuda(), torch.from_numpy(lengths).cuda()
    F = _F()
    o, lse = F.decode_attention_paged(q, kp, vp, tb, tl, chunk=128)
    # the contiguous kernel on the gathered rows, same split length
    S = maxp * ps
    kc = kp[tb.long()].permute(0, 2, 1, 3, 4).reshape(B, Hkv, S, D).contiguous()
    vc = vp[tb.long()].permute(0, 2, 1, 3, 4).reshape(B, Hkv, S, D).contiguous()
    o2, lse2 = F.decode_attention(q, kc, vc, tl, chunk=128)
    # the same pages in a small pool: 32-bit offsets
    small_k, small_v = kp[tb.long().reshape(-1)].contiguous(), vp[tb.long().reshape(-1)].contiguous()
    tb_small = torch.arange(B * maxp, dtype=torch.int32, device="cuda").reshape(B, maxp)
    o3, lse3 = F.decode_attention_paged(q, small_k, small_v, tb_small, tl, chunk=128)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(o3, o2) and torch.equal(lse3, lse2)
    del pool, kp, vp
    torch.cuda.empty_cache()
