"""Pins the CPU oracle (oracle/sdpa.py) before it is trusted as the checker of the GPU kernels.

Each check is chosen so that a plausible mistake (dropped scale, wrong causal alignment, swapped
operands, wrong GQA grouping, a sign or log-base slip in the LSE or the merge, wrong fp8 rounding)
fails at least one of them; ``test_planted_mistakes_are_caught`` plants such mistakes in a copy of the
oracle and asserts that the pins reject each one.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import dtorch_cpu_path as cpu
from oracle import sdpa as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sdpa_golden.npz")


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))


# --------------------------------------------------------------------------- golden fixtures

@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("case", ["c1_small", "gqa_full", "causal_rect", "scaled"])
def test_golden_sdpa(golden, case):
    g = {k.split("/", 1)[1]: golden[k] for k in golden.files if k.startswith(case + "/")}
    scale = None if np.isnan(g["scale"]) else float(g["scale"])
    o, lse = orc.sdpa_fwd(g["q"], g["k"], g["v"], is_causal=bool(g["causal"]), scale=scale,
                          enable_gqa=g["q"].shape[1] != g["k"].shape[1])
    assert np.max(np.abs(o - g["o"])) < 2e-5
    assert np.max(np.abs(lse - g["lse"])) < 2e-5


def test_golden_decode(golden):
    g = {k.split("/", 1)[1]: golden[k] for k in golden.files if k.startswith("decode/")}
    o, _ = orc.decode(g["q"], g["k"], g["v"], g["lengths"])
    assert np.max(np.abs(o - g["o"])) < 2e-5


def test_cpu_path_decode_matches_golden_and_oracle(golden):
    # DTorch's CPU path for decode (a per-sequence libtorch call over the true length, Lq = 1, GQA) against
    # the committed fixture and the fp64 oracle; with the padding rows poisoned with NaN, so that a loop
    # reading past a sequence's length would fail.
    g = {k.split("/", 1)[1]: golden[k] for k in golden.files if k.startswith("decode/")}
    kc, vc = g["k"].copy(), g["v"].copy()
    for b, L in enumerate(g["lengths"]):
        kc[b, :, int(L):] = np.nan
        vc[b, :, int(L):] = np.nan
    o = cpu.decode(_t(g["q"]), _t(kc), _t(vc), [int(x) for x in g["lengths"]]).double().numpy()
    assert np.max(np.abs(o - g["o"])) < 2e-6
    ro, _ = orc.decode(g["q"], g["k"], g["v"], g["lengths"])
    assert np.max(np.abs(o - ro)) < 2e-5
    # a planted mistake: attending over the padded capacity instead of the true lengths
    wrong = cpu.decode(_t(g["q"]), _t(g["k"]), _t(g["v"]), [g["k"].shape[2]] * len(g["lengths"])).double().numpy()
    assert np.max(np.abs(wrong - g["o"])) > 1e-2


def test_golden_fp8(golden):
    g = {k.split("/", 1)[1]: golden[k] for k in golden.files if k.startswith("fp8/")}
    codes, desc = orc.fp8_quantize_per_head(g["x"])
    assert np.array_equal(codes, g["codes"])
    assert np.array_equal(desc, g["descale"])


# --------------------------------------------------------------------------- library routine

@pytest.mark.parametrize("B,Hq,Hkv,L,S,D,causal", [
    (1, 8, 8, 128, 128, 64, True),
    (2, 4, 2, 37, 91, 32, False),
    (1, 6, 3, 50, 20, 16, True),   # L > S, top-left causal
    (2, 2, 1, 1, 77, 64, False),   # decode-like
])
def test_oracle_matches_libtorch_cpu(B, Hq, Hkv, L, S, D, causal):
    rng = np.random.default_rng(1)
    q = rng.standard_normal((B, Hq, L, D), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    o, lse = orc.sdpa_fwd(q, k, v, is_causal=causal, enable_gqa=Hq != Hkv)
    ref = cpu.sdpa(_t(q), _t(k), _t(v), is_causal=causal, enable_gqa=Hq != Hkv).double().numpy()
    assert np.max(np.abs(o - ref)) < 2e-5
    g = Hq // Hkv
    _, ref_lse = cpu.sdpa_with_lse(_t(q), _t(k).repeat_interleave(g, 1), _t(v).repeat_interleave(g, 1),
                                   is_causal=causal)
    assert np.max(np.abs(lse - ref_lse.double().numpy())) < 2e-5


def test_offsets_match_explicit_mask():
    # bottom-right alignment (q_offset = S - L) equals torch with an explicit boolean mask
    rng = np.random.default_rng(2)
    L, S, D = 19, 45, 32
    q, k, v = (rng.standard_normal((1, 2, n, D), dtype=np.float32) for n in (L, S, S))
    o, _ = orc.sdpa_fwd(q, k, v, is_causal=True, q_offset=S - L, k_offset=0)
    mask = torch.ones(L, S, dtype=torch.bool).tril(diagonal=S - L)
    ref = cpu.sdpa(_t(q), _t(k), _t(v), attn_mask=mask).double().numpy()
    assert np.max(np.abs(o - ref)) < 2e-5


def test_fully_masked_rows_are_zero_with_neg_inf_lse():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 1, 8, 16)) for _ in range(3))
    o, lse = orc.sdpa_fwd(q, k, v, is_causal=True, q_offset=0, k_offset=4)  # rows 0..3 see nothing
    assert np.all(o[..., :4, :] == 0) and np.all(np.isneginf(lse[..., :4]))
    assert np.all(np.isfinite(lse[..., 4:]))
    # an empty key set is the same case for every row, and an empty sequence in decode likewise; the
    # merge identity (a -inf block adds nothing) then holds for it too
    o0, l0 = orc.sdpa_fwd(q, k[..., :0, :], v[..., :0, :])
    assert o0.shape == q.shape and np.all(o0 == 0) and np.all(np.isneginf(l0))
    od, ld = orc.decode(q[:, :, :1], k, v, [0])
    assert np.all(od == 0) and np.all(np.isneginf(ld))
    om, lm = orc.lse_merge([o0, o], [l0, lse])
    assert np.allclose(om, o, atol=1e-15) and np.array_equal(np.isneginf(lm), np.isneginf(lse))


# --------------------------------------------------------------------------- closed forms

def test_closed_forms():
    rng = np.random.default_rng(4)
    D, S = 32, 23
    q = rng.standard_normal((1, 1, 5, D))
    k = rng.standard_normal((1, 1, S, D))
    v = rng.standard_normal((1, 1, S, D))
    scale = 1 / math.sqrt(D)
    # single key: O = V0, LSE = scale q.k0
    o, lse = orc.sdpa_fwd(q, k[:, :, :1], v[:, :, :1])
    assert np.allclose(o, np.broadcast_to(v[:, :, :1], o.shape), atol=1e-12)
    assert np.allclose(lse[0, 0], scale * q[0, 0] @ k[0, 0, 0], atol=1e-12)
    # zero query: O = mean(V), LSE = log S
    o, lse = orc.sdpa_fwd(np.zeros_like(q), k, v)
    assert np.allclose(o, v.mean(axis=2, keepdims=True), atol=1e-12)
    assert np.allclose(lse, math.log(S), atol=1e-12)
    # constant V: O = const
    o, _ = orc.sdpa_fwd(q, k, np.full_like(v, 1.75))
    assert np.allclose(o, 1.75, atol=1e-12)
    # causal row 0 sees only key 0
    o, lse = orc.sdpa_fwd(q, k, v, is_causal=True)
    assert np.allclose(o[0, 0, 0], v[0, 0, 0], atol=1e-12)
    assert np.allclose(lse[0, 0, 0], scale * q[0, 0, 0] @ k[0, 0, 0], atol=1e-12)


def test_key_permutation_invariance():
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((2, 3, n, 16)) for n in (7, 29, 29))
    perm = rng.permutation(29)
    o1, l1 = orc.sdpa_fwd(q, k, v)
    o2, l2 = orc.sdpa_fwd(q, k[:, :, perm], v[:, :, perm])
    assert np.allclose(o1, o2, atol=1e-12) and np.allclose(l1, l2, atol=1e-12)


def test_gqa_equals_repeat_kv():
    # python/dtorch/test/modules/llama.py:80-85: expand on a new axis after the head axis, reshape
    rng = np.random.default_rng(6)
    B, Hkv, g, S, D = 2, 3, 4, 33, 16
    q = rng.standard_normal((B, Hkv * g, S, D))
    k, v = (rng.standard_normal((B, Hkv, S, D)) for _ in range(2))
    rep = lambda x: np.broadcast_to(x[:, :, None], (B, Hkv, g, S, D)).reshape(B, Hkv * g, S, D)
    o1, l1 = orc.sdpa_fwd(q, k, v, is_causal=True, enable_gqa=True)
    o2, l2 = orc.sdpa_fwd(q, rep(k), rep(v), is_causal=True)
    assert np.allclose(o1, o2, atol=1e-12) and np.allclose(l1, l2, atol=1e-12)
    with pytest.raises(ValueError):
        orc.sdpa_fwd(q, k, v)


def test_decode_equals_prefill_at_lq1():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, Smax, D = 3, 8, 2, 64, 32
    q = rng.standard_normal((B, Hq, 1, D))
    kc, vc = (rng.standard_normal((B, Hkv, Smax, D)) for _ in range(2))
    lengths = [1, 64, 30]
    o, lse = orc.decode(q, kc, vc, lengths)
    for b, L in enumerate(lengths):
        o2, l2 = orc.sdpa_fwd(q[b], kc[b, :, :L], vc[b, :, :L], enable_gqa=True)
        assert np.allclose(o[b], o2, atol=1e-12) and np.allclose(lse[b], l2, atol=1e-12)
    # is_causal with Lq=1 < Lk would keep key 0 only (top-left): decode must not behave like that
    o3, _ = orc.sdpa_fwd(q[1], kc[1], vc[1], is_causal=True, enable_gqa=True)
    assert not np.allclose(o3, o[1])


def test_paged_cache_round_trip_and_decode():
    # Scatter a contiguous cache into a shuffled page pool with an independent fancy-indexing write,
    # then gather_pages must rebuild it bit for bit and decode_paged must equal decode; the pool's
    # unused pages hold NaN, so reading a wrong page or a row past the length would show.
    rng = np.random.default_rng(12)
    B, Hq, Hkv, D, ps, max_pages = 3, 8, 2, 32, 16, 5
    lengths = np.array([80, 1, 37])
    q = rng.standard_normal((B, Hq, 1, D))
    kc, vc = (rng.standard_normal((B, Hkv, max_pages * ps, D)) for _ in range(2))
    num_pages = B * max_pages + 4
    perm = rng.permutation(num_pages)[:B * max_pages].reshape(B, max_pages)
    kp = np.full((num_pages, Hkv, ps, D), np.nan)
    vp = np.full((num_pages, Hkv, ps, D), np.nan)
    for b in range(B):
        used = -(-int(lengths[b]) // ps)  # pages holding a token of sequence b
        blocks = kc[b, :, :max_pages * ps].reshape(Hkv, max_pages, ps, D).transpose(1, 0, 2, 3)
        vblocks = vc[b, :, :max_pages * ps].reshape(Hkv, max_pages, ps, D).transpose(1, 0, 2, 3)
        kp[perm[b, :used]] = blocks[:used]
        vp[perm[b, :used]] = vblocks[:used]
    g = orc.gather_pages(kp, perm, lengths, max_len=max_pages * ps)
    for b in range(B):
        L = int(lengths[b])
        assert np.array_equal(g[b, :, :L], kc[b, :, :L])
        assert np.all(g[b, :, L:] == 0)
    o, lse = orc.decode_paged(q, kp, vp, perm, lengths)
    o2, l2 = orc.decode(q, kc, vc, lengths)
    assert np.array_equal(o, o2) and np.array_equal(lse, l2)
    assert np.all(np.isfinite(o))


# --------------------------------------------------------------------------- merge

def test_merge_equals_single_pass():
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((2, 3, n, 16)) for n in (11, 50, 50))
    o_ref, l_ref = orc.sdpa_fwd(q, k, v)
    cuts = [0, 7, 8, 31, 50]
    parts = [orc.sdpa_fwd(q, k[:, :, a:b], v[:, :, a:b]) for a, b in zip(cuts[:-1], cuts[1:])]
    o, l = orc.lse_merge([p[0] for p in parts], [p[1] for p in parts])
    assert np.allclose(o, o_ref, atol=1e-12) and np.allclose(l, l_ref, atol=1e-12)
    # associativity: ((0,1),(2,3)) == (0,1,2,3)
    a = orc.lse_merge([parts[0][0], parts[1][0]], [parts[0][1], parts[1][1]])
    b = orc.lse_merge([parts[2][0], parts[3][0]], [parts[2][1], parts[3][1]])
    o2, l2 = orc.lse_merge([a[0], b[0]], [a[1], b[1]])
    assert np.allclose(o2, o_ref, atol=1e-12) and np.allclose(l2, l_ref, atol=1e-12)
    # one block is the identity; a -inf block is a no-op
    o1, l1 = orc.lse_merge([o_ref], [l_ref])
    assert np.allclose(o1, o_ref, atol=1e-15) and np.allclose(l1, l_ref, atol=1e-15)
    junk = np.full_like(o_ref, 123.0)
    o3, l3 = orc.lse_merge([o_ref, junk], [l_ref, np.full_like(l_ref, -np.inf)])
    assert np.allclose(o3, o_ref, atol=1e-15) and np.allclose(l3, l_ref, atol=1e-15)


def test_ring_step_equals_full_causal():
    rng = np.random.default_rng(9)
    n, C, Hq, Hkv, D = 4, 16, 4, 2, 16
    q_all = rng.standard_normal((1, Hq, n * C, D))
    k_all, v_all = (rng.standard_normal((1, Hkv, n * C, D)) for _ in range(2))
    o_full, l_full = orc.sdpa_fwd(q_all, k_all, v_all, is_causal=True, enable_gqa=True)
    kch = [k_all[:, :, i * C:(i + 1) * C] for i in range(n)]
    vch = [v_all[:, :, i * C:(i + 1) * C] for i in range(n)]
    for idx in range(n):
        _, o, l = orc.ring_step(q_all[:, :, idx * C:(idx + 1) * C], kch, vch, idx)
        assert np.allclose(o, o_full[:, :, idx * C:(idx + 1) * C], atol=1e-12)
        assert np.allclose(l, l_full[:, :, idx * C:(idx + 1) * C], atol=1e-12)
    # the libtorch CPU ring restatement agrees too
    idx = 3
    o_t, l_t = cpu.ring_step(_t(q_all[:, :, idx * C:]), [_t(x) for x in kch], [_t(x) for x in vch], idx)
    assert np.max(np.abs(o_t - o_full[:, :, idx * C:])) < 2e-5
    assert np.max(np.abs(l_t - l_full[:, :, idx * C:])) < 2e-5


# --------------------------------------------------------------------------- fp8

def test_e4m3fn_all_codes_round_trip():
    codes = np.arange(256, dtype=np.uint8)
    vals = orc.e4m3fn_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).double().numpy()
    assert np.array_equal(np.isnan(vals), np.isnan(ref))
    fin = ~np.isnan(vals)
    assert np.array_equal(vals[fin], ref[fin])
    back = orc.e4m3fn_encode(vals[fin].astype(np.float32))
    # +0 and -0 both decode to 0 and re-encode with their sign
    assert np.array_equal(back, codes[fin])


def test_e4m3fn_encode_matches_torch_cast():
    rng = np.random.default_rng(10)
    grid = orc.e4m3fn_decode(np.arange(0, 127, dtype=np.uint8))  # all non-negative finite values
    mids = (grid[1:] + grid[:-1]) / 2  # exact ties -> round to even
    x = np.concatenate([grid, mids, np.nextafter(mids, 0), np.nextafter(mids, 1000),
                        rng.standard_normal(200000) * 60, rng.standard_normal(2000) * 1e-3,
                        [448, 460, 464, 470, 1e6, 2.0 ** -10, 2.0 ** -9 * 0.5, 2.0 ** -9 * 1.5]]).astype(np.float32)
    x = np.concatenate([x, -x])
    mine = orc.e4m3fn_encode(x)
    ref = torch.from_numpy(x).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_fp8_quantize_per_head_matches_torch():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 3, 40, 32)).astype(np.float32) * 2.5
    codes, desc = orc.fp8_quantize_per_head(x)
    amax = np.abs(x).max(axis=(-2, -1))
    assert np.array_equal(desc, (amax / np.float32(448)).astype(np.float32))
    y = torch.from_numpy(x) * torch.from_numpy((np.float32(448) / amax).astype(np.float32))[..., None, None]
    ref = y.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, ref)
    # the largest element of each head maps to +-448
    deq = orc.fp8_dequantize_per_head(codes, desc)
    assert np.allclose(np.abs(deq).max(axis=(-2, -1)), amax, rtol=1e-6)


# --------------------------------------------------------------------------- cost

def test_reference_cost_formula():
    # dtorch/tests/test_operator_cost.cc:171-183
    assert orc.reference_cost_flops((2, 8, 16, 64), (2, 8, 20, 64), (2, 8, 20, 64)) == 2 * 2 * 8 * 16 * 20 * (64 + 64)
    assert orc.reference_cost_flops((2, 8, 16, 64), (2, 8, 20, 64), (2, 8, 20, 64)) == 1310720


def test_algorithmic_flops_configs():
    # causal pairs: S(S+1)/2 with the diagonal; config figures used by the benchmark
    assert orc.causal_pairs(2048, 2048) == 2048 * 2049 // 2
    assert orc.algorithmic_flops(4, 32, 2048, 2048, 128, 128, True) == 137506062336
    assert orc.algorithmic_flops(1, 8, 512, 512, 64, 64, True) == 268959744
    assert orc.algorithmic_flops(1, 24, 4608, 4608, 128, 128, False) == 260919263232
    ring = 3 * orc.algorithmic_flops(1, 32, 4096, 4096, 128, 128, False) + \
        orc.algorithmic_flops(1, 32, 4096, 4096, 128, 128, True)
    assert ring == 962106228736


# --------------------------------------------------------------------------- the pins catch mistakes

def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(12)
    L, S, D = 24, 40, 16
    q, k, v = (rng.standard_normal((1, 2, n, D)).astype(np.float32) for n in (L, S, S))
    ref = cpu.sdpa(_t(q), _t(k), _t(v), is_causal=True).double().numpy()
    _, ref_lse = cpu.sdpa_with_lse(_t(q), _t(k), _t(v), is_causal=True)
    good, good_lse = orc.sdpa_fwd(q, k, v, is_causal=True)
    assert np.max(np.abs(good - ref)) < 2e-5
    # 1. bottom-right instead of top-left causal alignment
    bad, _ = orc.sdpa_fwd(q, k, v, is_causal=True, q_offset=S - L)
    assert np.max(np.abs(bad - ref)) > 1e-2
    # 2. dropped softmax scale
    bad, _ = orc.sdpa_fwd(q, k, v, is_causal=True, scale=1.0)
    assert np.max(np.abs(bad - ref)) > 1e-2
    # 3. K and V swapped
    bad, _ = orc.sdpa_fwd(q, v, k, is_causal=True)
    assert np.max(np.abs(bad - ref)) > 1e-2
    # 4. LSE in log2 instead of natural log
    assert np.max(np.abs(good_lse / math.log(2) - ref_lse.double().numpy())) > 1e-2
    # 5. interleaved instead of contiguous GQA grouping
    q4 = rng.standard_normal((1, 4, 8, D))
    k2, v2 = (rng.standard_normal((1, 2, 8, D)) for _ in range(2))
    ref_g = cpu.sdpa(_t(q4), _t(k2), _t(v2), enable_gqa=True).double().numpy()
    bad_g, _ = orc.sdpa_fwd(q4, np.tile(k2, (1, 2, 1, 1)), np.tile(v2, (1, 2, 1, 1)))
    assert np.max(np.abs(bad_g - ref_g)) > 1e-2
    # 6. merge weights without the max shift overflow/underflow: exact weights differ
    lse_big = [np.full((1,), 1000.0), np.full((1,), 999.0)]
    o, l = orc.lse_merge([np.ones((1, 1)), np.zeros((1, 1))], lse_big)
    assert np.isfinite(l).all() and abs(o[0, 0] - 1 / (1 + math.exp(-1))) < 1e-12
    # 7. fp8 round-half-up instead of half-to-even differs from torch at ties
    tie = np.float32(1.0625)  # between 1.0 and 1.125: even mantissa is 1.0
    assert orc.e4m3fn_decode(orc.e4m3fn_encode(np.array([tie])))[0] == 1.0


def test_kv_append_round_trip_and_capacity():
    # appending a sequence in pieces reproduces it; positions past S_max are dropped and lengths saturate
    rng = np.random.default_rng(31)
    B, H, S, D = 3, 2, 40, 8
    full = rng.standard_normal((B, H, S, D))
    cache = np.zeros((B, H, 32, D))
    lengths = np.array([0, 5, -3], dtype=np.int64)  # a negative length counts as 0
    start = np.maximum(lengths, 0).copy()
    pos = 0
    for n in (1, 7, 3, 30):
        orc.kv_append(cache, lengths, full[:, :, pos:pos + n])
        pos += n
    for b in range(B):
        n_in = min(32 - start[b], S)
        assert np.array_equal(cache[b, :, start[b]:start[b] + n_in], full[b, :, :n_in])
        assert lengths[b] == min(start[b] + 41, 32)
    assert np.all(cache[1, :, :5] == 0)  # rows before the starting length untouched


def test_kv_append_paged_matches_contiguous():
    rng = np.random.default_rng(32)
    B, H, D, ps, max_pages = 3, 2, 8, 16, 3
    P = B * max_pages + 2
    table = rng.permutation(P)[:B * max_pages].reshape(B, max_pages).astype(np.int32)
    pages = np.zeros((P, H, ps, D))
    contig = np.zeros((B, H, max_pages * ps, D))
    lp = np.array([0, 3, 17], dtype=np.int64)
    lc = lp.copy()
    for n in (1, 9, 16, 20):
        new = rng.standard_normal((B, H, n, D))
        orc.kv_append_paged(pages, table, lp, new)
        orc.kv_append(contig, lc, new)
    assert np.array_equal(lp, lc)
    assert np.array_equal(orc.gather_pages(pages, table, lp, max_len=max_pages * ps), np.where(
        np.arange(max_pages * ps)[None, None, :, None] < lc[:, None, None, None], contig, 0.0))


def test_kv_append_paged_drops_tokens_without_a_page():
    # The drop rule pinned against the contiguous append: a token whose slot names no page of the pool (-1,
    # or an id at or past num_pages) writes nothing, and the length advances as for a written token.  Pages
    # written through valid slots equal the contiguous cache's rows; no other page changes (a clamp into
    # the pool would overwrite page 0 or the last page, both of which hold other data here).
    rng = np.random.default_rng(34)
    B, H, D, ps, max_pages = 2, 1, 4, 16, 3
    P = 5
    table = np.array([[3, -1, 1], [2, 7, -5]], dtype=np.int32)
    pages = rng.standard_normal((P, H, ps, D))
    before = pages.copy()
    contig = np.zeros((B, H, max_pages * ps, D))
    lp = np.array([10, 12], dtype=np.int64)
    lc = lp.copy()
    new = rng.standard_normal((B, H, 30, D))
    orc.kv_append_paged(pages, table, lp, new)
    orc.kv_append(contig, lc, new)
    assert np.array_equal(lp, lc) and np.array_equal(lp, [40, 42])
    for b in range(B):
        for slot in range(max_pages):
            pg = int(table[b, slot])
            rows = range(slot * ps, (slot + 1) * ps)
            if 0 <= pg < P:
                for t in rows:
                    want = contig[b, :, t] if lc[b] - 30 <= t < lc[b] else before[pg, :, t % ps]
                    assert np.array_equal(pages[pg, :, t % ps], want), (b, slot, t)
    assert np.array_equal(pages[0], before[0]) and np.array_equal(pages[4], before[4])


def test_masks_match_libtorch():
    # boolean and additive masks, broadcast from several shapes, with and without is_causal
    rng = np.random.default_rng(33)
    B, H, L, S, D = 2, 3, 11, 17, 16
    q, k, v = (rng.standard_normal((B, H, n, D), dtype=np.float32) for n in (L, S, S))
    keep = rng.random((L, S)) < 0.6
    keep[:, 0] = True  # every row keeps a key (torch zeroes fully hidden rows; covered elsewhere)
    fmask = np.where(rng.random((B, 1, L, S)) < 0.3, np.finfo(np.float32).min, rng.standard_normal((B, 1, L, S)))
    fmask[..., 0] = 0.0
    fmask = fmask.astype(np.float32)
    for mask, causal in ((keep, False), (keep, True), (fmask, False), (fmask, True), (fmask[:, :, :1], False)):
        o, lse = orc.sdpa_fwd(q, k, v, attn_mask=mask, is_causal=causal)
        tm = torch.from_numpy(np.ascontiguousarray(mask))
        ref = cpu.sdpa(_t(q), _t(k), _t(v), attn_mask=tm, is_causal=causal).double().numpy()
        assert np.max(np.abs(o - ref)) < 2e-5, (mask.dtype, mask.shape, causal)
