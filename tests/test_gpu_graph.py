"""HIP graph capture.  The decode step: one KVCache.decode (append + split-KV decode + merge) captured,
then replayed with new inputs.  Every replay must equal the eager step bit for bit: the kernels allocate
nothing, clear nothing with memset, and read the sequence lengths from device memory, so a replay appends
at the current length and advances it.  The prefill entry points (causal GQA, wide heads with key blocks and
their merge, a mask, native fp8 in three launches and in four with its tail split, the ring step) captured
the same way.  Eager work and
synchronisations run between the replays.
"""
import numpy as np
import pytest
import torch

from tests.attn_cases import randn, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_step_graph_replays_match_eager(dtype):
    from dtorch_amd.nn.kv_cache import KVCache
    rng = np.random.default_rng(11)
    B, Hq, Hkv, D, L0, steps = 2, 8, 2, 128, 300, 6
    T = L0 + steps
    q, k, v = (to_dev(randn(rng, (B, h, T, D)), dtype) for h in (Hq, Hkv, Hkv))

    eager = KVCache(B, Hkv, max_len=T, head_dim=D, dtype=dtype)
    eager.prefill(q[:, :, :L0], k[:, :, :L0], v[:, :, :L0])
    ref = [eager.decode(q[:, :, j:j + 1], k[:, :, j:j + 1], v[:, :, j:j + 1]).clone() for j in range(L0, T)]
    torch.cuda.synchronize()

    cache = KVCache(B, Hkv, max_len=T, head_dim=D, dtype=dtype)
    cache.prefill(q[:, :, :L0], k[:, :, :L0], v[:, :, :L0])
    sq, sk, sv = (torch.zeros(B, h, 1, D, dtype=dtype, device="cuda") for h in (Hq, Hkv, Hkv))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cache.decode(sq, sk, sv)  # captured: nothing runs until replay
    torch.cuda.synchronize()
    assert int(cache.lengths[0]) == L0  # capture did not execute the append
    for n, j in enumerate(range(L0, T)):
        sq.copy_(q[:, :, j:j + 1])
        sk.copy_(k[:, :, j:j + 1])
        sv.copy_(v[:, :, j:j + 1])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref[n]), j
        assert np.array_equal(cache.lengths.cpu().numpy(), np.full(B, j + 1))
    assert torch.equal(cache.k, eager.k) and torch.equal(cache.v, eager.v)
    # the replays advanced the device lengths past the host copy: eager decode keeps covering the whole
    # capacity until sync_lengths() refreshes it
    assert cache._span() == cache.capacity
    assert np.array_equal(cache.sync_lengths(), np.full(B, T))
    assert cache._span() == T


@pytest.mark.parametrize("case", ["causal_gqa", "wide_key_blocks", "masked", "native_fp8", "native_fp8_tail",
                                  "ring_step", "stream_k"])
def test_prefill_graph_replays_match_eager(case):
    # The prefill entry points under capture, replayed with new inputs copied into the captured tensors:
    # every replay equals the eager call bit for bit.  The wide-head case takes the key-block split, so its
    # workspace and the LSE merge launch are captured too; the fp8 tail case (832 query blocks over 768 slots)
    # takes the tail split and its merge launch; the stream-K case (128 row-layout items on 256 CUs) its
    # records in the workspace and their merge launch.
    import dtorch_amd.nn.functional as F
    rng = np.random.default_rng(sum(map(ord, case)))
    shapes = {"causal_gqa": (2, 8, 2, 300, 300, 128), "wide_key_blocks": (1, 2, 1, 256, 2048, 512),
              "masked": (1, 4, 4, 200, 260, 64), "native_fp8": (1, 4, 2, 256, 256, 128),
              "native_fp8_tail": (1, 32, 8, 3300, 2100, 128),
              "ring_step": (1, 4, 2, 128, 256, 128),  # a 128-row Q chunk against two 128-key chunks
              "stream_k": (1, 8, 8, 4096, 4096, 128)}
    B, Hq, Hkv, Sq, Sk, D = shapes[case]
    mask = torch.from_numpy(rng.random((Sq, Sk)) < 0.7).cuda() if case == "masked" else None
    opt = F.SdpaOption(sage_attn_type="native_fp8") if case.startswith("native_fp8") else F.SdpaOption()

    def call(q, k, v):
        if case == "ring_step":
            ks, vs = [k[:, :, :128], k[:, :, 128:]], [v[:, :, :128], v[:, :, 128:]]
            return F.ring_attention_step(q, ks, vs, q_chunk_index=1)
        return F.scaled_dot_product_attention_with_lse(q, k, v, is_causal=case in ("causal_gqa",), enable_gqa=True,
                                                       attn_mask=mask, sdpa_option=opt)

    inputs = [tuple(to_dev(randn(rng, (B, h, s, D))) for h, s in ((Hq, Sq), (Hkv, Sk), (Hkv, Sk))) for _ in range(3)]
    ref = [tuple(t.clone() for t in call(*x)) for x in inputs]
    torch.cuda.synchronize()
    sq, sk, sv = (torch.zeros_like(t) for t in inputs[0])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(sq, sk, sv)
    torch.cuda.synchronize()
    for n in (0, 1, 2, 0):
        for dst, src in zip((sq, sk, sv), inputs[n]):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, ref[n])), (case, n)
