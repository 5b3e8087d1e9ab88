"""The decode step under HIP graph capture: one KVCache.decode (append + split-KV decode + merge) captured,
then replayed with new inputs.  Every replay must equal the eager step bit for bit: the kernels allocate
nothing, clear nothing with memset, and read the sequence lengths from device memory, so a replay appends
at the current length and advances it.  Eager work and synchronisations run between the replays.
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
