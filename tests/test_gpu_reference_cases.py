"""The reference's own SDPA test matrix, run through this build's front end.

python/dtorch/test/operators/test_scaled_dot_product_attention.py checks DTorch against torch on:
  - fp16 [32, 32, 128, 64] uniform [0, 1) inputs with enable_gqa=True (:23-37);
  - joint attention: the concatenation of a [8, 32, 512, 64] and a [8, 32, 128, 64] stream along the
    sequence, attended and split back (:73-162), with rtol = atol = 1e-3;
  - the same 128-token shape causal and non-causal (the SageAttention case, :165-226).
Here the expected values come from the fp64 oracle on the fp16-rounded inputs, with the reference's own
tolerance, |out - ref| <= 1e-3 + 1e-3 |ref|.
"""
import numpy as np
import pytest
import torch

from oracle import sdpa as orc

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-3


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _rand(g, shape):
    return torch.rand(shape, generator=g, dtype=torch.float32).to(torch.float16)


def _close(out, ref):
    out = out.detach().float().cpu().double().numpy()
    err = np.abs(out - ref) - (ATOL + RTOL * np.abs(ref))
    assert float(err.max()) <= 0.0, float(np.abs(out - ref).max())


@pytest.mark.parametrize("is_causal", [False, True])
def test_reference_matrix_fp16_rand_32x32x128x64(is_causal):
    g = torch.Generator().manual_seed(0)
    q, k, v = (_rand(g, (32, 32, 128, 64)) for _ in range(3))
    out = _F().scaled_dot_product_attention(q.cuda(), k.cuda(), v.cuda(), is_causal=is_causal, enable_gqa=True)
    torch.cuda.synchronize()
    ref, _ = orc.sdpa_fwd(q.double().numpy(), k.double().numpy(), v.double().numpy(), is_causal=is_causal,
                          enable_gqa=True)
    _close(out, ref)


def test_reference_joint_attention_concat_split():
    g = torch.Generator().manual_seed(1)
    q, k, v = (_rand(g, (8, 32, 512, 64)) for _ in range(3))
    qo, ko, vo = (_rand(g, (8, 32, 128, 64)) for _ in range(3))
    qc, kc, vc = (torch.cat([a, b], dim=2) for a, b in ((q, qo), (k, ko), (v, vo)))
    out = _F().scaled_dot_product_attention(qc.cuda(), kc.cuda(), vc.cuda(), is_causal=False, scale=None)
    torch.cuda.synchronize()
    ref, _ = orc.sdpa_fwd(qc.double().numpy(), kc.double().numpy(), vc.double().numpy())
    n = q.shape[2]
    _close(out[:, :, :n], ref[:, :, :n])
    _close(out[:, :, n:], ref[:, :, n:])
