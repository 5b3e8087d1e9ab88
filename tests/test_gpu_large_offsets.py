"""GPU parity at the 32-bit offset limits of the inline-asm tile loops.

The head-dim-128 program (prefill_rows64.hip) and the head-dim-512 program (prefill_wide512.hip) compute a
key tile's byte offset from the head's first key row as one 32-bit scalar product, so the host sends a call to
them only while (Sk + 128) * pitch (head dim 128) or (Sk + 64) * pitch (head dim 512) stays below 2^31 bytes;
past that, the call takes the kernel that addresses tiles in 64 bits (prefill_fwd_kernel, prefill_wide_kernel).
Each case views K and V as rows of one ~2 GB buffer at a pitch just below or just above the limit, so the last
tiles sit near 2^31 bytes from the first, and checks the output bit for bit against the same call on
contiguous copies (the two kernels of each head dim return identical bits) and against the fp64 oracle.
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


def _pitch(Sk, margin, D, above):
    """Row pitch in elements (a multiple of 8) just below or just above (Sk + margin) * pitch * 2 = 2^31."""
    p = ((1 << 31) - 1) // ((Sk + margin) * 2)
    p -= p % 8
    if above:
        p += 8
    assert ((Sk + margin) * p * 2 >= 1 << 31) == above and p >= 2 * D
    return p


def _strided_kv(k, v, pitch, device):
    """K and V as [B, Hkv, Sk, D] views of one buffer whose key rows are `pitch` elements apart (V at +D)."""
    B, H, Sk, D = k.shape
    buf = torch.zeros(Sk * pitch, dtype=torch.bfloat16, device=device)
    shape, stride = (B, H, Sk, D), (0, 0, pitch, 1)
    sk = torch.as_strided(buf, shape, stride, 0)
    sv = torch.as_strided(buf, shape, stride, D)
    sk.copy_(k)
    sv.copy_(v)
    return buf, sk, sv


@pytest.mark.parametrize("D,Hq,causal,margin,above", [
    (128, 4, True, 128, False),   # head-dim-128 program, last tile ~2^31 bytes in
    (128, 4, True, 128, True),    # just past the limit: prefill_fwd_kernel
    (128, 1, False, 128, False),  # the non-GQA row layout of the same program
    (512, 1, False, 64, False),   # head-dim-512 program
])
def test_key_rows_near_2_31_bytes(D, Hq, causal, margin, above):
    rng = np.random.default_rng(31 + D + Hq + int(above))
    Sq, Sk = 192, 1000
    q, k, v = randn(rng, (1, Hq, Sq, D)), randn(rng, (1, 1, Sk, D)), randn(rng, (1, 1, Sk, D))
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    pitch = _pitch(Sk, margin, D, above)
    print(f"D={D} Hq={Hq} causal={causal} pitch={pitch} elements, last row at {(Sk - 1) * pitch * 2} bytes",
          flush=True)
    buf, sk, sv = _strided_kv(tk, tv, pitch, tq.device)
    F = _F()
    gqa = Hq > 1
    o, lse = F.scaled_dot_product_attention_with_lse(tq, sk, sv, is_causal=causal, enable_gqa=gqa)
    o2, lse2 = F.scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=causal, enable_gqa=gqa)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.equal(lse, lse2)
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=causal, enable_gqa=gqa)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL
    del buf, sk, sv
