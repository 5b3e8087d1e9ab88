"""GPU parity of the stream-K form of the head-dim-128 row layout (prefill_rows64_sk_kernel + its merge).

Non-causal bf16/fp16 calls at D = 128 whose groups are not multiples of 4 (MHA included: the MMDiT joint
attention of the reference's diffusers ports, python/dtorch/applications/huggingface/diffusers/models/
attention_processor.py) run as 256-row work items, one workgroup per CU.  When those items do not fill
whole rounds of the CUs, and the caller passes the workspace dtattn_prefill_workspace_size() asks for, each
CU takes an equal share of all (item, key tile) units; items a share boundary cuts are finished from
partial records by a second launch.  Checked against the same call without the workspace (the plain grid of
prefill_rows64_kernel): rows of uncut items bit for bit, rows of cut items within 8e-3 on O and 1e-5 on the
LSE, and both against the fp64 oracle on sampled rows; the split's run-to-run determinism; and that causal,
grouped-query (groups of 4k) and whole-round calls plan no workspace.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs

pytestmark = pytest.mark.gpu


def _args(q, k, v, o, lse, causal):
    from dtorch_amd import _lib
    a = _lib.PrefillArgs()
    a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    a.B, a.Hq, a.Sq, a.D = q.shape
    a.Hkv, a.Sk, a.Dv = k.shape[1], k.shape[2], v.shape[3]
    for dst, t in ((a.q_stride, q), (a.k_stride, k), (a.v_stride, v), (a.o_stride, o)):
        dst[0], dst[1], dst[2] = t.stride(0), t.stride(1), t.stride(2)
    a.lse_stride[0], a.lse_stride[1] = lse.stride(0), lse.stride(1)
    a.dtype = a.o_dtype = 0 if q.dtype == torch.bfloat16 else 1
    a.causal = int(causal)
    return a


def _ws_bytes(q, k, v, causal=False):
    from dtorch_amd import _lib
    lib = _lib.cabi()
    o = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], device=q.device)
    a = _args(q, k, v, o, lse, causal)
    lib.dtattn_prefill_workspace_size.argtypes = [ctypes.c_void_p]
    lib.dtattn_prefill_workspace_size.restype = ctypes.c_size_t
    return lib.dtattn_prefill_workspace_size(ctypes.byref(a))


def _prefill(q, k, v, workspace):
    """dtattn_prefill_fwd through ctypes, non-causal, with or without the workspace it asks for."""
    from dtorch_amd import _lib
    lib = _lib.cabi()
    o = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], device=q.device)
    a = _args(q, k, v, o, lse, False)
    ws = None
    if workspace:
        n = _ws_bytes(q, k, v)
        ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), n
    lib.dtattn_prefill_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.dtattn_last_error.restype = ctypes.c_char_p
    st = lib.dtattn_prefill_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.dtattn_last_error().decode()
    return o, lse


def _cut_items(B, Hq, Sq, Sk, G):
    """Indices of the 256-row items a share boundary cuts (the kernel's own partition)."""
    nqb, nt = (Sq + 255) // 256, (Sk + 63) // 64
    units = nqb * B * Hq * nt
    cut = set()
    for r in range(1, G):
        u = units * r // G
        if u % nt:
            cut.add(u // nt)
    return cut, nqb


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,dtype", [
    (1, 24, 24, 4096, 4096, torch.bfloat16),  # 384 items over 256 CUs: 1.5 rounds
    (1, 8, 8, 4096, 4096, torch.bfloat16),    # 128 items: half the CUs idle on the plain grid
    (1, 12, 6, 2000, 5000, torch.bfloat16),   # groups of 2, ragged Sq and Sk (a tail tile of 8 keys)
    (2, 6, 6, 1500, 3000, torch.float16),     # fp16, two sequences
])
def test_streamk_against_plain_grid_and_oracle(B, Hq, Hkv, Sq, Sk, dtype):
    G = torch.cuda.get_device_properties(0).multi_processor_count & ~7
    g = torch.Generator(device="cuda").manual_seed(Sq + Sk)
    q = torch.randn(B, Hq, Sq, 128, generator=g, device="cuda").to(dtype)
    k = torch.randn(B, Hkv, Sk, 128, generator=g, device="cuda").to(dtype)
    v = torch.randn(B, Hkv, Sk, 128, generator=g, device="cuda").to(dtype)
    print(f"stream-K B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} {dtype}, {G} workgroups", flush=True)
    assert _ws_bytes(q, k, v) > 0, "no stream-K plan"
    o, lse = _prefill(q, k, v, True)
    o2, lse2 = _prefill(q, k, v, True)
    ou, lseu = _prefill(q, k, v, False)
    import dtorch_amd.nn.functional as F
    fo, flse = F.scaled_dot_product_attention_with_lse(q, k, v, enable_gqa=Hq != Hkv)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(fo, o) and torch.equal(flse, lse)  # the operator passes the workspace
    cut, nqb = _cut_items(B, Hq, Sq, Sk, G)
    assert cut, "no item was cut"
    whole = torch.ones(B, Hq, Sq, dtype=torch.bool, device="cuda")
    for i in cut:
        qb, bh = i % nqb, i // nqb
        whole[bh // Hq, bh % Hq, qb * 256:(qb + 1) * 256] = False
    assert torch.equal(o[whole], ou[whole]) and torch.equal(lse[whole], lseu[whole])
    assert not torch.equal(o[~whole], ou[~whole])  # the merge ran
    assert float((o.float() - ou.float()).abs().max()) <= 8e-3
    assert float(((lse - lseu).abs() / lseu.abs().clamp(min=1)).max()) <= 1e-5
    # rows of a cut item (its first and last rows) and of an uncut one, against the oracle
    i = min(cut)
    qb, bh = i % nqb, i // nqb
    b, h = bh // Hq, bh % Hq
    rows = np.unique(np.clip([qb * 256, qb * 256 + 100, qb * 256 + 255, 0, Sq - 1], 0, Sq - 1))
    qs = q[b:b + 1, h:h + 1, rows].float().cpu().double().numpy()
    hk = h // (Hq // Hkv)
    ks = k[b:b + 1, hk:hk + 1].float().cpu().double().numpy()
    vs = v[b:b + 1, hk:hk + 1].float().cpu().double().numpy()
    ro, rl = orc.sdpa_fwd(qs, ks, vs)
    assert max_abs(host(o[b:b + 1, h:h + 1, rows]), ro) <= O_TOL_BF16
    assert lse_rel(host(lse[b:b + 1, h:h + 1, rows]), rl) <= LSE_TOL


def test_streamk_not_planned():
    dev = "cuda"
    q = torch.randn(1, 24, 4608, 128, device=dev, dtype=torch.bfloat16)
    kv = torch.randn(1, 24, 4608, 128, device=dev, dtype=torch.bfloat16)
    assert _ws_bytes(q, kv, kv, causal=True) == 0                 # causal calls
    kv8 = torch.randn(1, 6, 4608, 128, device=dev, dtype=torch.bfloat16)
    assert _ws_bytes(q, kv8, kv8) == 0                            # groups of 4: the grouped-query form
    q16 = torch.randn(2, 32, 4096, 128, device=dev, dtype=torch.bfloat16)
    kv16 = torch.randn(2, 32, 4096, 128, device=dev, dtype=torch.bfloat16)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _ws_bytes(q16, kv16, kv16) == 0                    # 1024 items: four whole rounds
    q64 = torch.randn(1, 24, 4608, 64, device=dev, dtype=torch.bfloat16)
    assert _ws_bytes(q64, q64, q64) == 0                          # head dim 64
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _ws_bytes(q, kv, kv) == 0  # 432 items of 72 tiles: the records would cost more than the last round
