"""GPU parity of the stream-K form of the head-dim-128 row layout (prefill_rows64_sk_kernel + its merge).

Non-causal bf16/fp16 calls at D = 128 run as work items of one workgroup per CU: 256 rows of one head (MHA
and groups that are not multiples of 4, the MMDiT joint attention of the reference's diffusers ports among
them: python/dtorch/applications/huggingface/diffusers/models/attention_processor.py), or the 4 query heads
of a kv head over 64 rows (groups of 4k: the ring step's key blocks, python/dtorch/nn/
scaled_dot_product_attention_with_cp.py:87-101).  When those items do not fill whole rounds of the CUs, and
the caller passes the workspace dtattn_prefill_workspace_size() asks for, each CU takes an equal share of
all (item, key tile) units; items a share boundary cuts are finished by a second launch from partial records
(O over the piece's row sums in the input dtype, as the ring step's blocks keep it, and fp32 row maxima and
sums).  Checked against the same call without the workspace (the plain grids of prefill_rows64_kernel and
prefill_rows64_gqa_kernel): rows of uncut items bit for bit, rows of cut items within 8e-3 on O and 1e-5 on
the LSE, and both against the fp64 oracle on sampled rows; the split's run-to-run determinism; and that
causal, whole-round and C5a-shaped calls plan no workspace.
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


def _cut_rows(B, Hq, Hkv, Sq, Sk, G):
    """Mask [B, Hq, Sq] of the rows of items a share boundary cuts (the kernel's own partition), and one cut
    item's (b, heads, rows)."""
    group = Hq // Hkv
    gqa = group % 4 == 0
    nqb, nt = ((Sq + 63) // 64 if gqa else (Sq + 255) // 256), (Sk + 63) // 64
    units = nqb * B * (Hq // 4 if gqa else Hq) * nt
    cut = sorted({units * r // G // nt for r in range(1, G) if (units * r // G) % nt})
    mask = torch.zeros(B, Hq, Sq, dtype=torch.bool)
    items = []
    for i in cut:
        qb, rest = i % nqb, i // nqb
        if gqa:
            nsub = group // 4
            b, r2 = rest // (Hkv * nsub), rest % (Hkv * nsub)
            heads = [(r2 // nsub) * group + (r2 % nsub) * 4 + w for w in range(4)]
            rows = slice(qb * 64, min(Sq, qb * 64 + 64))
        else:
            b, heads, rows = rest // Hq, [rest % Hq], slice(qb * 256, min(Sq, qb * 256 + 256))
        for h in heads:
            mask[b, h, rows] = True
        items.append((b, heads, rows))
    return mask.cuda(), items


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,dtype", [
    (1, 24, 24, 4096, 4096, torch.bfloat16),  # 384 items over 256 CUs: 1.5 rounds
    (1, 8, 8, 4096, 4096, torch.bfloat16),    # 128 items: half the CUs idle on the plain grid
    (1, 12, 6, 2000, 5000, torch.bfloat16),   # groups of 2, ragged Sq and Sk (a tail tile of 8 keys)
    (2, 6, 6, 1500, 3000, torch.float16),     # fp16, two sequences
    (1, 16, 4, 2048, 4096, torch.bfloat16),   # grouped-query form: 128 items of 4 heads x 64 rows
    (1, 32, 8, 1000, 8192, torch.bfloat16),   # grouped-query form, ragged Sq (16 blocks, the last of 40 rows)
    (2, 24, 3, 700, 6000, torch.float16),     # groups of 8 (two 4-head subgroups per kv head), fp16
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
    cutm, items = _cut_rows(B, Hq, Hkv, Sq, Sk, G)
    assert items, "no item was cut"
    whole = ~cutm
    assert torch.equal(o[whole], ou[whole]) and torch.equal(lse[whole], lseu[whole])
    assert not torch.equal(o[~whole], ou[~whole])  # the merge ran
    assert float((o.float() - ou.float()).abs().max()) <= 8e-3
    assert float(((lse - lseu).abs() / lseu.abs().clamp(min=1)).max()) <= 1e-5
    # rows of a cut item (its first and last rows) and of an uncut one, against the oracle
    b, heads, rs = items[0]
    h = heads[-1]
    rows = np.unique(np.clip([rs.start, (rs.start + rs.stop) // 2, rs.stop - 1, 0, Sq - 1], 0, Sq - 1))
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
    q16 = torch.randn(2, 32, 4096, 128, device=dev, dtype=torch.bfloat16)
    kv16 = torch.randn(2, 32, 4096, 128, device=dev, dtype=torch.bfloat16)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _ws_bytes(q16, kv16, kv16) == 0                    # 1024 items: four whole rounds
    q64 = torch.randn(1, 24, 4608, 64, device=dev, dtype=torch.bfloat16)
    assert _ws_bytes(q64, q64, q64) == 0                          # head dim 64
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _ws_bytes(q, kv, kv) == 0  # C5a: 432 items of 72 tiles, the records cost what the last round saves


def test_streamk_strided_layout_and_no_lse():
    # [B, S, H, D] storage (row pitch H * D) and the one-output operator (no LSE pointer: the records still
    # carry the row sums, the merge writes O alone); the result equals the plain grid on uncut rows
    import dtorch_amd.nn.functional as F
    G = torch.cuda.get_device_properties(0).multi_processor_count & ~7
    g = torch.Generator(device="cuda").manual_seed(77)
    B, Hq, Hkv, Sq, Sk = 1, 12, 6, 2000, 5000
    q = torch.randn(B, Sq, Hq, 128, generator=g, device="cuda").to(torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, Sk, Hkv, 128, generator=g, device="cuda").to(torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, Sk, Hkv, 128, generator=g, device="cuda").to(torch.bfloat16).transpose(1, 2)
    assert _ws_bytes(q, k, v) > 0, "no stream-K plan"
    o = F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
    o_lse, _ = F.scaled_dot_product_attention_with_lse(q, k, v, enable_gqa=True)
    ou, _ = _prefill(q, k, v, False)
    torch.cuda.synchronize()
    assert torch.equal(o, o_lse)
    cutm, items = _cut_rows(B, Hq, Hkv, Sq, Sk, G)
    assert items
    assert torch.equal(o[~cutm], ou[~cutm])
    assert float((o.float() - ou.float()).abs().max()) <= 8e-3
