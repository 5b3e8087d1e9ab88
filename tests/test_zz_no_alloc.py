"""The allocation-free decode entry point against the allocating one, through the C ABI.

dtattn_decode_splitkv_noalloc runs the same kernels as dtattn_decode_splitkv with the split partials
in the library's per-device scratch array instead of a caller workspace, so its outputs must be
bit-identical.  Two calls in a row, the second on a smaller problem (the scratch keeps the first call's
contents), then a call whose partials exceed the scratch is rejected before any launch.  The file name
makes pytest collect it last.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16, FP16, FP32 = 0, 1, 3
SCRATCH_BYTES = 32 << 20


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("lengths", ctypes.c_void_p), ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("S_max", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 2), ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3),
        ("o_stride", ctypes.c_int64 * 2), ("lse_stride", ctypes.c_int64 * 1),
        ("dtype", ctypes.c_int32), ("scale", ctypes.c_float), ("chunk", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


def _lib():
    from dtorch_amd import _lib as L
    lib = L.cabi()
    for name in ("dtattn_decode_splitkv", "dtattn_decode_splitkv_noalloc"):
        getattr(lib, name).argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
        getattr(lib, name).restype = ctypes.c_int
    lib.dtattn_decode_workspace_size.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int32]
    lib.dtattn_decode_workspace_size.restype = ctypes.c_size_t
    lib.dtattn_last_error.restype = ctypes.c_char_p
    return lib


def _case(B, Hq, Hkv, S_max, D, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g, device="cuda").to(dtype)
    k = torch.randn(B, Hkv, S_max, D, generator=g, device="cuda").to(dtype)
    v = torch.randn(B, Hkv, S_max, D, generator=g, device="cuda").to(dtype)
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, S_max, size=B, endpoint=True).astype(np.int32)
    lengths[0] = 0  # an empty sequence
    return q, k, v, torch.from_numpy(lengths).cuda()


def _args(q, k, v, lengths, o, lse, code, chunk=0, ws=None):
    a = DecodeArgs()
    a.q, a.k_cache, a.v_cache = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.lengths, a.o, a.lse = lengths.data_ptr(), o.data_ptr(), lse.data_ptr()
    a.B, a.Hq, a.Hkv, a.S_max, a.D = q.shape[0], q.shape[1], k.shape[1], k.shape[2], q.shape[3]
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.k_stride[:] = [k.stride(0), k.stride(1), k.stride(2)]
    a.v_stride[:] = [v.stride(0), v.stride(1), v.stride(2)]
    a.o_stride[:] = [o.stride(0), o.stride(1)]
    a.lse_stride[:] = [lse.stride(0)]
    a.dtype, a.scale, a.chunk = code, float("nan"), chunk  # NaN: 1/sqrt(D)
    a.workspace = ws.data_ptr() if ws is not None else None
    a.workspace_bytes = ws.numel() if ws is not None else 0
    return a


def _both(lib, B, Hq, Hkv, S_max, D, dtype, code, chunk, seed):
    q, k, v, lengths = _case(B, Hq, Hkv, S_max, D, dtype, seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o_ref, o_na = torch.empty_like(q), torch.empty_like(q)
    l_ref = torch.empty(B, Hq, device="cuda")
    l_na = torch.empty(B, Hq, device="cuda")
    ws_bytes = lib.dtattn_decode_workspace_size(B, Hq, S_max, D, chunk)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    a = _args(q, k, v, lengths, o_ref, l_ref, code, chunk, ws)
    assert lib.dtattn_decode_splitkv(ctypes.byref(a), stream) == 0, lib.dtattn_last_error()
    n = _args(q, k, v, lengths, o_na, l_na, code, chunk, None)
    assert lib.dtattn_decode_splitkv_noalloc(ctypes.byref(n), stream) == 0, lib.dtattn_last_error()
    torch.cuda.synchronize()
    return o_ref, l_ref, o_na, l_na


def test_noalloc_decode_matches_allocating_entry_point():
    lib = _lib()
    print("noalloc decode: call 1, B=64 Hq=32 Hkv=8 S_max=4096 D=128 bf16", flush=True)
    o_ref, l_ref, o_na, l_na = _both(lib, 64, 32, 8, 4096, 128, torch.bfloat16, BF16, 0, 1)
    assert torch.equal(o_ref, o_na) and torch.equal(l_ref, l_na)
    assert torch.isfinite(o_na[1:]).all()
    print("noalloc decode: call 2, B=3 Hq=8 Hkv=2 S_max=1000 D=64 fp16, chunk 128", flush=True)
    o_ref, l_ref, o_na, l_na = _both(lib, 3, 8, 2, 1000, 64, torch.float16, FP16, 128, 2)
    assert torch.equal(o_ref, o_na) and torch.equal(l_ref, l_na)
    print("noalloc decode: call 3, B=5 Hq=4 Hkv=4 S_max=700 D=128 fp32", flush=True)
    o_ref, l_ref, o_na, l_na = _both(lib, 5, 4, 4, 700, 128, torch.float32, FP32, 0, 3)
    assert torch.equal(o_ref, o_na) and torch.equal(l_ref, l_na)


def test_noalloc_decode_rejects_calls_beyond_the_scratch():
    lib = _lib()
    B, Hq, Hkv, S_max, D = 64, 32, 8, 65536, 128
    assert lib.dtattn_decode_workspace_size(B, Hq, S_max, D, 384) > SCRATCH_BYTES
    q = torch.zeros(B, Hq, 1, D, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(1, 1, 16, D, dtype=torch.bfloat16, device="cuda")  # only its address is passed
    lengths = torch.zeros(B, dtype=torch.int32, device="cuda")
    o, lse = torch.empty_like(q), torch.empty(B, Hq, device="cuda")
    a = _args(q, k, k, lengths, o, lse, BF16, 384, None)
    a.Hkv, a.S_max = Hkv, S_max
    a.k_stride[:] = [Hkv * S_max * D, S_max * D, D]
    a.v_stride[:] = [Hkv * S_max * D, S_max * D, D]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.dtattn_decode_splitkv_noalloc(ctypes.byref(a), stream) == 3  # DTATTN_ERR_WORKSPACE
    assert b"scratch" in lib.dtattn_last_error()


_FIRST_CALL_CAPTURED = r'''
import ctypes, os, sys
sys.path.insert(0, os.environ["DTATTN_REPO"])
import torch
import tests.test_zz_no_alloc as T
lib = T._lib()
q, k, v, lengths = T._case(4, 8, 2, 1000, 128, torch.bfloat16, 7)
o_na, l_na = torch.empty_like(q), torch.empty(4, 8, device="cuda")
a = T._args(q, k, v, lengths, o_na, l_na, T.BF16)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first noalloc call: the scratch lookup runs under capture
    st = lib.dtattn_decode_splitkv_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
assert st == 0, lib.dtattn_last_error()
for _ in range(3):
    o_na.zero_()
    graph.replay()
    torch.cuda.synchronize()
o_ref, l_ref = torch.empty_like(q), torch.empty(4, 8, device="cuda")
ws = torch.empty(lib.dtattn_decode_workspace_size(4, 8, 1000, 128, 0), dtype=torch.uint8, device="cuda")
r = T._args(q, k, v, lengths, o_ref, l_ref, T.BF16, 0, ws)
assert lib.dtattn_decode_splitkv(ctypes.byref(r), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
torch.cuda.synchronize()
assert torch.equal(o_na, o_ref) and torch.equal(l_na, l_ref)
print("first call captured: replays equal the allocating entry point")
'''


def test_noalloc_first_call_of_a_process_under_graph_capture():
    # The per-device scratch address is looked up on a device's first call; here that call is recorded into
    # a HIP graph in a fresh process (so no earlier test has made the lookup), and its replays must equal
    # the allocating entry point.
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, DTATTN_REPO=root)
    print("noalloc decode: first call of a fresh process under graph capture (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED], cwd=root, env=env, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "replays equal the allocating entry point" in r.stdout


def test_noalloc_graph_replay_after_an_eager_call_on_another_shape():
    # One scratch array per device: a captured call replayed after an eager noalloc call of another shape
    # (which left its own partials in the scratch) must still equal the allocating entry point, and so must
    # that eager call.  Calls on one stream are ordered, so they share the scratch safely.
    lib = _lib()
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    qa, ka, va, la = _case(16, 32, 8, 3000, 128, torch.bfloat16, 21)
    qb, kb, vb, lb = _case(5, 8, 8, 777, 64, torch.float16, 22)
    oa, sa = torch.empty_like(qa), torch.empty(16, 32, device="cuda")
    ob, sb = torch.empty_like(qb), torch.empty(5, 8, device="cuda")
    a = _args(qa, ka, va, la, oa, sa, BF16)
    b = _args(qb, kb, vb, lb, ob, sb, FP16)
    assert lib.dtattn_decode_splitkv_noalloc(ctypes.byref(a), stream()) == 0  # eager warm-up of shape A
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert lib.dtattn_decode_splitkv_noalloc(ctypes.byref(a), stream()) == 0
    torch.cuda.synchronize()
    ref_a = _both(lib, 16, 32, 8, 3000, 128, torch.bfloat16, BF16, 0, 21)
    ref_b = _both(lib, 5, 8, 8, 777, 64, torch.float16, FP16, 0, 22)
    for _ in range(2):
        oa.zero_()
        ob.zero_()
        assert lib.dtattn_decode_splitkv_noalloc(ctypes.byref(b), stream()) == 0  # eager, shape B
        graph.replay()                                                         # shape A from the graph
        torch.cuda.synchronize()
        assert torch.equal(ob, ref_b[0]) and torch.equal(sb, ref_b[1])
        assert torch.equal(oa, ref_a[0]) and torch.equal(sa, ref_a[1])
