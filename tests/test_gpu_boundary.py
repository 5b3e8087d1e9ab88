"""GPU checks of the host boundary: rank > 4 views, zero-head errors and concurrent callers.

* rank-5/6/7 q/k/v (views with size-1 axes before H, head slices of a fused tensor) against the oracle,
  with an attention mask and the LSE, through every operator that folds batch axes (prefill, merge,
  fp8 quantize);
* head counts of zero raise ValueError instead of dividing by zero;
* four threads, each on its own default-priority stream like the reference's per-device KernelStream
  threads (dtorch/core/kernel_stream/kernel_stream.cc:72-93, cuda_kernel_stream.cc:25-43), run the
  operators concurrently and get bit-identical results to a serial run; a validation error in one
  thread leaves the other threads' dtattn_last_error() alone.
"""
import ctypes
import threading

import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, host, lse_rel, max_abs, randn, rounded, to_dev

pytestmark = pytest.mark.gpu


def _F():
    import dtorch_amd.nn.functional as F
    return F


def _ref(q, k, v, **kw):
    """Oracle on rank-n inputs: fold the leading axes, run, unfold."""
    lead = q.shape[:-3]
    f = lambda x: x.reshape((-1,) + x.shape[-3:])
    o, l = orc.sdpa_fwd(f(q), f(k), f(v), **kw)
    return o.reshape(lead + o.shape[1:]), l.reshape(lead + l.shape[1:])


def test_rank5_transposed_view_with_size1_axis():
    # x.transpose(1, 2).unsqueeze(1): [2, 1, H, S, D] whose batch stride is not H * stride(H)
    rng = np.random.default_rng(31)
    B, S, H, D = 2, 96, 4, 128
    q, k, v = (randn(rng, (B, S, H, D)) for _ in range(3))
    tq, tk, tv = (to_dev(x).transpose(1, 2).unsqueeze(1) for x in (q, k, v))
    assert tq.shape == (B, 1, H, S, D) and tq.stride(0) != H * tq.stride(2)
    mask = torch.from_numpy(rng.random((S, S)) > 0.2).cuda()
    mask[:, 0] = True
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=True, attn_mask=mask)
    torch.cuda.synchronize()
    rq, rk, rv = (rounded(x).transpose(0, 2, 1, 3)[:, None] for x in (q, k, v))
    ro, rl = _ref(rq, rk, rv, is_causal=True, attn_mask=mask.cpu().numpy())
    assert o.shape == (B, 1, H, S, D) and lse.shape == (B, 1, H, S)
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL
    # the plain SdpaOp entry (one output) on the same view
    o1 = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True, attn_mask=mask)
    assert torch.equal(o1, o)


@pytest.mark.parametrize("shape_fn", [
    lambda x: x.unsqueeze(0),                 # [1, B, H, S, D]
    lambda x: x[:, None, None],               # [B, 1, 1, H, S, D]
    lambda x: x.reshape((2, 2) + x.shape[1:]).unsqueeze(1),  # [2, 1, 2, H, S, D]
])
def test_rank_gt4_layouts_with_gqa(shape_fn):
    rng = np.random.default_rng(32)
    B, Hq, Hkv, S, D = 4, 8, 2, 80, 64
    q, k, v = randn(rng, (B, Hq, S, D)), randn(rng, (B, Hkv, S, D)), randn(rng, (B, Hkv, S, D))
    tq, tk, tv = (shape_fn(to_dev(x)) for x in (q, k, v))
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv, is_causal=True, enable_gqa=True)
    torch.cuda.synchronize()
    ro, rl = orc.sdpa_fwd(rounded(q), rounded(k), rounded(v), is_causal=True, enable_gqa=True)
    assert o.shape == tq.shape
    assert max_abs(host(o).reshape(ro.shape), ro) <= O_TOL_BF16
    assert lse_rel(host(lse).reshape(rl.shape), rl) <= LSE_TOL


def test_head_slice_of_fused_rank5_tensor():
    # q/k/v are head slices of one [A, 1, 3H, S, D] projection output: batch stride 3H*S*D
    rng = np.random.default_rng(33)
    A, H, S, D = 3, 4, 70, 128
    qkv = to_dev(randn(rng, (A, 1, 3 * H, S, D)))
    tq, tk, tv = qkv[:, :, :H], qkv[:, :, H:2 * H], qkv[:, :, 2 * H:]
    F = _F()
    o, lse = F.scaled_dot_product_attention_with_lse(tq, tk, tv)
    torch.cuda.synchronize()
    h = host(qkv)
    ro, rl = _ref(h[:, :, :H], h[:, :, H:2 * H], h[:, :, 2 * H:])
    assert max_abs(host(o), ro) <= O_TOL_BF16
    assert lse_rel(host(lse), rl) <= LSE_TOL
    # the merge and the fp8 quantizer fold the same way: a strided rank-5 block set
    big = torch.zeros((A, 1, 2 * H, S, D), dtype=torch.bfloat16, device="cuda")
    big[:, :, :H] = o
    ov = big[:, :, :H]
    mo, ml = F.lse_merge([ov, o], [lse, lse])
    torch.cuda.synchronize()
    assert max_abs(host(mo), host(o)) <= 1e-2  # merging a block with itself returns it
    assert lse_rel(host(ml), host(lse) + np.log(2.0)) <= 1e-6
    codes, desc = F.quantize_fp8_per_head(tq)
    torch.cuda.synchronize()
    rc, rd = orc.fp8_quantize_per_head(h[:, :, :H].reshape(A, H, S, D).astype(np.float32))
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(desc.cpu().numpy().reshape(rd.shape), rd)


def test_zero_head_inputs_raise():
    F = _F()
    q = torch.randn(1, 4, 16, 64, device="cuda", dtype=torch.bfloat16)
    kv0 = torch.empty(1, 0, 16, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="at least one head"):
        F.scaled_dot_product_attention(q, kv0, kv0, enable_gqa=True)
    with pytest.raises(ValueError, match="at least one head"):
        F.scaled_dot_product_attention_with_lse(q, kv0, kv0, enable_gqa=True)
    q1 = torch.randn(2, 4, 1, 64, device="cuda", dtype=torch.bfloat16)
    cache0 = torch.empty(2, 0, 32, 64, device="cuda", dtype=torch.bfloat16)
    lengths = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="multiple of kv heads"):
        F.decode_attention(q1, cache0, cache0, lengths)
    pool0 = torch.empty(4, 0, 16, 64, device="cuda", dtype=torch.bfloat16)
    bt = torch.zeros(2, 2, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="multiple of kv heads"):
        F.decode_attention_paged(q1, pool0, pool0, bt, lengths)
    # zero query heads with zero kv heads is an empty problem, not an error
    q0 = torch.empty(1, 0, 16, 64, device="cuda", dtype=torch.bfloat16)
    o = F.scaled_dot_product_attention(q0, kv0, kv0)
    assert o.shape == (1, 0, 16, 64)


def _workloads(seed):
    """One input set per operator, on the device."""
    rng = np.random.default_rng(seed)
    pre = [to_dev(randn(rng, s)) for s in ((2, 8, 300, 128), (2, 2, 300, 128), (2, 2, 300, 128))]
    dec_q = to_dev(randn(rng, (8, 8, 1, 128)))
    dec_k = to_dev(randn(rng, (8, 2, 2000, 128)))
    dec_v = to_dev(randn(rng, (8, 2, 2000, 128)))
    dec_l = torch.from_numpy(rng.integers(1, 2000, 8).astype(np.int32)).cuda()
    return pre, (dec_q, dec_k, dec_v, dec_l)


def _run_all(F, pre, dec):
    o = F.scaled_dot_product_attention(*pre, is_causal=True, enable_gqa=True)
    o2, l2 = F.scaled_dot_product_attention_with_lse(*pre, is_causal=False, enable_gqa=True, q_offset=3)
    do, dl = F.decode_attention(*dec)
    mo, ml = F.lse_merge([o, o2], [l2, l2])
    return [o, o2, l2, do, dl, mo, ml]


def test_concurrent_threads_on_own_streams_match_serial():
    F = _F()
    inputs = [_workloads(40 + i) for i in range(4)]
    serial = [[t.clone() for t in _run_all(F, *inputs[i])] for i in range(4)]
    torch.cuda.synchronize()
    results, errors = [None] * 4, []
    start = threading.Barrier(4)

    def worker(i):
        try:
            s = torch.cuda.Stream()  # default priority
            with torch.cuda.stream(s):
                start.wait()
                outs = None
                for _ in range(10):
                    outs = _run_all(F, *inputs[i])
                s.synchronize()
                results[i] = [t.clone() for t in outs]
                s.synchronize()
        except Exception as e:  # surfaced in the main thread
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(4):
        for a, b in zip(results[i], serial[i]):
            assert torch.equal(a, b), i


def test_validation_error_in_one_thread_leaves_others_alone():
    from dtorch_amd import _lib
    lib = _lib.cabi()
    lib.dtattn_last_error.restype = ctypes.c_char_p
    lib.dtattn_prefill_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    F = _F()
    pre, dec = _workloads(50)
    msgs, errors = {}, []
    start = threading.Barrier(3)

    def bad_caller():
        try:
            start.wait()
            for _ in range(200):
                assert lib.dtattn_prefill_fwd(None, None) == 1
                m = lib.dtattn_last_error()
                assert b"args is NULL" in m, m
            msgs["bad"] = lib.dtattn_last_error()
        except Exception as e:
            errors.append(repr(e))

    def host_op_caller():
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                start.wait()
                for _ in range(20):
                    with pytest.raises(ValueError, match="enable_gqa"):
                        F.scaled_dot_product_attention(*pre)  # head counts differ without enable_gqa
                    _run_all(F, pre, dec)
                msgs["op"] = lib.dtattn_last_error()
                s.synchronize()
        except Exception as e:
            errors.append(repr(e))

    def good_caller():
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                start.wait()
                for _ in range(20):
                    _run_all(F, pre, dec)
                msgs["good"] = lib.dtattn_last_error()
                s.synchronize()
        except Exception as e:
            errors.append(repr(e))

    threads = [threading.Thread(target=f) for f in (bad_caller, host_op_caller, good_caller)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    torch.cuda.synchronize()
    assert b"args is NULL" in msgs["bad"]
    assert msgs["good"] == b"", msgs["good"]       # no failing call on this thread
    assert b"args is NULL" not in msgs["op"]       # the host check threw before any C ABI call
