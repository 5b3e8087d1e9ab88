#!/usr/bin/env python3
"""Benchmark of the MI355X attention operator (one GPU).

Step = one causal GQA prefill forward with LSE on the Llama-3-8B attention shape (B=4, Hq=32, Hkv=8,
S=2048, D=128, bf16), inputs resident in HBM.  ``value`` is algorithmic TFLOP/s (visible pairs only:
4*B*Hq*D*S(S+1)/2) over the timed steps.  Also reported, each on its own synthetic inputs: split-KV
decode HBM GB/s (B=64, Hq=32, Hkv=8, D=128, lengths U[512, 8192]) with a contiguous and a paged cache,
one decode step (KV-cache append of one token + decode), eager and as a HIP graph replay, the ring step (4 blocks + LSE merge), MMDiT
joint attention in bf16 and fp8, the VAE attention (one head of 512, in bf16 and in fp32), the small causal MHA case in fp32
and bf16, and fp32 prefill on the headline shape.  The CPU baseline is
libtorch's CPU SDPA (the call SdpaOp::Compute makes on a CPU mesh) on the same prefill, in fp32 on the
bf16-rounded inputs (and in bf16 beside it), timed on this host over about ten seconds of repetitions,
and compared with the GPU output.

Order: CPU baseline, secondary workloads, then the headline (W warmup steps, extended to at least
0.25 s of launches, then K timed steps).  The GPU's clocks need some 30 ms of sustained load to settle
after idling (measured: back-to-back prefill launches rise from ~610 to ~925 TFLOP/s over the first
30 ms), so the headline warm-up is time-based and every secondary measurement first runs its workload
for 0.15 s untimed.  The CPU baseline also times the decode workload (per-sequence libtorch CPU SDPA)
right after the GPU decode measurement, on the same cache values.

Prints ONE JSON line on stdout; human-readable detail goes to stderr.
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15   # MI355X dense bf16 MFMA, FLOP/s (published)
PEAK_FP8 = 5.0e15    # MI355X dense fp8 MFMA
PEAK_HBM = 8.0e12    # MI355X HBM3E, B/s
PEAK_FP32 = 157.3e12  # MI355X dense fp32 MFMA
HEADLINE_SETTLE_S = 0.25  # minimum untimed back-to-back headline launches before the timed steps

# HBM bytes per launch of the headline kernel, from the two calibrated rocprofv3 --pmc runs
# (FETCH_SIZE, WRITE_SIZE) summarised in this file.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "prefill_rows64_gqa_causal_b4_s2048_traffic.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def causal_flops(B, Hq, S, D):
    return 4 * B * Hq * D * S * (S + 1) // 2


def profiled_traffic():
    """traffic_bytes_per_launch from the committed profile summary, or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


class Timer:
    """HIP events on the stream the kernels launch on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, reps, settle=0.15, flush=None, batch=1):
        """Median and mean seconds per call over `reps` timed groups of `batch` back-to-back calls (the host
        runs ahead of the GPU inside a group, so a call's Python and launch overhead is not GPU idle time)."""
        t = self.torch
        t0 = time.perf_counter()
        n = 0
        while n < 2 or time.perf_counter() - t0 < settle:
            fn()
            n += 1
            if n % 8 == 0:
                t.cuda.synchronize()
        t.cuda.synchronize()
        times = []
        for _ in range(reps):
            if flush is not None:
                flush()
            s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(batch):
                fn()
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e) * 1e-3 / batch)
        return float(np.median(times)), float(np.mean(times))


def _timed_reps(fn, min_seconds, min_reps=3):
    fn()  # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < min_reps or time.perf_counter() - t0 < min_seconds:
        fn()
        reps += 1
    return reps, time.perf_counter() - t0


def cpu_baseline(torch, qn, kn, vn, min_seconds):
    """libtorch CPU SDPA (all threads) on the full headline workload: in fp32 on the bf16-rounded inputs
    (the reported value), and in bf16 (the same call on the bf16 tensors themselves)."""
    from oracle import dtorch_cpu_path as cpu

    threads = torch.get_num_threads()
    qb, kb, vb = (torch.from_numpy(x).to(torch.bfloat16) for x in (qn, kn, vn))
    q, k, v = (x.float() for x in (qb, kb, vb))
    B, Hq, S, D = q.shape
    flops = causal_flops(B, Hq, S, D)
    out = cpu.sdpa(q, k, v, is_causal=True, enable_gqa=True)  # the reference output for the GPU check
    reps, dt = _timed_reps(lambda: cpu.sdpa(q, k, v, is_causal=True, enable_gqa=True), min_seconds)
    rate = flops * reps / dt
    reps_b, dt_b = _timed_reps(lambda: cpu.sdpa(qb, kb, vb, is_causal=True, enable_gqa=True), min_seconds / 2)
    rate_b = flops * reps_b / dt_b
    info = {
        "value": round(rate / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
        "sample": f"libtorch CPU SDPA (SdpaOp::Compute's call on a CPU mesh) in fp32 on the bf16-rounded inputs, "
                  f"whole workload (B={B}, Hq={Hq}, Hkv={k.shape[1]}, S={S}, D={D}, causal, GQA), {reps} "
                  f"repetitions in {dt:.1f} s on {threads} threads; host: {_physical_cores()} physical cores, "
                  f"{os.cpu_count()} logical CPUs",
        "bf16": {"TFLOP/s": round(rate_b / 1e12, 4), "reps": reps_b, "seconds": round(dt_b, 1),
                 "note": "the same call on the bf16 tensors"},
    }
    log(f"CPU baseline: fp32 {rate / 1e12:.3f} TFLOP/s ({reps} reps, {dt:.1f} s), bf16 {rate_b / 1e12:.3f} "
        f"TFLOP/s ({reps_b} reps, {dt_b:.1f} s), {threads} threads")
    return info, out


def cpu_decode_baseline(torch, qd, kc, vc, lens_np, dbytes, min_seconds):
    """DTorch's CPU path for the decode workload: libtorch CPU SDPA per sequence over its true length
    (is_causal=False, enable_gqa=True), fp32 on the bf16 values of the GPU run's own caches."""
    from oracle import dtorch_cpu_path as cpu

    threads = torch.get_num_threads()
    q = qd.float().cpu()
    ks = [kc[b:b + 1, :, :int(L)].float().cpu() for b, L in enumerate(lens_np)]
    vs = [vc[b:b + 1, :, :int(L)].float().cpu() for b, L in enumerate(lens_np)]

    def run():
        for b in range(len(ks)):
            cpu.sdpa(q[b:b + 1], ks[b], vs[b], enable_gqa=True)

    reps, dt = _timed_reps(run, min_seconds, min_reps=2)
    per = dt / reps
    # the fp32 caches move twice the bf16 bytes; the rate is quoted on the workload's bf16 bytes, like the GPU's
    info = {"GB/s": round(dbytes / per / 1e9, 2), "ms": round(per * 1e3, 2), "reps": reps, "threads": threads,
            "sample": "64 sequences, lengths U[512, 8192], per-sequence libtorch CPU SDPA (Lq = 1, GQA 32/8) "
                      "in fp32 on the bf16 cache values; rate on the bf16 workload bytes"}
    log(f"CPU decode baseline: {per * 1e3:.1f} ms per batch ({dbytes / per / 1e9:.1f} GB/s of bf16 workload "
        f"bytes), {reps} reps on {threads} threads")
    del ks, vs
    return info


def cpu_rate(torch, name, fn, flops, min_seconds, sample, min_reps=3):
    """One CPU-path timing beside its GPU workload: 1 warm-up, then repetitions for at least `min_seconds`
    (and at least `min_reps`); TFLOP/s on the same algorithmic FLOPs as the GPU figure."""
    reps, dt = _timed_reps(fn, min_seconds, min_reps=min_reps)
    rate = flops * reps / dt
    threads = torch.get_num_threads()
    log(f"CPU baseline {name}: {rate / 1e12:.4f} TFLOP/s ({reps} reps, {dt:.1f} s, {threads} threads)")
    return {"TFLOP/s": round(rate / 1e12, 4), "ms": round(dt / reps * 1e3, 2), "reps": reps,
            "seconds": round(dt, 1), "threads": threads, "physical_cores": _physical_cores(),
            "logical_cpus": os.cpu_count(), "sample": sample}


def _prefill_plain(q, k, v):
    """Non-causal bf16/fp16 prefill through the C ABI with no workspace: the plain grid of work items."""
    import ctypes
    import torch
    from dtorch_amd import _lib
    o = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], device=q.device)
    a = _lib.PrefillArgs()
    a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    a.B, a.Hq, a.Sq, a.D = q.shape
    a.Hkv, a.Sk, a.Dv = k.shape[1], k.shape[2], v.shape[3]
    for dst, t in ((a.q_stride, q), (a.k_stride, k), (a.v_stride, v), (a.o_stride, o)):
        dst[0], dst[1], dst[2] = t.stride(0), t.stride(1), t.stride(2)
    a.lse_stride[0], a.lse_stride[1] = lse.stride(0), lse.stride(1)
    a.dtype = a.o_dtype = 0 if q.dtype == torch.bfloat16 else 1
    lib = _lib.cabi()
    lib.dtattn_prefill_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    st = lib.dtattn_prefill_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if st != 0:
        raise RuntimeError(f"dtattn_prefill_fwd failed ({st})")
    return o, lse


def secondary_workloads(torch, F, dev, timer, cpu_info=None, cpu_seconds=0.0):
    extras = {}
    # Cache flush between decode reps: READ 1 GiB (more than the 8 x 4 MB L2 plus the 256 MB MALL), so
    # the K/V bytes of the previous rep are evicted without leaving dirty lines behind.  A write flush
    # (zero_) would leave up to the MALL's size of dirty lines whose write-back then competes with the
    # measured reads (measured: 212.7 us against 205.4 us for the decode workload).
    flush_buf = torch.zeros(1 << 29, dtype=torch.float16, device=dev)

    def flush():
        torch.sum(flush_buf, dtype=torch.float32)

    # split-KV decode
    Bd, Hqd, Hkvd, Smax, Dd = 64, 32, 8, 8192, 128
    g = torch.Generator(device=dev).manual_seed(0)
    qd = torch.randn(Bd, Hqd, 1, Dd, device=dev, generator=g).to(torch.bfloat16)
    kc = torch.randn(Bd, Hkvd, Smax, Dd, device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn(Bd, Hkvd, Smax, Dd, device=dev, generator=g).to(torch.bfloat16)
    lens_np = np.random.default_rng(0).integers(512, 8192, size=Bd, endpoint=True).astype(np.int32)
    lens = torch.from_numpy(lens_np).to(dev)
    tot = int(lens_np.sum())
    dbytes = 4096 * tot + Bd * Hqd * Dd * 2 * 2 + Bd * Hqd * 4
    med, _ = timer.run(lambda: F.decode_attention(qd, kc, vc, lens), reps=20, flush=flush)
    gbs = dbytes / med / 1e9
    extras["decode_c3"] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs * 1e9 / PEAK_HBM, 4),
                           "us": round(med * 1e6, 1), "bytes": dbytes, "sum_len": tot,
                           "note": "L2/MALL flushed by a 1 GiB read before every rep"}
    log(f"decode B=64 Hq=32 Hkv=8 lengths U[512,8192]: {med * 1e6:.1f} us, {gbs:.0f} GB/s "
        f"({100 * gbs * 1e9 / PEAK_HBM:.1f}% of HBM)")
    if cpu_info is not None:
        cpu_info["decode_c3"] = cpu_decode_baseline(torch, qd, kc, vc, lens_np, dbytes, cpu_seconds)

    # one decode step: append the new token's K/V (written at position L - 1 of each sequence, so the
    # attended length stays the bench's), then decode; lengths are reset outside the timed region
    base = (lens - 1).to(torch.int32)
    lens_run = base.clone()
    k1 = torch.randn(Bd, 1, Hkvd, Dd, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    v1 = torch.randn(Bd, 1, Hkvd, Dd, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)

    def step():
        F.kv_cache_append(kc, vc, lens_run, k1, v1)
        F.decode_attention(qd, kc, vc, lens_run)

    def reset():
        flush()
        lens_run.copy_(base)

    med_s, _ = timer.run(step, reps=20, flush=reset)
    extras["decode_step_c3"] = {"us": round(med_s * 1e6, 1), "GB/s": round(dbytes / med_s / 1e9, 1),
                                "note": "kv_cache_append of 1 token per sequence + decode_attention"}
    log(f"decode step (append 1 token + decode): {med_s * 1e6:.1f} us")

    # a launch-bound decode step (one sequence, 4096 cached tokens, 32/8 heads): eager calls against one
    # replay of the same step captured in a HIP graph (the kernels allocate nothing and read the lengths
    # from device memory, so the graph replays them as they are)
    kq = torch.randn(1, Hkvd, 4096, Dd, device=dev, generator=g).to(torch.bfloat16)
    vq = torch.randn(1, Hkvd, 4096, Dd, device=dev, generator=g).to(torch.bfloat16)
    q_1 = torch.randn(1, Hqd, 1, Dd, device=dev, generator=g).to(torch.bfloat16)
    kn_1 = torch.randn(1, Hkvd, 1, Dd, device=dev, generator=g).to(torch.bfloat16)
    vn_1 = torch.randn(1, Hkvd, 1, Dd, device=dev, generator=g).to(torch.bfloat16)
    len_1 = torch.full((1,), 4095, dtype=torch.int32, device=dev)

    def step_1():
        F.kv_cache_append(kq, vq, len_1, kn_1, vn_1)
        return F.decode_attention(q_1, kq, vq, len_1)

    def reset_1():
        len_1.fill_(4095)

    med_e, _ = timer.run(step_1, reps=50, flush=reset_1)
    reset_1()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step_1()
    med_g, _ = timer.run(graph.replay, reps=50, flush=reset_1)
    extras["decode_step_b1_4k"] = {"us_eager": round(med_e * 1e6, 1), "us_graph": round(med_g * 1e6, 1),
                                   "note": "one sequence, 4096 cached tokens, 32/8 heads: append + decode, "
                                           "eager calls vs one HIP graph replay"}
    log(f"decode step, 1 sequence x 4096 tokens: eager {med_e * 1e6:.1f} us, graph replay {med_g * 1e6:.1f} us")
    del graph, kq, vq

    # the same caches in 16-token pages [P, Hkv, 16, D], scattered over the pool by a random block table
    ps = 16
    npg = Smax // ps
    perm = torch.from_numpy(np.random.default_rng(1).permutation(Bd * npg).astype(np.int64)).to(dev)

    def paged(c):
        pool = torch.empty((Bd * npg, Hkvd, ps, Dd), dtype=c.dtype, device=dev)
        pool[perm] = c.view(Bd, Hkvd, npg, ps, Dd).permute(0, 2, 1, 3, 4).reshape(Bd * npg, Hkvd, ps, Dd)
        return pool

    kp, vp = paged(kc), paged(vc)
    del kc, vc
    bt = perm.view(Bd, npg).to(torch.int32)
    med_p, _ = timer.run(lambda: F.decode_attention_paged(qd, kp, vp, bt, lens), reps=20, flush=flush)
    gbs_p = dbytes / med_p / 1e9
    extras["decode_c3_paged16"] = {"GB/s": round(gbs_p, 1), "frac_hbm": round(gbs_p * 1e9 / PEAK_HBM, 4),
                                   "us": round(med_p * 1e6, 1), "bytes": dbytes,
                                   "note": "16-token pages in random pool order; L2/MALL flushed by a 1 GiB read before every rep"}
    log(f"paged decode, 16-token pages: {med_p * 1e6:.1f} us, {gbs_p:.0f} GB/s "
        f"({100 * gbs_p * 1e9 / PEAK_HBM:.1f}% of HBM)")
    del kp, vp, qd, bt, perm

    # ring step: 4 blocks (1 causal diagonal + 3 full) + merge
    C = 4096
    q4 = torch.randn(1, 32, C, 128, device=dev, generator=g).to(torch.bfloat16)
    k4 = [torch.randn(1, 8, C, 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(4)]
    v4 = [torch.randn(1, 8, C, 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(4)]
    blocks = []

    def ring_blocks():
        blocks.clear()
        for c in range(4):
            blocks.append(F.scaled_dot_product_attention_with_lse(
                q4, k4[c], v4[c], is_causal=(c == 3), enable_gqa=True, q_offset=3 * C, k_offset=c * C))

    rflops = 3 * (4 * 32 * 128 * C * C) + causal_flops(1, 32, C, 128)
    med, _ = timer.run(ring_blocks, reps=5)
    extras["ring_c4_blocks"] = {"TFLOP/s": round(rflops / med / 1e12, 1),
                                "frac_bf16": round(rflops / med / PEAK_BF16, 4), "ms": round(med * 1e3, 3)}
    mbytes = 5 * (32 * C * 128 * 2 + 32 * C * 4)
    med_m, _ = timer.run(lambda: F.lse_merge([b[0] for b in blocks], [b[1] for b in blocks]), reps=20,
                         flush=flush)
    extras["ring_c4_merge"] = {"GB/s": round(mbytes / med_m / 1e9, 1),
                               "frac_hbm": round(mbytes / med_m / PEAK_HBM, 4), "us": round(med_m * 1e6, 1)}
    log(f"ring step 4x4096: blocks {med * 1e3:.3f} ms ({rflops / med / 1e12:.0f} TFLOP/s), merge "
        f"{med_m * 1e6:.1f} us ({mbytes / med_m / 1e9:.0f} GB/s)")
    if cpu_info is not None:
        from oracle import dtorch_cpu_path as cpu
        cq = q4.float().cpu()
        ck = [x.float().cpu() for x in k4]
        cv = [x.float().cpu() for x in v4]
        cpu_info["ring_c4"] = cpu_rate(
            torch, "C4 ring step", lambda: cpu.ring_step(cq, ck, cv, 3), rflops, cpu_seconds / 2,
            "libtorch CPU flash attention per block in fp32 on the bf16 values (3 full blocks + the causal "
            "diagonal, GQA by repeat_kv) and the NumPy LSE merge; whole workload", min_reps=1)
        del cq, ck, cv
    del q4, k4, v4, blocks

    # MMDiT joint attention, bf16 and fp8
    q5, k5, v5 = (torch.randn(1, 24, 4608, 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    f5 = 4 * 24 * 128 * 4608 * 4608
    med, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(q5, k5, v5), reps=10, batch=4)
    extras["mmdit_c5a_bf16"] = {"TFLOP/s": round(f5 / med / 1e12, 1), "frac_bf16": round(f5 / med / PEAK_BF16, 4),
                                "us": round(med * 1e6, 1)}
    # a non-causal call with fewer 256-row work items than CUs (8 heads of 4096): the operator's workspace
    # runs it as stream-K shares; the same call with the plain grid for comparison (the C ABI without one)
    qs, ks, vs = (torch.randn(1, 8, 4096, 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    fs = 4 * 8 * 128 * 4096 * 4096
    med_s, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(qs, ks, vs), reps=10, batch=4)
    med_p, _ = timer.run(lambda: _prefill_plain(qs, ks, vs), reps=10, batch=4)
    extras["prefill_streamk_1x8x4096"] = {"TFLOP/s": round(fs / med_s / 1e12, 1), "us": round(med_s * 1e6, 1),
                                          "plain_grid_TFLOP/s": round(fs / med_p / 1e12, 1),
                                          "note": "128 items of 256 rows on 256 CUs: stream-K shares vs the plain grid"}
    log(f"non-causal 1x8x4096: stream-K {fs / med_s / 1e12:.0f} TFLOP/s, plain grid {fs / med_p / 1e12:.0f} TFLOP/s")
    # fp8: the native_fp8 op end to end (per-head quantization of q, k, v plus the attention, three
    # launches and the tail merge), and the attention alone on codes quantized beforehand (the codes entry
    # point: the attention kernel and the tail merge)
    from dtorch_amd import _lib
    opt = F.SdpaOption(sage_attn_type="native_fp8")
    med8, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(q5, k5, v5, sdpa_option=opt), reps=10,
                        batch=4)
    (q8, qd), (k8, kd), (v8, vd) = (F.quantize_fp8_per_head(x) for x in (q5, k5, v5))
    kern8, _ = timer.run(lambda: _lib.prefill_fp8_codes(q8, k8, v8, qd, kd, vd, torch.bfloat16), reps=10, batch=4)
    extras["mmdit_c5b_fp8"] = {"TFLOP/s_end_to_end": round(f5 / med8 / 1e12, 1),
                               "TFLOP/s_attention_kernel": round(f5 / kern8 / 1e12, 1),
                               "frac_fp8_kernel": round(f5 / kern8 / PEAK_FP8, 4),
                               "kernel_us": round(kern8 * 1e6, 1), "us": round(med8 * 1e6, 1),
                               "note": "end to end: native_fp8 op from bf16 inputs; kernel: attention on codes"}
    log(f"MMDiT 1x24x4608: bf16 {f5 / med / 1e12:.0f} TFLOP/s; fp8 end-to-end {f5 / med8 / 1e12:.0f} TFLOP/s "
        f"({med8 * 1e6:.0f} us), attention kernel on codes {f5 / kern8 / 1e12:.0f} TFLOP/s ({kern8 * 1e6:.0f} us)")
    if cpu_info is not None:
        from oracle import dtorch_cpu_path as cpu
        c5 = [x.float().cpu() for x in (q5, k5, v5)]
        cpu_info["mmdit_c5a"] = cpu_rate(
            torch, "C5a MMDiT", lambda: cpu.sdpa(*c5), f5, cpu_seconds / 4,
            "libtorch CPU SDPA in fp32 on the bf16 values, non-causal, whole workload (B=1, H=24, S=4608, D=128)")
        deq = [(c.view(torch.float8_e4m3fn).float() * d[..., None, None].float()).cpu() for c, d in
               ((q8, qd), (k8, kd), (v8, vd))]
        cpu_info["mmdit_c5b"] = cpu_rate(
            torch, "C5b MMDiT on dequantized fp8", lambda: cpu.sdpa(*deq), f5, cpu_seconds / 4,
            "libtorch CPU SDPA in fp32 on the dequantized e4m3fn codes (per-head descales), whole workload")
        del c5, deq
    del q8, k8, v8
    del q5, k5, v5

    # the VAE mid-block attention of the diffusers ports: 128x128 latent pixels, one head of 512 dims
    qv5, kv5, vv5 = (torch.randn(1, 1, 16384, 512, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    fv = 4 * 512 * 16384 * 16384
    med, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(qv5, kv5, vv5), reps=5)
    extras["vae_attention_d512"] = {"TFLOP/s": round(fv / med / 1e12, 1), "frac_bf16": round(fv / med / PEAK_BF16, 4),
                                    "us": round(med * 1e6, 1)}
    log(f"VAE attention 1x1x16384 D=512: {fv / med / 1e12:.0f} TFLOP/s")
    # the same attention run in fp32 (a port that keeps the VAE in fp32): the wide fp32 kernel
    qv5, kv5, vv5 = (x.float() for x in (qv5, kv5, vv5))
    med, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(qv5, kv5, vv5), reps=3)
    extras["vae_attention_d512_fp32"] = {"TFLOP/s": round(fv / med / 1e12, 1),
                                         "frac_fp32": round(fv / med / PEAK_FP32, 4), "us": round(med * 1e6, 1)}
    log(f"VAE attention 1x1x16384 D=512, fp32: {fv / med / 1e12:.1f} TFLOP/s ({fv / med / PEAK_FP32 * 100:.1f}% of fp32 peak)")
    del qv5, kv5, vv5

    # the CPU-runnable causal MHA case (B=1, H=8, S=512, D=64) in its own dtype, fp32, and in bf16
    q1, k1, v1 = (torch.randn(1, 8, 512, 64, device=dev, generator=g) for _ in range(3))
    q1_32, k1_32, v1_32 = q1, k1, v1
    f1 = causal_flops(1, 8, 512, 64)
    med32, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(q1, k1, v1, is_causal=True), reps=20)
    q1, k1, v1 = (x.to(torch.bfloat16) for x in (q1, k1, v1))
    med, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(q1, k1, v1, is_causal=True), reps=20)
    extras["c1_causal_mha_d64"] = {"TFLOP/s_fp32": round(f1 / med32 / 1e12, 2), "us_fp32": round(med32 * 1e6, 1),
                                   "TFLOP/s_bf16": round(f1 / med / 1e12, 2), "us_bf16": round(med * 1e6, 1)}
    if cpu_info is not None:
        from oracle import dtorch_cpu_path as cpu
        c1 = [x.cpu() for x in (q1_32, k1_32, v1_32)]
        cpu_info["c1_causal_mha_d64"] = cpu_rate(
            torch, "C1 causal MHA fp32", lambda: cpu.sdpa(*c1, is_causal=True), f1, min(2.0, cpu_seconds / 4),
            "libtorch CPU SDPA in fp32, causal, B=1 H=8 S=512 D=64 (the reference's own CPU case)")
    del q1, k1, v1

    # fp32 prefill on the headline shape (fp32 inputs are computed in fp32 on the fp32 matrix cores)
    qf, kf, vf = (torch.randn(4, h, 2048, 128, device=dev, generator=g) for h in (32, 8, 8))
    f2 = causal_flops(4, 32, 2048, 128)
    med, _ = timer.run(lambda: F.scaled_dot_product_attention_with_lse(qf, kf, vf, is_causal=True, enable_gqa=True),
                       reps=10)
    extras["prefill_c2_shape_fp32"] = {"TFLOP/s": round(f2 / med / 1e12, 1), "frac_fp32": round(f2 / med / PEAK_FP32, 4),
                                       "us": round(med * 1e6, 1)}
    log(f"fp32 prefill 4x32x2048 causal GQA: {f2 / med / 1e12:.1f} TFLOP/s ({f2 / med / PEAK_FP32 * 100:.1f}% of fp32 peak)")
    del qf, kf, vf
    del flush_buf
    return extras


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-extras", action="store_true", help="only the headline prefill")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="length of the CPU baseline sample")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 device copies of 1 GiB (known traffic) to scale rocprof byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}); the attention "
              "operator is not sharded across GPUs here.", file=sys.stderr)
        sys.exit(2)

    import torch
    import dtorch_amd.nn.functional as F

    dev = torch.device("cuda:0")
    pk = F.device_peaks(0)
    log(f"device {pk.arch}: {pk.cu_count} CUs @ {pk.clock_hz / 1e9:.2f} GHz -> bf16 {pk.bf16_flops / 1e15:.2f} "
        f"PFLOP/s, fp8 {pk.fp8_flops / 1e15:.2f} PFLOP/s (computed); published peaks used: bf16 2.5, fp8 5.0 "
        f"PFLOP/s, HBM 8.0 TB/s")
    timer = Timer(torch)
    if args.copy_calibration:
        src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("copy calibration: 3 x copy of 1 GiB (1,048,576 KiB read and written per launch)")

    # headline inputs: Llama-3-8B attention shape
    B, Hq, Hkv, S, D = 4, 32, 8, 2048, 128
    rng = np.random.default_rng(0)
    qn = rng.standard_normal((B, Hq, S, D), dtype=np.float32)
    kn = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    vn = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    flops = causal_flops(B, Hq, S, D)

    cpu_info, cpu_out = (None, None) if args.no_cpu else cpu_baseline(torch, qn, kn, vn, args.cpu_seconds)
    extras = {} if args.no_extras else secondary_workloads(torch, F, dev, timer, cpu_info, args.cpu_seconds / 2)

    # ---------------------------------------------------------------- headline: W warmup, K timed steps
    q, k, v = (torch.from_numpy(x).to(torch.bfloat16).to(dev) for x in (qn, kn, vn))

    def step():
        return F.scaled_dot_product_attention_with_lse(q, k, v, is_causal=True, enable_gqa=True)

    # Warm-up: W steps, extended to at least HEADLINE_SETTLE_S of back-to-back launches, whatever W is,
    # so that the timed steps never fall inside the clock ramp.
    out = None
    t_w, n_w = time.perf_counter(), 0
    while n_w < args.warmup or time.perf_counter() - t_w < HEADLINE_SETTLE_S:
        out = step()
        n_w += 1
        if n_w % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"headline warm-up: {n_w} steps in {time.perf_counter() - t_w:.3f} s")
    # One event pair on the launch stream brackets the K launches: their GPU time over K is the average
    # launch duration (it includes the dispatch gaps, so it bounds the kernel time from above).  An event
    # pair per step would add ~7 us of event packets to every step (measured: 147 -> 154 us per step).
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e_start.record()
    for _ in range(args.steps):
        out = step()
    e_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    value = flops / (wall / args.steps) / 1e12
    k_avg = e_start.elapsed_time(e_end) * 1e-3 / args.steps
    achieved = flops / k_avg / 1e12
    log(f"prefill causal GQA B=4 Hq=32 Hkv=8 S=2048 D=128 bf16: {ms_per_step:.3f} ms/step wall, kernel avg "
        f"{k_avg * 1e6:.1f} us -> {achieved:.1f} TFLOP/s ({100 * achieved * 1e12 / PEAK_BF16:.1f}% of bf16 peak)")

    result = {
        "metric": "prefill attn TFLOP/s (MFMA util %) + decode attn HBM GB/s, 1xMI355X",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) from numpy default_rng(0), cast to bf16 (secondary workloads: torch.randn "
                "on the device)",
        "config": {"workload": "Llama-3-8B-shape causal GQA prefill attention with LSE", "B": B, "Hq": Hq,
                   "Hkv": Hkv, "S": S, "D": D, "causal": True, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_BF16, 4), "traffic": profiled_traffic(),
                     "kernel": "prefill_rows64_gqa_kernel<bf16,causal>",
                     "work_per_launch": f"{flops} FLOP (4*B*Hq*D*S(S+1)/2)",
                     "avg_launch_us": round(k_avg * 1e6, 2)},
    }
    if cpu_info is not None:
        cpu_info["gpu_vs_cpu_max_abs_err"] = round(float((out[0].float().cpu() - cpu_out.float()).abs().max()), 5)
        result["cpu_baseline"] = cpu_info
    result["extras"] = extras
    print(json.dumps(result), flush=True)


def _physical_cores():
    try:
        ids = set()
        with open("/proc/cpuinfo") as f:
            phys = core = None
            for line in f:
                if line.startswith("physical id"):
                    phys = line.split(":")[1].strip()
                elif line.startswith("core id"):
                    core = line.split(":")[1].strip()
                    ids.add((phys, core))
        return len(ids) or None
    except OSError:
        return None


if __name__ == "__main__":
    main()
