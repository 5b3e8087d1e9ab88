"""CPU oracle for the attention operator (test infrastructure, never a product path).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only as the checker or as the timed CPU baseline.  The HIP
library under ``dtorch_amd`` never imports it and has no CPU fallback.

Modules
-------
``sdpa``            fp64 NumPy restatement of SDPA (O and per-row LSE), GQA, split-KV decode,
                    LSE merge, the ring-attention step, and the OCP fp8 e4m3fn per-head
                    quantizer.  Every function cites the reference file:line whose behaviour it
                    restates.
``dtorch_cpu_path`` the arithmetic DTorch runs on a CPU mesh: ``SdpaOp::Compute`` calls libtorch's
                    ``scaled_dot_product_attention`` on CPU tensors
                    (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109).
                    It is the CPU baseline that ``bench.py`` times and the library routine the fp64
                    restatement is pinned against.

Parity pins (all in ``tests/test_oracle.py``): libtorch CPU SDPA and its flash-attention-for-CPU
log-sum-exp on seeded inputs, the committed golden fixtures under ``tests/golden/`` (written by
libtorch's CPU SDPA), closed forms (single key, zero query, constant V, causal row 0), invariants
(key permutation, GQA == repeat_kv, decode == prefill at Lq=1, merge == single pass, merge
associativity, fully-masked block is a no-op), torch's ``float8_e4m3fn`` cast for the fp8 encoder
(exhaustive over all finite fp32 bucket boundaries sampled), and the reference's own cost figure
(dtorch/tests/test_operator_cost.cc:171-183, 1,310,720).  No function here is "parity unpinned".
"""
