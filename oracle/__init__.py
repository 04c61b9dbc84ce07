"""CPU oracle for the Transformer forward hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the semantics the gfx950 kernels must
reproduce.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or the timed CPU baseline); the product path under the package directory
never imports it.

Modules and the reference code each function follows:

* :mod:`oracle.forward`  -- the official model (pre-LN blocks, fp32 softmax
  with probability cast, exact GELU, final LayerNorm), seeded inputs and
  initialisation (official/torch_transformer_benchmark.py:29-172, :234-272),
  the query-blocked attention order (solution/operators/attention/sdpa.py:116-170)
  and an exact per-row float64 attention for sampled rows of long sequences.
* :mod:`oracle.norm`     -- residual add + LayerNorm / RMSNorm
  (solution/operators/norm/residual_add.py:28-39 + nn.LayerNorm;
  solution/kernels/norm/triton_mixed_residual.py:41-76 for the mixed stream).
* :mod:`oracle.compare`  -- the official OR-rule comparator
  (official/torch_transformer_benchmark.py:289-356) and the bf16/fp32 gates.
* :mod:`oracle.workload` -- FLOP and byte models
  (benchmarking/shape14_measure.py:36-46) and the BASELINE configurations.

Pinning (tests/test_oracle.py): every function is checked against at least
one of the reference's own known answers, a float64 library routine, a
brute-force loop on tiny inputs, or an invariant that a plausible mistake
(dropped term, wrong sign, transposed operand, wrong mask side) violates.
"""
