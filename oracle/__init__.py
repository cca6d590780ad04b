"""CPU oracle for the fused disentangled attention — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import anything from this package, and only as the
checker (or the timed CPU baseline), never as the thing measured or shipped.
The product package ``deberta_amd`` never imports it.

Contents:
  eager.py  line-faithful torch-CPU restatement of the reference's
            DisentangledSelfAttention and its helpers (pszemraj/deberta,
            src/deberta/modeling/deberta_v2_native.py:28-112, 168-652,
            1036-1068; mask_utils.py:8-32; training/compile.py:310-349).
  brute.py  independent fp64 numpy triple loops of the same math (forward
            and the analytic backward), for tiny shapes.

How each function is pinned (no known-answer vectors exist in the
reference's tests, so the pins are closed forms, invariants and the
brute-force cross-check): see tests/test_oracle_*.py.
"""
