"""CPU oracle for the split-KV paged decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the timed CPU restatement). The product package
``mxflashattn_amd`` never imports it.

Modules:
  reference_port  fp32 torch-CPU restatement of mxflashattn/reference.py
                  (attention_single/batched/varlen/kvcache).
  c_oracle        ctypes wrapper of decode_ref.c: fp64 paged decode and
                  bitwise block-table / slot-mapping appends.
  split_model     fp64 NumPy model of the split partials and their LSE merge.
  build_ref       compiles the reference's own ATen implementation of the path
                  (csrc/mxmac) into oracle/_ref/ with one g++ line.
  ref_aten        loads that build (None where it was not built); it pins
                  reference_port (tests/test_oracle_ref.py) and is the
                  "reference" CPU baseline of bench.py.

How each function is pinned (golden vectors, closed forms, invariants) is
listed in tests/test_oracle.py; every function here has at least one check
that a dropped term, swapped index or transposed operand would fail. The
golden vectors of the reference's own build (tests/golden/, written by
tests/golden/make_golden.py from oracle/_ref) pin reference_port and the C
oracle where the reference is absent (tests/test_golden.py).
"""
