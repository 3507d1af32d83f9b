"""CPU oracle for the FfnAgent Dense-FFN mailbox step.

TEST INFRASTRUCTURE ONLY.  Nothing in ``crosspool_amd`` may import, call, link
or execute anything under ``oracle/``; only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg use it, and only as the checker (or, for
``cpu_baseline``, as the timed CPU restatement).  The product path fails loudly
when its HIP library is missing instead of falling back here.

Contents
--------
``ffn_oracle``   torch-CPU / numpy restatement of the reference's formulas
                 (gather, scatter, RMSNorm, gated SiLU, Dense partial, metrics,
                 deterministic weights, capacity buckets, workspace layout).
``c/``           an independent plain-C restatement of the same transport and
                 Dense formulas (scalar, fp64 accumulation), built into
                 ``oracle/_build/libxpool_oracle.so`` by ``oracle/build_oracle.py``
                 and used by the tests to cross-check ``ffn_oracle``.
``c_oracle``     ctypes loader for that library.

Pinning status (each function's docstring names its reference file:line and
the checks that pin it; see tests/test_oracle.py):

* gather / scatter / copy_bytes -- pinned: closed form + the reference's own
  cooperative-copy byte cases (cooperative_test.cu:77-111) + C restatement.
* gated_silu, dense_partial_reference -- pinned: pure-Python exact
  (fractions.Fraction) brute force on the 4x16x8 test shape with the
  reference's deterministic weights, the C restatement, and invariants
  (zero weights -> zero, row independence, linearity of the down projection).
* rmsnorm -- parity unpinned by any reference test (the reference has no
  RMSNorm on this path; SGLang's lives in an un-vendored dependency).  It is
  pinned only against the textbook formula: fp64 brute force, the C
  restatement and closed forms (constant rows, eps-dominated rows).
* derive_payload_row_capacities / WorkspaceLayout -- pinned by the
  reference's unit-test known answers (test_execution.py:18-60).
"""
