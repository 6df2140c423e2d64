"""CPU oracle for the grouped 4-bit expert GEMM -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg import this package, and only as the checker or the timed CPU baseline.
The product path (``nf4_grouped`` / ``mxfp4_grouped``) never imports it.

Contents:
  * ``spec``  -- numpy executable spec of the reference's locked summation
    order (reference kernel/cpu_grouped.py:53-144) plus fp64 references.
  * ``native``-- ctypes bindings to ``liboracle.so`` (this directory's C
    restatement, ``gnf4_oracle.c``) and, when it was built, to ``_ref/``: the
    reference's own ``gnf4_native/cpu_kernels.c`` compiled from its source.

Parity status of each oracle function (what pins it):
  * codebooks      -- literal values checked against the reference sources'
                      literals and transformers' FP4_VALUES.
  * decode rows    -- exhaustive 256-byte x code tables, closed form, MXFP4
                      byte 0x21 known answer, e8m0 0x00 / 0xFF edges.
  * locked GEMV    -- bit-exact against the compiled reference (_ref) and the
                      committed golden vectors it produced; fp64 agreement.
  * locked dgrad   -- same as the GEMV; independent fp64 transpose check.
  * packers        -- closed-form properties (argmin, first index on ties,
                      round trip); brute force on small inputs.
"""
