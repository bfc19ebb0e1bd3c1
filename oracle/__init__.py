"""CPU oracle for the fused layer kernels — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package: as the checker of the HIP path, or as
the timed CPU baseline. The product (``nspeech_amd`` and
``libnspeech_rocm.so``) never imports, links or calls anything here.

Two layers:

* ``oracle.restated`` — ctypes bindings to ``nsr_oracle.c``, a plain-C
  restatement of the reference's CPU op sequences (Candle f32 tensor ops,
  op for op, with the reference file:line in each function's comment).
* ``oracle.closed_form`` — numpy float64 closed forms of the same maths,
  used with library routines (torch, numpy) to pin the restatement.

Parity status of each function is recorded in its docstring; functions whose
only check is an invariant or a closed form say so there.
"""
