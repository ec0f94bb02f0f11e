"""CPU oracle for the quantized linear-layer hot path - TEST INFRASTRUCTURE.

This package restates the reference's algorithms (jtiro232/Alpacca, files
cited per function) on the CPU so that the HIP library can be checked
against them.  It is a checker, never a product path:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
  of ``bench.py`` may import, call, link or run anything under ``oracle/``;
* ``alpacca_amd`` (the product) never imports it and has no CPU fallback.

Modules
  quants_ref   GGUF block decoders: a vectorized NumPy restatement of
               alpacca/quants.py:338-528, a scalar restatement of the pure
               decoders (quants.py:50-224), an exact rational decoder, and
               the Q8_0/Q4_0 encoders (quants.py:533-559).
  qmatrix_ref  QuantMatrix.matvec / matmul_t / rows_at in the reference's own
               float32 order (alpacca/qmatrix.py:148-246), a float64 matvec,
               and the normalized error metric of the parity tests.
  model_ref    the decode and batched prefill steps of alpacca/model.py on
               these matrices, and the greedy loops of smoke.py / bench.py.
  sample_ref   greedy selection with the repetition penalty and its window
               (alpacca/sample.py:31-45).
  cbaseline    ctypes front of matvec_loop.c, a C/OpenMP transliteration of
               the Numba loop alpacca/kernels.py:49-69 (CPU baseline only).

How each function is pinned (checked against something other than itself)
is listed in tests/test_oracle_*.py; every decoder is pinned bit-for-bit.
"""
