"""CPU oracle for the HiF4 attention path: test infrastructure only.

This package restates, in numpy, the reference's HiF4 codec, its Walsh-Hadamard
transform and its tiled flash-attention simulator so that the HIP kernels can be
checked against it.  It is imported only by ``tests/``, by
``__graft_entry__.smoke()`` (as the checker) and by the ``cpu_baseline`` leg of
``bench.py``.  The product package never imports it, and nothing in it runs on
the GPU.

Modules:
  hif4       -- HiF4 S1P2 fake quantization, levels 123 / 12 / 13, plus the packed
                code/metadata view of the same result.
  hadamard   -- normalized Sylvester-order fast Walsh-Hadamard transform.
  attention  -- tiled online-softmax attention simulator with Q/K/P/V quantization.
  linear     -- the quantized Linear's activation path (input scale, HiSQ rotation,
                clamp, companding, online Hadamard, HiF4 QDQ).
  inputs     -- seeded, version-stable synthetic inputs (PCG64) for tests and bench.
"""
