"""CPU oracle for the fused normalization path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
anything from here, and only as the checker (or, for the CPU baseline, as the thing timed on the
host).  The product path (``fused-layernorm-cuda-operator_amd/``) never imports it: with the HIP
extension missing it raises instead of falling back.

Contents:
  * ``norms``    -- numpy fp64 restatement of every op on the path (LayerNorm / RMSNorm forward,
                    LN+GELU, residual add, fp8 e4m3fn quantization, backward closed forms).
  * ``c_oracle`` -- ctypes wrapper of ``fln_oracle.c``, a plain-C fp64-accumulating restatement of
                    the LayerNorm / RMSNorm forward and backward, for full-size checks and the
                    CPU baseline.  Build with ``make -C oracle``.

The reference's own kernels (CUDA, ``csrc/*.cu``) cannot be compiled in this image (no nvcc, and
hipifying them is excluded), so there is no ``oracle/_ref`` build; every function here is pinned
instead against PyTorch-CPU library routines, closed forms, invariants, finite differences and a
known-answer fp8 table (``tests/test_oracle.py``).
"""
