"""CPU oracle for the FP8 block-scaled matmul and RMSNorm hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``train-gpt_amd/``) imports,
links or runs anything here.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` use this package, and only as the
checker / the timed CPU restatement, never as the thing measured on the GPU.

Contents (each function cites the reference file:line it restates):

* ``bf16``     -- bf16 <-> f32 bit helpers (round-to-nearest-even).
* ``fp8_ref``  -- OCP e4m3fn encode/decode, ``_quantize_to_fp8``
                  (fp8.py:39-47), the block-scaled forward (fp8.py:50-78),
                  the straight-through and FP8 backward (fp8.py:85-98) and the
                  pre-quantized-weight GEMV.
* ``norm_ref`` -- ``_rms_norm_pure`` (kernels.py:30-33), the fused
                  norm -> quantize composition and the norm VJP
                  (kernels.py:104-118).
* ``cbind``    -- ctypes access to ``tg_oracle.c``, a C restatement of the
                  e4m3fn encoder and the 1x128 quantizer used for exhaustive
                  sweeps and as the timed CPU baseline.

Parity pinning (what checks each function; see tests/test_oracle_*.py):

* e4m3fn encode: all 2**32 f32 bit patterns against torch's CPU
  ``float8_e4m3fn`` cast (an independent implementation), plus known answers.
* quantize: closed-form scale checks, the amax element encodes to +-448,
  zero blocks, NaN/inf propagation, the ``ones`` known answer.
* dequant GEMM: float64 brute force on tiny shapes, the ``ones @ ones == 128``
  known answer (debug_fp8.py:104-109), linearity in the scales.
* rms_norm_pure: constant rows give +-gamma, scale invariance, op-by-op bf16
  rounding checked against torch's bf16 arithmetic.
* norm VJP: float64 finite differences.

The exact bits that XLA-CPU produces for the f32 mean reduction order, the
rsqrt lowering and the f32 -> e4m3fn convert cannot be imported here (JAX is
not installed in this image); the oracle fixes them to IEEE-754 correctly
rounded operations and an order-free (float64) sum.  That choice is stated
in each function's docstring.
"""
