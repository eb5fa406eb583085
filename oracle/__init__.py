"""CPU oracle for the MXFP4 weight-only Qwen3 MLP path.

TEST INFRASTRUCTURE ONLY. This package is a CPU restatement of the reference
algorithm (Jason-Young123/tinyInfer) used to check the HIP product path. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or, for the baseline, as
the timed CPU restatement of the reference's torch path). The product package
``tinyinfer_amd`` never imports it and has no CPU fallback.

Modules
-------
``oracle.mxfp4``  codec: e2m1/e8m0 decode, ``dequantize_chunk``,
                  ``quantize_chunk`` (reference ``tinyinfer/quantization/
                  quantize_mxfp4.py:21-85``).
``oracle.mlp``    the reference's dequant-then-matmul torch CPU path
                  (``tinyinfer/layers/linear.py:19-21``,
                  ``tinyinfer/layers/activation.py:7-11``,
                  ``tinyinfer/models/qwen3.py:155-158``), an fp64 brute force
                  and a restatement of the reference GPU kernel's rounding
                  points (``tinyinfer/csrc/mlp_fp4.cu:140,424``).

Pinning status (what checks each function, in ``tests/``):

* ``decode_e2m1`` / ``decode_e8m0`` / ``dequantize_chunk``: exhaustive 16x256
  known-answer table derived independently from the OCP MX field definitions
  and torch's ``float8_e8m0fnu`` (test_oracle_codec.py).
* ``quantize_chunk``: brute-force nearest-code search with ties-to-even, exact
  exponent model (correctly rounded fp32 log2, shown equal to torch's CPU log2
  for every binade), idempotence, round-trip error bound, special cases
  (test_oracle_codec.py).
* ``mlp_reference`` / ``mlp_kernel_semantics``: fp64 brute force on tiny
  shapes, power-of-two scale invariance, permutation invariance, zero weights
  (test_oracle_mlp.py).

No function here is "parity unpinned".
"""
