"""CPU oracle for the SVDQuantLinear hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference
``krea2_svdquant`` quantized-linear path so that the HIP kernels of
``krea2_svdquant_amd`` can be checked against it.  It is never part of the
product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement of the reference
``pytorch_sim`` path).  The product path raises when its HIP library is
missing; it never falls back to anything in here.

Modules
-------
``numerics``  bit-exact bf16 / fp16 rounding helpers (numpy).
``pack``      restatement of ``src/krea2_svdquant/quant/pack.py:6-70``
              (group-wise symmetric INT4 quantize / dequantize / nibble pack)
              plus the per-group A4 activation quantizer the W4A4 path adds.
``sim``       restatement of ``svdquant_linear_sim``
              (``src/krea2_svdquant/quant/svd.py:119-163``) in CPU torch bf16,
              and float64 evaluators of the W4A4 / W4A16 quantized math,
              including the LoRA side branch (``runtime/linear.py:11-45``).
``synth``     seeded synthetic layer states following
              ``quant/svd.py:26-116`` and ``scripts/convert_simulated.py:184-208``.

Pinning (what each function is checked against) is listed in the tests:
``tests/test_oracle_pack.py``, ``tests/test_oracle_sim.py``.  Every function
here has at least one check that does not restate its own formula (reference
known-answer tests, torch's own bf16 arithmetic applied the way the reference
applies it, closed forms and brute force on tiny inputs).
"""
