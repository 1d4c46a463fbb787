"""CPU oracle for the quantized decode pack: TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's fp64 contracts and its CPU
control paths for the three pack operators:

- ``quant_contract``  MLX-affine quantizer, dequantizer, ``r_contract``, the
                      six-member fp32 ensemble and the six artefact faults
                      (vladmt06/kernelverify ``kernelverify/schemas/quant_contract.py``);
- ``floor``           the shipped verdict formula ``max(base_tol, K * floor)``
                      (``kernelverify/tolerance/floor.py:76-89``);
- ``native_kernels``  the CPU control paths with their fault seams
                      (``kernelverify/reference/native_kernels.py:41-221``);
- ``native_ops``      fp64 references and ensemble tolerances per operator
                      (``kernelverify/schemas/native_ops.py``);
- ``verify``          the single gate between a surface and a pass/fail claim
                      (``kernelverify/pack/verify.py:61-149``);
- ``extensions``      the BASELINE-only generalisations the reference does not
                      carry: per-sequence and GQA KV decode, top-k routing from
                      logits at any k, and the SwiGLU expert composition.

Who may import it: ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and there only as the checker or as the
timed CPU baseline. Nothing in ``kernelverify_amd`` imports this package; the
product path runs on the HIP library or fails.

Parity status of every function is listed in each module's header. A function
marked "parity unpinned" has no check beyond its own definition.
"""
