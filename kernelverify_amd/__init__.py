"""kernelverify_amd: the MI355X-native quantized decode kernel pack.

The three operators of vladmt06/kernelverify's pack (``kernelverify/pack/``),
hand-written in HIP for gfx950 behind the C ABI of ``include/kvpack.h``
(``libkvpack.so``), with the reference's pack / runner / gate interfaces on
the host side:

- ``kernelverify_amd.pack``     pack modules: wide_qmv, kv_attention,
                                moe_dispatch, evidence, gate drivers
- ``kernelverify_amd.runners``  HipRunner beside the reference's MetalRunner
- ``kernelverify_amd.lib``      ctypes binding of libkvpack.so
- ``kernelverify_amd.hip``      ctypes binding of the HIP runtime
- ``kernelverify_amd.build``    hipcc build of libkvpack.so
- ``kernelverify_amd.report``   verification certificates (schema v2)
- ``kernelverify_amd.serving``  the PyTorch-ROCm serving door (routed
                                linear with the flattened-M rule, KV door)
- ``kernelverify_amd.checkpoint`` MLX-affine safetensors checkpoints read
                                without repacking

There is no CPU implementation of any operator here: without the built
library and a gfx950 device every compute call raises.
"""

__version__ = "0.1.0"
