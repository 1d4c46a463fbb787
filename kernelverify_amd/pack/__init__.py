"""The kernel pack on MI355X: host modules for the three operator families.

Mirrors vladmt06/kernelverify ``kernelverify/pack/``: ``wide_qmv``,
``kv_attention``, ``moe_dispatch``, ``evidence`` (gate evidence records) and
``gate`` (verify-then-time drivers). Each family module exposes the
reference's host API (``SUPPORTED_BITS``, ``pack_codes``/``quantize_cache``/
``quantize_experts``, ``launch_config``, ``kernel_spec``) and a ``run_*``
function that calls libkvpack on device buffers.
"""
