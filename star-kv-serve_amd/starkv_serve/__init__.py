"""STAR-KV paged decode attention for MI355X (gfx950).

``starkv_serve.kernels.paged_decode`` and ``starkv_serve.kernels.paged_quant`` keep
the module paths, names and signatures of the reference plugin's kernels; their
GPU work runs in the hand-written HIP library ``libstarkv_hip.so`` (C ABI:
``include/starkv_hip.h``).
"""
