"""CPU oracle for the cooperative EXL3 MoE expert path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or as the timed CPU baseline. The product path (``eva_amd``) never
imports it and has no CPU fallback.

Modules:

- ``exl3``     - MUL1 codebook, trellis bit windows, tile map, dequantization,
                 128-point Hadamard with the reference's fp32 butterfly order.
- ``coop``     - routing, slot grouping (run table), the coop expert math with
                 the reference's rounding points, the shared expert, the layer.
- ``synth``    - seeded synthetic inputs for the BASELINE configurations.
- ``torch_cpu``- PyTorch-CPU restatement of the layer (the timed CPU baseline).
- ``cnative``  - ctypes loader for the independent scalar C restatement
                 (``exl3_oracle.c``), used to cross-check ``exl3``.
"""
