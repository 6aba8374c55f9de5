"""Host-side helpers for the MI355X (gfx950) StripedHyena2 prefill library.

The product is the C-ABI shared library ``libevo_hip.so`` (declared in
``include/evo/evo.h`` and ``include/evo/hip_ops.h``). This package holds the
ctypes bindings to it and the seeded random-init artifact writer.
"""
