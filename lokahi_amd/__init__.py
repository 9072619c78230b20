"""lokahi_amd — the Strata per-token inference hot path on AMD MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (``include/strata_hip.h``,
``lokahi_amd/_lib/libstrata_hip.so``), bound with ctypes and registered as the
``"hip"`` backend of a registry that mirrors the reference's
``ollm.backends`` hook.  Importing the package does not touch the GPU; the
library is loaded on first use and every op fails loudly without it.
"""
__version__ = "0.1.0"
