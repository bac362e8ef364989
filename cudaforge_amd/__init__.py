"""MI355X-native (gfx950) speculative-decoding verification.

Drop-in for the verification path of Bahaa-Labs/CUDAForge:

* ``cudaforge_amd.speculative`` mirrors ``cudaforge/speculative.py``
  (``SpeculativeEngine``, ``SpeculativeBatchResult``);
* ``SpeculativeConfig``, ``SpeculativeVerificationResult`` and
  ``SpeculativeEngine`` at package level mirror the reference's native engine
  (``cudaforge/__init__.py:18-20``);
* ``cudaforge_amd.verify`` holds the tensor-level entry points over the C ABI
  of ``libcfa.so`` (include/cudaforge_amd.h).

Every compute call goes through the HIP library; importing this package does
not load it, but the first call does and raises if it is missing.
"""
from .native import SpeculativeConfig, SpeculativeEngine, SpeculativeVerificationResult

__version__ = "0.1.0"

__all__ = [
    "SpeculativeConfig",
    "SpeculativeEngine",
    "SpeculativeVerificationResult",
    "__version__",
]
