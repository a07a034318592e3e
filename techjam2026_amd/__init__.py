"""kf950: the KernelForge transformer-layer forward, native to MI355X (gfx950).

Drop-in: `techjam2026_amd.submission.UserOptimizedTransformer`. Kernels: libkf950.so
(C ABI in include/kf950.h), bound through ctypes in `_lib.py` and wrapped with the
reference's op signatures in `kernels.py`; the fused stack is `optimized.FusedTransformer`.
"""
__version__ = "0.1.0"
