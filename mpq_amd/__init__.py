"""mpq_amd: MI355X-native per-layer quantization hot path of MPQ.

Hand-written HIP kernels for gfx950 behind a C-ABI (``include/mpq_amd.h``),
driven from Python with the reference's own entry points (``solver``,
``priors``, ``polish``, ``adapters``).  Tensors live on the ROCm device;
there is no CPU fallback.
"""
__all__ = []
