"""SageAttention quantized attention on MI355X (gfx950).

Drop-in for LuXuxue/sageattention-rdna3's package surface
(sageattention/__init__.py:1-4): ``sageattn``, ``sageattn_qk_int8_pv_fp16_cuda``
and ``__version__``.
"""
from .core import sageattn, sageattn_qk_int8_pv_fp16_cuda

__all__ = ["sageattn", "sageattn_qk_int8_pv_fp16_cuda"]
__version__ = "0.1.0"
