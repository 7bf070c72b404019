"""megakernel_amd: MI355X (gfx950) persistent decode megakernel for a
Qwen3-0.6B-shaped decoder, behind the reference's C ABI (megakernel.so).

Product modules: ``_lib`` (ctypes binding), ``bridge`` (MegakernelEngine),
``weights`` (flat weight format, device-side synthetic weights), ``config``
(shapes and byte accounting), ``launcher`` (build and device detection).
"""
from .config import BASELINE, QWEN3_06B, TINY, ModelShape  # noqa: F401

__all__ = ["BASELINE", "QWEN3_06B", "TINY", "ModelShape"]
