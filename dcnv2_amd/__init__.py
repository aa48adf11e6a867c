"""dcnv2_amd: MI355X (gfx950) modulated deformable convolution v2.

Drop-in for TseLin-Liu/DCNv2's operator path: ``dcnv2_amd._C`` mirrors the
native module ``Conv2d._C`` and ``dcnv2_amd.dcn_v2_mm`` mirrors
``dcn_v2_mm.py``.  The kernels live in ``lib/libdcnv2_amd.so`` (C ABI:
``include/dcnv2_amd.h``); build them with ``python -m dcnv2_amd.build``.
"""
from . import _C  # noqa: F401
from .dcn_v2_mm import DCN, DCNv2, _DCNv2, dcn_v2_conv, deform_conv2d  # noqa: F401

__all__ = ["DCN", "DCNv2", "dcn_v2_conv", "deform_conv2d", "_C"]
