"""vxg_amd -- MI355X (gfx950) compressed-weight matmul engine for vxg-tensor.

The device path is the HIP library ``libvxt_hip.so`` behind the C ABI in
``include/vxt_hip.h``; :mod:`vxg_amd.engine` is the host-side mirror of the
reference's engine API, :mod:`vxg_amd.formats` the weight containers and
:mod:`vxg_amd.synth` the seeded benchmark inputs.
"""
from .formats import Cb4G64Matrix, CodebookMatrix, FormatError, Q8Matrix  # noqa: F401

__all__ = ["Cb4G64Matrix", "CodebookMatrix", "FormatError", "Q8Matrix"]
