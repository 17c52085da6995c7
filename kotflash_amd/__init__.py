"""kotflash_amd: MI355X (gfx950) attention kernels behind the KOTFlash API.

``attention`` and ``kotflash_amd.cache`` are drop-ins for the reference's
``kotflash.attention`` and ``kotflash.cache`` (reference kotflash/__init__.py:1-7);
the kernels are hand-written HIP for gfx950 in ``csrc/`` behind the C ABI of
``include/kotflash_amd.h``.
"""
from .attention import attention
from .kernels.hip_forward import hip_available, triton_available, triton_turing_supported

__all__ = ["attention", "hip_available", "triton_available", "triton_turing_supported"]
__version__ = "0.1.0"
