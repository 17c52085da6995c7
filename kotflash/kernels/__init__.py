"""``kotflash.kernels``: the reference's kernel-module names (reference
kotflash/kernels/triton_forward.py, triton_backward.py, triton_decode.py)
bound to the gfx950 launchers that replace them. The Triton kernels are not
part of this build; the launcher functions keep the reference's names and
signatures (``attention_forward``, ``attention_backward``,
``strided_decode_supported``, ``attention_forward_strided_decode``,
``attention_forward_strided_append``, ``triton_available``,
``triton_turing_supported``)."""
import importlib as _importlib
import sys as _sys

_SUBMODULES = {
    "triton_forward": "kotflash_amd.kernels.hip_forward",
    "triton_backward": "kotflash_amd.kernels.hip_backward",
    "triton_decode": "kotflash_amd.kernels.hip_decode",
}
for _name, _target in _SUBMODULES.items():
    _module = _importlib.import_module(_target)
    _sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module
del _name, _target, _module
