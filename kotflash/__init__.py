"""``kotflash``: the reference's import path, served by the MI355X build.

Callers of the reference import ``kotflash`` and its submodules by name
(reference kotflash/__init__.py:1-7; its tests/test_attention.py:8-9,
tests/test_kv_cache.py:7, tests/test_planning.py:5,
tests/test_preallocated_cache.py:6, examples/gqa_kv_cache_decode.py:13-14,
benchmarks/benchmark_decode.py:26-27). This package answers to those names
with the ``kotflash_amd`` modules that implement them. Each reference
submodule name is registered in ``sys.modules`` as the implementing module
itself, not a copy, so ``kotflash.cache`` and ``kotflash_amd.cache`` are one
object: module state, ``isinstance`` checks and monkeypatching are shared.

    kotflash.attention       kotflash_amd.attention
    kotflash.cache           kotflash_amd.cache
    kotflash._planning       kotflash_amd._planning
    kotflash._cuda_append    kotflash_amd._hip_append (append_kv_cuda)
    kotflash.kernels.*       kotflash.kernels (triton_* names -> hip_* modules)

As in the reference, the package attribute ``kotflash.attention`` is the
``attention`` function, while ``from kotflash.attention import ...`` reaches
the module.
"""
import importlib as _importlib
import sys as _sys

_SUBMODULES = {
    "attention": "kotflash_amd.attention",
    "cache": "kotflash_amd.cache",
    "_planning": "kotflash_amd._planning",
    "_cuda_append": "kotflash_amd._hip_append",
}
for _name, _target in _SUBMODULES.items():
    _sys.modules[f"{__name__}.{_name}"] = _importlib.import_module(_target)

from . import kernels  # noqa: E402  (registers kotflash.kernels.triton_*)
from kotflash_amd import __version__, attention, hip_available  # noqa: E402
from kotflash_amd.kernels.hip_forward import triton_available, triton_turing_supported  # noqa: E402

for _name in ("cache", "_planning", "_cuda_append"):
    globals()[_name] = _sys.modules[f"{__name__}.{_name}"]
del _name, _target

__all__ = ["attention", "hip_available", "triton_available", "triton_turing_supported"]
