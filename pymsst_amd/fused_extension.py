"""Extension loader: MI355X counterpart of the reference's ``fused_extension.py``.

Reference: baicai-1145/pymsst ``src/pymsst/training/fused_extension.py:11-57``.
Same public names (``FusedKernelUnavailable``, ``load_fused_band_split_extension``)
and the same failure contract: any reason the fused kernels cannot run raises
``FusedKernelUnavailable`` with a message.  The difference is the build: the
reference JIT-compiles CUDA with ``torch.utils.cpp_extension.load``; this loader
binds the prebuilt gfx950 library ``libpymsst_amd.so`` through its C ABI
(build it with ``python -m pymsst_amd.build``).  ``PYMSST_AMD_LIB`` overrides the
library path.
"""

from __future__ import annotations

from functools import lru_cache

import torch

from ._lib import FusedKernelUnavailable, load_library


def load_fused_band_split_extension():
    """Return the (cached) :class:`~pymsst_amd.extension.HipFusedExtension`.

    Raises :class:`FusedKernelUnavailable` when there is no GPU, when torch was
    not built for ROCm, or when the library is missing or fails to load
    (``fused_extension.py:15-20,39-41,56-57``).
    """
    if torch.version.hip is None:
        raise FusedKernelUnavailable("PyTorch was not built with ROCm/HIP")
    if not torch.cuda.is_available():
        raise FusedKernelUnavailable("no HIP GPU is available")
    return _cached_extension()


@lru_cache(maxsize=1)
def _cached_extension():
    load_library()
    from .extension import HipFusedExtension

    return HipFusedExtension()


__all__ = ["FusedKernelUnavailable", "load_fused_band_split_extension"]
