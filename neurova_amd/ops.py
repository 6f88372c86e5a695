"""Op resolution for the low-bit path (``cuda_ops()``).

Mirrors ``langburst/langburst/ops.py:811-823`` with one deliberate difference:
this build has no CPU fallback.  ``cuda_ops()`` returns the compiled
``langburst_cuda`` module or raises, including when the reference's
``LANGBURST_CPU_FALLBACK`` / ``LANGBURST_SKIP_CUDA_EXT`` switches ask for the
CPU path, so a caller can never silently run something other than the gfx950
kernels.
"""
from __future__ import annotations

import os
from functools import lru_cache


class ExtensionMissingError(RuntimeError):
    pass


@lru_cache(maxsize=1)
def cuda_ops():
    if os.environ.get("LANGBURST_CPU_FALLBACK", "0") == "1" or os.environ.get("LANGBURST_SKIP_CUDA_EXT", "0") == "1":
        raise ExtensionMissingError(
            "this MI355X build provides no CPU fallback for the low-bit ops; "
            "unset LANGBURST_CPU_FALLBACK / LANGBURST_SKIP_CUDA_EXT"
        )
    from . import load_extension

    try:
        return load_extension()
    except ImportError as exc:
        raise ExtensionMissingError(
            "langburst_cuda is not built. Build the gfx950 kernels with:\n  python -m neurova_amd.build"
        ) from exc
