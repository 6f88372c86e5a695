"""MI355X (gfx950) build of LangBurst's low-bit weight-only projection path.

Importing this package registers the compiled PyTorch-ROCm module under the
reference's module name ``langburst_cuda`` (so ``import langburst_cuda`` and
``neurova_amd.ops.cuda_ops()`` both resolve to it).  The HIP kernels live in
``lib/liblangburst_lowbit.so`` behind the C ABI declared in
``include/langburst_lowbit.h``; build both with ``python -m neurova_amd.build``.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import sys
from pathlib import Path

__all__ = ["extension_path", "library_path", "load_extension"]

_PKG = Path(__file__).resolve().parent


def extension_path() -> Path:
    return _PKG / "_ext" / "langburst_cuda.so"


def library_path() -> Path:
    return _PKG / "lib" / "liblangburst_lowbit.so"


def load_extension():
    """Import the compiled ``langburst_cuda`` module, registering it in ``sys.modules``.

    Raises ``ImportError`` when the extension has not been built.
    """
    mod = sys.modules.get("langburst_cuda")
    if mod is not None:
        return mod
    path = extension_path()
    if not path.exists():
        raise ImportError(f"langburst_cuda is not built ({path} missing); run `python -m neurova_amd.build`")
    import torch  # noqa: F401  (binds the PyTorch-ROCm HIP runtime before our library loads)

    loader = importlib.machinery.ExtensionFileLoader("langburst_cuda", str(path))
    spec = importlib.util.spec_from_file_location("langburst_cuda", str(path), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    sys.modules["langburst_cuda"] = mod
    return mod


try:  # register eagerly when built; stay importable (for building) when not
    load_extension()
except ImportError:
    pass
