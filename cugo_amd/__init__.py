"""cugo_amd - MI355X (gfx950) batch engine for Cugo's two-player Shin Matgo.

The product is libcugo_hip.so (HIP kernels behind the C ABI of include/cugo_hip.h) and the
PyTorch-ROCm extension `_cugo_torch50_hip` over it.  `load_extension()` returns that module;
it is a drop-in for the reference's `cugo_torch50_ext.load_extension()`
(python/cugo_torch50_ext.py:141-193).  Build in-tree with `python -m cugo_amd.build`.
"""

from __future__ import annotations

from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIBRARY = PKG_DIR / "libcugo_hip.so"

from .cugo_torch50_ext import load_extension  # noqa: E402

__all__ = ["LIBRARY", "PKG_DIR", "load_extension"]
