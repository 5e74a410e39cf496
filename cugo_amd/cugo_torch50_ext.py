"""Drop-in for the reference loader `cugo_torch50_ext.load_extension`
(python/cugo_torch50_ext.py:141-193).

The reference JIT-compiles its CUDA extension on first use; here the HIP extension is
built ahead of time, in-tree (`python -m cugo_amd.build`), and this function imports it.
There is no fallback: without a GPU or without the built extension it raises.
"""

from __future__ import annotations

import importlib
from typing import Any

_MODULE = "cugo_amd._cugo_torch50_hip"


def load_extension(*, verbose: bool = False) -> Any:
    import torch

    if not torch.cuda.is_available():  # same condition and message as the reference
        raise RuntimeError("PyTorch CUDA is not available")
    try:
        module = importlib.import_module(_MODULE)
    except ImportError as exc:  # pragma: no cover - depends on the build
        raise RuntimeError(
            "the cugo_amd HIP extension is not built; run `python -m cugo_amd.build`") from exc
    if verbose:
        print(f"cugo_amd: loaded {module.__file__}")
    return module
