"""Scan primitives of atlas_pytorch/omega.py on the HIP kernels.

`OmegaNeuralMemory.store_memories` (omega.py:120-330) drives its Omega section with two
primitives over per-chunk tensors `[(B H), n, ...]`: the inclusive window sum along n
(`_sliding_sum_along_n`, omega.py:24-33) and the scalar-gated associative scan (`AssocScan`,
used at omega.py:267 and :315). Both are provided here on ROCm tensors (libatlas_mem.so:
atlas_window_sum, atlas_scan_fwd / atlas_scan_bwd), with the same argument conventions, so the
module's per-sample gradient code (kept in PyTorch) can call them unchanged.
"""

from __future__ import annotations

from torch import Tensor

from .functional import AssocScan, assoc_scan, window_sum

__all__ = ["_sliding_sum_along_n", "assoc_scan", "AssocScan"]


def _sliding_sum_along_n(x: Tensor, window: int) -> Tensor:
    """Sum of the last `window` entries along dim 1, inclusive (omega.py:24-33)."""
    return window_sum(x, window)
