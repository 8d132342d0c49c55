"""Right-affine associative scan (atlas_pytorch/affine_scan.py:36-158) on the HIP kernels.

    H_t = H_{t-1} A_t + B_t,   A: [N, T, D, D],  B: [N, T, R, D],  prev = H_0: [N, R, D]

`affine_associative_scan(A, B, *, prev=None, remove_prev=False)` returns [N, T, R, D] (or
[N, T+1, R, D] starting with prev when prev is given and remove_prev is False), with gradients
for A, B and prev. The scan runs in fp32 in libatlas_mem.so (atlas_affine_scan_fwd / _bwd:
chunked compose / chain / apply passes on the fp32 matrix cores, D, R <= 64); other dtypes are
computed in fp32 and cast back.
"""

from __future__ import annotations

from torch import Tensor

from .functional import affine_associative_scan

__all__ = ["affine_associative_scan"]
