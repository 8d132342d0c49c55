"""The Omega section of atlas_pytorch/omega.py on the HIP kernels.

`OmegaNeuralMemory.store_memories` (omega.py:120-330) turns per-chunk surprises of each memory-MLP
parameter, `[(B H), n, *param]`, into per-chunk weight updates. Its Omega section
(omega.py:262-318) is provided here as `omega_store_chain`, a function over plain tensors built on
the library's primitives: the scalar-gated scan (`atlas_scan_fwd` / `_bwd`: the momentum scans and
the `1 - decay` scan with `remove_prev=False`) and the inclusive window sum along n
(`atlas_window_sum`: the omega window over the carried `__omega_buf` and the chunk). The
per-sample gradients that produce the surprises (torch.func vmap over the memory MLP) stay in
PyTorch, as does NeuralMemory itself.

Also here: `_sliding_sum_along_n` (omega.py:24-33), the scan `assoc_scan` / `AssocScan`, and the
feature map `apply_poly_features` (omega.py:90-118).
"""

from __future__ import annotations

import math
from typing import Callable

import torch
from torch import Tensor

from .functional import AssocScan, assoc_scan, tensor_feature_map, window_sum

__all__ = ["_sliding_sum_along_n", "assoc_scan", "AssocScan", "omega_store_chain", "apply_poly_features",
           "OmegaPolyFeatures", "OMEGA_GATE_OFF", "newtonschulz5"]

OMEGA_GATE_OFF = 1e-3   # every gate below this (over the whole batch): the chunk's updates are zero (omega.py:311)


def _sliding_sum_along_n(x: Tensor, window: int) -> Tensor:
    """Sum of the last `window` entries along dim 1, inclusive (omega.py:24-33)."""
    return window_sum(x, window)


def _bcast(g: Tensor, like: Tensor) -> Tensor:
    while g.ndim < like.ndim:
        g = g.unsqueeze(-1)
    return g


def newtonschulz5(t: Tensor, steps: int = 5, eps: float = 1e-7,
                  coefs: tuple[float, float, float] = (3.4445, -4.7750, 2.0315)) -> Tensor:
    """Quintic Newton-Schulz orthogonalisation of the trailing two dims (the published Muon
    iteration that NeuralMemory's `newtonschulz5`, neural_memory.py:158-186, computes): tensors with
    at most 3 dims are returned unchanged; otherwise each matrix X (transposed first when it has
    more rows than columns) is scaled to unit Frobenius norm (at least eps) and iterated
    `steps` times as A = X X^T, X <- a X + (b A + c A A) X. Runs in fp32 on torch's matrix
    products (both operands contiguous) and returns t's dtype. A default for the orthogonaliser
    arguments of `omega_store_chain`."""
    if t.ndim <= 3:
        return t
    dt = t.dtype
    x = t.float()
    transpose = x.shape[-2] > x.shape[-1]
    if transpose:
        x = x.transpose(-1, -2)
    lead = x.shape[:-2]
    x = x.reshape(-1, *x.shape[-2:]).contiguous()
    x = x / x.norm(dim=(-1, -2), keepdim=True).clamp(min=eps)
    a, b, c = coefs
    for _ in range(steps):
        A = torch.matmul(x, x.transpose(-1, -2).contiguous())
        B = b * A + c * torch.matmul(A, A)
        x = a * x + torch.matmul(B, x)
    x = x.reshape(*lead, *x.shape[-2:])
    if transpose:
        x = x.transpose(-1, -2)
    return x.contiguous().to(dt)


def omega_store_chain(surprise: Tensor, decay_factor: Tensor, last_update: Tensor, *,
                      adaptive_momentum: Tensor | None = None, last_momentum: Tensor | None = None,
                      combine_momentums: Tensor | None = None, omega_gate: Tensor | None = None,
                      omega_window: int = 1, omega_buf: Tensor | None = None,
                      spectral_norm: Callable[[Tensor], Tensor] | None = None,
                      muon: Callable[[Tensor], Tensor] | None = None,
                      reference_shapes: bool = False):
    """The loop body of omega.py:254-322 for one parameter, on ROCm tensors.

    surprise [BH, n, *p] (the negated per-chunk gradients); decay_factor [BH, n] or [BH, n, 1];
    last_update [BH, *p]; adaptive_momentum [O, BH, n] (or [O, BH, n, 1]) with last_momentum
    [O, BH, *p] when the memory has momentum (order O); combine_momentums [O, BH, n] for the learned
    combination of the orders; omega_gate [BH, n] (or [BH, n, 1]); omega_buf [BH, e-1, *p], the
    carried `<name>__omega_buf` (zeros when None).

    Returns (update [BH, n+1, *p] led by last_update, next_last_update [BH, *p],
    next_last_momentum [O, BH, *p] or None, next_omega_buf [BH, e-1, *p] or None).

    When every gate of the batch is below 1e-3 the updates are zero (omega.py:311-313), chosen on
    the device (no host synchronisation); the result keeps the scanned branch's n + 1 steps (the
    reference's zero branch has n) and next_last_update is zero as in the reference.
    reference_shapes=True takes the reference's choice on the host instead (one synchronisation)
    and returns its n zero steps in that branch.

    The two Newton-Schulz points of the reference are caller-supplied orthogonalisers (for
    example `newtonschulz5`): spectral_norm (the memory's `spectral_norm_surprises`) is applied to
    the windowed update before the scan (omega.py:304-305); muon (`use_muon_optimizer`) to the
    scanned result (omega.py:317-318), before next_last_update is taken from it.
    """
    if surprise.dim() < 2:
        raise ValueError(f"surprise must be [BH, n, ...], got {tuple(surprise.shape)}")
    BH, n = surprise.shape[:2]
    if decay_factor.numel() != BH * n:
        raise ValueError(f"decay_factor must hold [BH={BH}, n={n}] values, got {tuple(decay_factor.shape)}")
    if tuple(last_update.shape) != (BH, *surprise.shape[2:]):
        raise ValueError(f"last_update must be {(BH, *surprise.shape[2:])}, got {tuple(last_update.shape)}")
    if omega_window < 1:
        raise ValueError("omega_window must be >= 1")
    base = surprise
    next_lm = None
    if adaptive_momentum is not None:                                  # omega.py:262-275
        O = adaptive_momentum.shape[0]
        if last_momentum is None or tuple(last_momentum.shape) != (O, BH, *surprise.shape[2:]):
            raise ValueError("last_momentum must be [O, BH, *param] with adaptive_momentum [O, BH, n]")
        am = adaptive_momentum.reshape(O, BH, n)
        momentum = surprise
        moms = []
        for o in range(O):
            momentum = assoc_scan(am[o], momentum, prev=last_momentum[o])
            moms.append(momentum)
        moms = torch.stack(moms)
        next_lm = moms[:, :, -1]
        if combine_momentums is not None:
            base = (_bcast(combine_momentums.reshape(O, BH, n), moms) * moms).sum(dim=0)
        else:
            base = moms[-1]
    gate = omega_gate.reshape(BH, n) if omega_gate is not None else None
    gated = base * _bcast(gate, base) if gate is not None else base   # omega.py:277-283
    next_buf = None
    if omega_window > 1:                                               # omega.py:286-302
        e = omega_window
        if omega_buf is None:
            omega_buf = gated.new_zeros((BH, e - 1, *gated.shape[2:]))
        elif tuple(omega_buf.shape) != (BH, e - 1, *gated.shape[2:]):
            raise ValueError(f"omega_buf must be {(BH, e - 1, *gated.shape[2:])}, got {tuple(omega_buf.shape)}")
        ext = torch.cat([omega_buf.to(gated.dtype), gated], dim=1)
        update = _sliding_sum_along_n(ext, e)[:, -n:]
        next_buf = ext[:, -(e - 1):]
    else:
        update = gated
    if spectral_norm is not None:                                      # omega.py:304-305
        update = spectral_norm(update)
    if reference_shapes and gate is not None and bool(torch.all(gate.amax(dim=1) < OMEGA_GATE_OFF)):
        zero = torch.zeros_like(update)                                # omega.py:311-313: n zero steps
        return zero, zero[:, -1], next_lm, next_buf
    scanned = assoc_scan(1.0 - decay_factor.reshape(BH, n), update, prev=last_update, remove_prev=False)   # :315
    if muon is not None:                                               # omega.py:317-318
        scanned = muon(scanned)
    if gate is not None and not reference_shapes:                      # omega.py:311-313, on the device
        off = torch.all(gate.amax(dim=1) < OMEGA_GATE_OFF)
        scanned = torch.where(off, torch.zeros_like(scanned), scanned)
    return scanned, scanned[:, -1], next_lm, next_buf


def apply_poly_features(x: Tensor, degree: int, mode: str, proj_cache: dict | None = None) -> Tensor:
    """omega.py:90-118: 'elementwise' sum_{i=1..degree} x^i; 'tensor' [x; vec(x x^T)] @ P with a
    fixed random P [d + d^2, d] = randn / sqrt(d + d^2) drawn once per (feature size, d, device
    type) and kept in `proj_cache` (not a parameter, as in the reference); 'off' or degree <= 1:
    x. The tensor map runs on the fused kernels (`functional.tensor_feature_map`)."""
    if degree <= 1 or mode == 'off':
        return x
    if mode == 'elementwise':
        out = x
        power = x
        for _ in range(2, degree + 1):
            power = power * x
            out = out + power
        return out
    if mode == 'tensor':
        d = x.shape[-1]
        feat_dim = d + d * d
        key = (feat_dim, d, x.device.type)
        cache = proj_cache if proj_cache is not None else {}
        proj = cache.get(key)
        if proj is None:
            proj = torch.randn(feat_dim, d, device=x.device, dtype=x.dtype) / math.sqrt(feat_dim)
            cache[key] = proj
        return tensor_feature_map(x, proj.to(x.dtype))
    return x


class OmegaPolyFeatures(torch.nn.Module):
    """The key / query feature map of OmegaNeuralMemory (omega.py:90-118) as a module with its
    own projection cache."""

    def __init__(self, degree: int = 1, mode: str = 'off'):
        super().__init__()
        self.degree = int(degree)
        self.mode = mode
        self._poly_proj_cache: dict = {}

    def forward(self, x: Tensor) -> Tensor:
        return apply_poly_features(x, self.degree, self.mode, self._poly_proj_cache)
