"""CPU restatement of the Omega section of OmegaNeuralMemory.store_memories (TEST INFRASTRUCTURE ONLY).

Only `tests/` may import this module; the product package never does.

Per parameter tensor of the memory MLP, over per-chunk surprises `[(B H), n, *param]`
(atlas_pytorch/omega.py:262-318):

    m^o_t   = am^o_t * m^o_{t-1} + m^{o-1}_t,  m^{-1} = surprise,  m^o_{-1} = last_momentum[o]  (:262-270, AssocScan)
    base_t  = sum_o combine^o_t m^o_t  (learned combine, :272-273)  or  m^{O-1}_t  (:275)
    g_t     = U_t * base_t                                     (omega gate, :277-283)
    w_t     = sum_{j<e} ext[e-1+t-j],  ext = [omega_buf; g]    (:286-300, cumsum window over n)
    next_buf = ext[-(e-1):]                                    (:302)
    update  = AssocScan(1 - decay, w, prev=last_update, remove_prev=False)   (:315)  -> n + 1 steps
    if all_bh max_t U < 1e-3: update = 0                       (:311-313)
    next_last_update = update[:, -1]                           (:321)

Two independent forms: `omega_store_chain` follows the reference op sequence (stacked scans,
cumsum-difference window on the concatenation); `omega_store_chain_loop` is a per-chunk textbook
loop. How they are pinned (tests/test_oracle_omega.py): agreement in float64; chunk invariance
(n chunks at once == two calls carrying last_update, last_momentum and the buffer); reductions to
closed forms (window 1, no momentum, no gate: a plain decay scan; constant gates: geometric sums);
the gate-below-1e-3 short-circuit; the window's known answers (tests/golden).

The reference's short-circuit branch returns n zero steps while its scanned branch returns n + 1;
both forms here return n + 1 zero steps (the product's shape, which needs no host sync to choose),
with next_last_update = 0 as in the reference; reference_shapes=True returns the reference's n.

The Newton-Schulz points (omega.py:304-305 `spectral_norm_surprises`, :317-318
`use_muon_optimizer`) take an orthogonaliser; `newtonschulz5` restates the published quintic
iteration NeuralMemory uses (neural_memory.py:158-186). It is pinned by its action on singular
values (tests/test_oracle_omega.py): the iteration maps X = U diag(s) V^T to
U diag(p^5(s / ||s||)) V^T with p(x) = a x + b x^3 + c x^5.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .recurrence import scalar_assoc_scan_sequential, sliding_sum_along_time


def _bcast(g: Tensor, like: Tensor) -> Tensor:
    while g.ndim < like.ndim:
        g = g.unsqueeze(-1)
    return g


def newtonschulz5(t: Tensor, steps: int = 5, eps: float = 1e-7, coefs=(3.4445, -4.7750, 2.0315)) -> Tensor:
    """neural_memory.py:158-186: tensors of at most 3 dims unchanged; otherwise per matrix over the
    trailing two dims (transposed when rows > cols): X / max(||X||_F, eps), then `steps` times
    A = X X^T, B = b A + c A A, X = a X + B X."""
    if t.ndim <= 3:
        return t
    transpose = t.shape[-2] > t.shape[-1]
    x = t.transpose(-1, -2) if transpose else t
    x = x / x.norm(dim=(-1, -2), keepdim=True).clamp(min=eps)
    a, b, c = coefs
    for _ in range(steps):
        A = x @ x.transpose(-1, -2)
        B = b * A + c * A @ A
        x = a * x + B @ x
    return x.transpose(-1, -2) if transpose else x


def omega_store_chain(surprise: Tensor, decay_factor: Tensor, last_update: Tensor, *,
                      adaptive_momentum: Tensor | None = None, last_momentum: Tensor | None = None,
                      combine_momentums: Tensor | None = None, omega_gate: Tensor | None = None,
                      omega_window: int = 1, omega_buf: Tensor | None = None,
                      spectral_norm=None, muon=None, reference_shapes: bool = False):
    """surprise [BH, n, *p]; decay_factor [BH, n] (or [BH, n, 1]); last_update [BH, *p];
    adaptive_momentum [O, BH, n] with last_momentum [O, BH, *p] (momentum on); combine_momentums
    [O, BH, n]; omega_gate [BH, n]; omega_buf [BH, e-1, *p]. Returns (update [BH, n+1, *p],
    next_last_update [BH, *p], next_last_momentum [O, BH, *p] or None, next_buf [BH, e-1, *p] or None)."""
    BH, n = surprise.shape[:2]
    base = surprise
    next_lm = None
    if adaptive_momentum is not None:                                  # omega.py:262-275
        momentum = surprise
        moms = []
        for o in range(adaptive_momentum.shape[0]):
            momentum = scalar_assoc_scan_sequential(adaptive_momentum[o], momentum, prev=last_momentum[o])
            moms.append(momentum)
        moms = torch.stack(moms)
        next_lm = moms[:, :, -1]
        if combine_momentums is not None:
            base = (_bcast(combine_momentums, moms) * moms).sum(dim=0)
        else:
            base = moms[-1]
    gated = base * _bcast(omega_gate, base) if omega_gate is not None else base   # :277-283
    next_buf = None
    if omega_window > 1:                                               # :286-302
        e = omega_window
        prev_buf = omega_buf if omega_buf is not None else gated.new_zeros((BH, e - 1, *gated.shape[2:]))
        ext = torch.cat([prev_buf, gated], dim=1)
        update = sliding_sum_along_time(ext, e)[:, -n:]
        next_buf = ext[:, -(e - 1):]
    else:
        update = gated
    if spectral_norm is not None:                                      # :304-305
        update = spectral_norm(update)
    off = omega_gate is not None and bool(torch.all(omega_gate.reshape(BH, n).amax(dim=1) < 1e-3))   # :311
    if off and reference_shapes:
        zero = torch.zeros_like(update)
        return zero, zero[:, -1], next_lm, next_buf
    decay = decay_factor.reshape(BH, n)
    scanned = scalar_assoc_scan_sequential(1.0 - decay, update, prev=last_update, remove_prev=False)   # :315
    if muon is not None:                                               # :317-318
        scanned = muon(scanned)
    if off:                                                            # :311-313
        scanned = torch.zeros_like(scanned)
    return scanned, scanned[:, -1], next_lm, next_buf


def omega_store_chain_loop(surprise: Tensor, decay_factor: Tensor, last_update: Tensor, *,
                           adaptive_momentum: Tensor | None = None, last_momentum: Tensor | None = None,
                           combine_momentums: Tensor | None = None, omega_gate: Tensor | None = None,
                           omega_window: int = 1, omega_buf: Tensor | None = None):
    """The same chain as a per-chunk loop (textbook form), same contract as omega_store_chain."""
    BH, n = surprise.shape[:2]
    e = omega_window
    O = adaptive_momentum.shape[0] if adaptive_momentum is not None else 0
    m = [last_momentum[o] for o in range(O)]
    hist = [omega_buf[:, i] for i in range(e - 1)] if (e > 1 and omega_buf is not None) else \
        [torch.zeros_like(surprise[:, 0]) for _ in range(e - 1)]
    u = last_update
    outs = [last_update]
    decay = decay_factor.reshape(BH, n)
    for t in range(n):
        x = surprise[:, t]
        for o in range(O):
            m[o] = _bcast(adaptive_momentum[o, :, t], x) * m[o] + x
            x = m[o]
        if O and combine_momentums is not None:
            x = sum(_bcast(combine_momentums[o, :, t], m[o]) * m[o] for o in range(O))
        if omega_gate is not None:
            x = _bcast(omega_gate.reshape(BH, n)[:, t], x) * x
        hist.append(x)
        w = sum(hist[-e:]) if e > 1 else x
        u = _bcast(1.0 - decay[:, t], w) * u + w
        outs.append(u)
    update = torch.stack(outs, dim=1)
    if omega_gate is not None and bool((omega_gate.reshape(BH, n).amax(dim=1) < 1e-3).all()):
        update = torch.zeros_like(update)
    next_lm = torch.stack(m) if O else None
    next_buf = torch.stack(hist[-(e - 1):], dim=1) if e > 1 else None
    return update, update[:, -1], next_lm, next_buf
