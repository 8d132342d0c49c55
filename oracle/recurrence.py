"""CPU restatement of the atlas-rnn memory-layer recurrence (TEST INFRASTRUCTURE ONLY).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import this
module. The product package never does.

Semantics (per head-batch row `bh`), restated from
`atlas_pytorch/rnn_memory.py:300-406` (Titans cell) and `:605-730` (Omega cell):

    delta_t = S_ref phi_t - v_t                         (rnn_memory.py:659-660)
    P_t     = delta_t phi_t^T                           (:663)
    g_t     = sum_{j=0}^{e-1} w[t, j] * P_{t-j}         (:666-687; window with carried buffer)
    Z_t     = beta_t Z_{t-1} + g_t                      (:698, AssocScan)
    S_t     = alpha_t S_{t-1} - eta_t Z_t               (:699-700)
              (no momentum: S_t = alpha_t S_{t-1} - eta_t g_t, :704-705)
    y_t     = S_{t-1} psi_t,  S_{-1} = S0               (:712-717)
    S_T     = clamp(S_{T-1}, -100, 100),  Z_T = Z_{T-1} (:701-702)
    buffer' = last e-1 of [buffer; Ghat_0 .. Ghat_{T-1}] (:673-687)

`scan_chunk_len` (`rnn_memory.py:584-601`) keeps S_ref at the call-start state and clamps S at
the end of every chunk; `clamp_every` reproduces that.

Gate modes (`lag_weights`):
* None: w = 1.
* token gate u [BH, T] (the reference's `omega_gate`, rnn_memory.py:666-668): the window sums
  u_p * P_p, so w[t, j] = u_{t-j}; the carried buffer holds gated products.
* lag gate U [BH, T, e] (BASELINE config C3 extension, no reference counterpart):
  w[t, j] = U[t, j]; the carried buffer holds ungated products and is weighted by U too.

How each function is pinned (tests/test_oracle.py):
* scalar_assoc_scan / _sequential: the reference's closed-form AssocScan tests
  (tests/test_rnn_all.py:832-887: identity, additive t+1, decay 0.5^(t+1), mixed 1/1.5/1.75)
  and prev-chaining (tests/test_titans.py:681-711); the two forms agree with each other.
* sliding_sum_along_time: known answers tests/test_rnn_all.py:890-896 and tests/test_atlas.py:147-169.
* poly_feature_map: closed forms (x + x^2 + x^3; tensor map against explicit Kronecker).
* memory_recurrence_loop vs memory_recurrence_vectorised: two independent forms that must agree
  in float64; plus closed forms: gated linear attention (S_ref=0, e=1, no momentum), cumulative
  linear attention (alpha=1), u=0 (no update), beta=0 (momentum == no momentum), e=1 Omega ==
  Titans, delta phi^T == S_ref G - B identity (tests/test_rnn_memory_refactor.py:25-50), chunk
  invariance (tests/test_rnn_all.py:335-374), brute-force torch.autograd.gradcheck of the loop
  (pins the backward used as the gradient oracle).
* affine_associative_scan vs affine_scan_sequential (sequential matmul loop).
"""

from __future__ import annotations

import torch
from torch import Tensor


# -----------------------------------------------------------------------------
# Scalar-gated associative scan (third-party `assoc_scan.AssocScan`, unpinned version).
# Call sites: rnn_memory.py:363,369,379,698,700,705; omega.py:267,315.
# out_t = gates_t * out_{t-1} + inputs_t ; prev is out_{-1}. remove_prev defaults to
# "prev given" (T outputs); remove_prev=False with prev returns T+1 outputs starting with prev.
# -----------------------------------------------------------------------------

def _expand_gates(gates: Tensor, inputs: Tensor) -> Tensor:
    g = gates
    while g.ndim < inputs.ndim:
        g = g.unsqueeze(-1)
    return g


def scalar_assoc_scan_sequential(gates: Tensor, inputs: Tensor, prev: Tensor | None = None,
                                 remove_prev: bool | None = None) -> Tensor:
    """Textbook loop form of AssocScan (semantics from its call sites listed above)."""
    g = _expand_gates(gates, inputs)
    T = inputs.shape[1]
    cur = prev if prev is not None else torch.zeros_like(inputs[:, 0])
    outs = []
    for t in range(T):
        cur = g[:, t] * cur + inputs[:, t]
        outs.append(cur)
    out = torch.stack(outs, dim=1) if T > 0 else inputs.clone()
    if remove_prev is None:
        remove_prev = prev is not None
    if prev is not None and not remove_prev:
        out = torch.cat([prev.unsqueeze(1), out], dim=1)
    return out


def _binary_op(a1, b1, a2, b2):
    # compose x -> a1 x + b1 then x -> a2 x + b2
    return a1 * a2, a2 * b1 + b2


def _odd_even_scan(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor]:
    """Log-depth odd/even recursion (the published structure of jax-style associative_scan,
    which AssocScan's pure-torch path follows)."""
    T = a.shape[1]
    if T < 2:
        return a, b
    a_red, b_red = _binary_op(a[:, :-1:2], b[:, :-1:2], a[:, 1::2], b[:, 1::2])
    a_odd, b_odd = _odd_even_scan(a_red, b_red)
    if T % 2 == 0:
        a_e, b_e = _binary_op(a_odd[:, :-1], b_odd[:, :-1], a[:, 2::2], b[:, 2::2])
    else:
        a_e, b_e = _binary_op(a_odd, b_odd, a[:, 2::2], b[:, 2::2])
    a_e = torch.cat([a[:, :1], a_e], dim=1)
    b_e = torch.cat([b[:, :1], b_e], dim=1)
    # interleave even/odd prefixes
    out_a = torch.empty_like(a)
    out_b = torch.empty_like(b)
    out_a[:, 0::2] = a_e
    out_a[:, 1::2] = a_odd
    out_b[:, 0::2] = b_e
    out_b[:, 1::2] = b_odd
    return out_a, out_b


def scalar_assoc_scan(gates: Tensor, inputs: Tensor, prev: Tensor | None = None,
                      remove_prev: bool | None = None) -> Tensor:
    """Vectorised (log-depth) AssocScan restatement; differentiable through autograd."""
    g = _expand_gates(gates, inputs).expand_as(inputs)
    x = inputs
    if prev is not None:
        x = torch.cat([(g[:, :1] * prev.unsqueeze(1) + x[:, :1]), x[:, 1:]], dim=1)
    _, out = _odd_even_scan(g, x)
    if remove_prev is None:
        remove_prev = prev is not None
    if prev is not None and not remove_prev:
        out = torch.cat([prev.unsqueeze(1), out], dim=1)
    return out


# -----------------------------------------------------------------------------
# Window sum: rnn_memory.py:50-61 (`_sliding_sum_along_time`), omega.py:24-33.
# -----------------------------------------------------------------------------

def sliding_sum_along_time(x: Tensor, window: int) -> Tensor:
    """Inclusive window sum along dim 1: y_t = sum_{k=max(0,t-w+1)}^{t} x_k (cumsum difference)."""
    if window <= 1:
        return x
    T = x.shape[1]
    window = min(window, T)
    c = x.cumsum(dim=1)
    shifted = torch.cat([c.new_zeros((c.shape[0], window, *c.shape[2:])), c[:, :-window]], dim=1)
    return c - shifted


# -----------------------------------------------------------------------------
# Feature maps: rnn_memory.py:90-132 (`PolynomialFeatureMap`), omega.py:90-118.
# -----------------------------------------------------------------------------

def poly_feature_map(x: Tensor, degree: int = 1, mode: str = 'off', proj: Tensor | None = None) -> Tensor:
    if degree <= 1 or mode == 'off':
        return x
    if mode == 'elementwise':          # rnn_memory.py:117-123: sum_{i=1}^{g} x^i
        out = x.clone()
        power = x
        for _ in range(2, degree + 1):
            power = power * x
            out = out + power
        return out
    if mode == 'tensor':               # rnn_memory.py:125-130: [x; vec(x x^T)] @ P
        assert proj is not None, "tensor map needs the projection buffer (state_dict 'phi.proj')"
        d = x.shape[-1]
        outer = torch.einsum('...i,...j->...ij', x, x).reshape(*x.shape[:-1], d * d)
        feats = torch.cat([x, outer], dim=-1)
        return feats @ proj.to(x.dtype)
    return x


# -----------------------------------------------------------------------------
# Gate weights per (target t, lag j).
# -----------------------------------------------------------------------------

def lag_weights(gate: Tensor | None, BH: int, T: int, window: int, dtype, device) -> tuple[Tensor, Tensor]:
    """Returns (w, c): w[bh, t, j] weights real sources p = t - j >= 0, c[bh, t, j] weights
    buffer sources p = t - j < 0."""
    e = window
    if gate is None:
        w = torch.ones(BH, T, e, dtype=dtype, device=device)
        return w, w.clone()
    if gate.ndim == 2:                 # token gate, applied to the source product (rnn_memory.py:666-668)
        w = torch.ones(BH, T, e, dtype=gate.dtype, device=gate.device)
        for j in range(e):
            if j < T:
                w[:, j:, j] = gate[:, :T - j]
        c = torch.ones_like(w)         # the buffer already holds gated products
        return w, c
    assert gate.ndim == 3 and gate.shape[-1] == e
    return gate, gate


# -----------------------------------------------------------------------------
# Form 1: per-token loop (the textbook recurrence).
# -----------------------------------------------------------------------------

def memory_recurrence_loop(phi_k: Tensor, phi_q: Tensor, v: Tensor, lr: Tensor, decay: Tensor,
                           beta: Tensor | None, gate: Tensor | None, S_ref: Tensor, S0: Tensor,
                           Z0: Tensor | None, buf: Tensor | None, window: int = 1,
                           clamp_every: int | None = None, clamp_final: bool = True):
    """Returns (y [BH,T,dv], S_T [BH,dv,dk], Z_T or None, buffer_out [BH,e-1,dv,dk] or None)."""
    BH, T, dk = phi_k.shape
    dv = v.shape[-1]
    e = window
    momentum = beta is not None
    w, c = lag_weights(gate, BH, T, e, phi_k.dtype, phi_k.device)
    S = S0
    Z = Z0 if Z0 is not None else torch.zeros_like(S0)
    if buf is None and e > 1:
        buf = torch.zeros(BH, e - 1, dv, dk, dtype=S0.dtype, device=S0.device)
    ys, P = [], []
    for t in range(T):
        ys.append(torch.einsum('bde,be->bd', S, phi_q[:, t]))
        delta = torch.einsum('bde,be->bd', S_ref, phi_k[:, t]) - v[:, t]
        P.append(torch.einsum('bi,bj->bij', delta, phi_k[:, t]))
        g = torch.zeros_like(S)
        for j in range(e):
            p = t - j
            if p >= 0:
                g = g + w[:, t, j, None, None] * P[p]
            else:
                g = g + c[:, t, j, None, None] * buf[:, p + e - 1]
        if momentum:
            Z = beta[:, t, None, None] * Z + g
            S = decay[:, t, None, None] * S - lr[:, t, None, None] * Z
        else:
            S = decay[:, t, None, None] * S - lr[:, t, None, None] * g
        boundary = clamp_every is not None and T > clamp_every and (t + 1) % clamp_every == 0 and t < T - 1
        if boundary or (t == T - 1 and clamp_final):
            S = S.clamp(-100, 100)
    y = torch.stack(ys, dim=1) if T > 0 else v.new_zeros(BH, 0, dv)
    buf_out = None
    if e > 1:
        if gate is not None and gate.ndim == 2:
            Gp = [gate[:, p, None, None] * P[p] for p in range(T)]
        else:
            Gp = P
        ext = [buf[:, i] for i in range(e - 1)] + Gp
        buf_out = torch.stack(ext[-(e - 1):], dim=1)
    return y, S, (Z if momentum else None), buf_out


# -----------------------------------------------------------------------------
# Form 2: vectorised mirror of the reference op sequence (rnn_memory.py:605-730).
# -----------------------------------------------------------------------------

def _vectorised_impl(phi_k, phi_q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf, e, scan):
    BH, T, dk = phi_k.shape
    dv = v.shape[-1]
    pred = torch.einsum('bde,bte->btd', S_ref, phi_k)            # rnn_memory.py:659
    delta_vec = pred - v                                          # :660
    g_raw = torch.einsum('bti,btj->btij', delta_vec, phi_k)       # :663
    lag_mode = gate is not None and gate.ndim == 3
    if gate is not None and not lag_mode:
        g_raw = g_raw * gate[..., None, None]                     # :666-668
    new_buf = None
    if e > 1:
        prev_g = buf if buf is not None else g_raw.new_zeros((BH, e - 1, dv, dk))
        g_ext = torch.cat([prev_g, g_raw], dim=1)                 # :680
        if lag_mode:
            g = sum(gate[:, :, j, None, None] * g_ext[:, e - 1 - j: e - 1 - j + T] for j in range(e))
        else:
            g = sliding_sum_along_time(g_ext, e)[:, -T:]          # :681
        new_buf = g_ext[:, -(e - 1):]                             # :684
    else:
        g = g_raw if not lag_mode else gate[:, :, 0, None, None] * g_raw
    Z0 = Z0 if Z0 is not None else torch.zeros_like(S0)
    lr_e = lr[..., None, None]
    if beta is not None:
        Z_all = scan(beta, g, prev=Z0)                            # :698
        S_all = scan(decay, -lr_e * Z_all, prev=S0)               # :699-700
        S_end = S_all[:, -1].clamp(-100, 100)                     # :701
        Z_end = Z_all[:, -1]
    else:
        S_all = scan(decay, -lr_e * g, prev=S0)                   # :704-705
        S_end = S_all[:, -1].clamp(-100, 100)
        Z_end = None
    y0 = torch.einsum('bde,be->bd', S0, phi_q[:, 0])              # :712
    if T > 1:
        y_rest = torch.einsum('btdp,btp->btd', S_all[:, :-1], phi_q[:, 1:])
        y = torch.cat([y0.unsqueeze(1), y_rest], dim=1)
    else:
        y = y0.unsqueeze(1)
    return y, S_end, Z_end, new_buf, S_all[:, -1], (Z_all[:, -1] if beta is not None else None)


def memory_recurrence_vectorised(phi_k: Tensor, phi_q: Tensor, v: Tensor, lr: Tensor, decay: Tensor,
                                 beta: Tensor | None, gate: Tensor | None, S_ref: Tensor, S0: Tensor,
                                 Z0: Tensor | None, buf: Tensor | None, window: int = 1,
                                 clamp_every: int | None = None, clamp_final: bool = True,
                                 scan=scalar_assoc_scan):
    """Same contract as `memory_recurrence_loop`, built from the reference's tensor ops:
    einsum delta -> gated outer product -> cumsum window -> scalar scans -> shifted retrieval.
    The `scan_chunk_len` loop follows rnn_memory.py:584-601 (S_ref fixed, state carried)."""
    T = phi_k.shape[1]
    e = window
    if clamp_every is not None and T > clamp_every:
        ys = []
        S, Z, b = S0, Z0, buf
        for start in range(0, T, clamp_every):
            end = min(T, start + clamp_every)
            sl = slice(start, end)
            y, S_end, Z_end, b, S_raw, _ = _vectorised_impl(
                phi_k[:, sl], phi_q[:, sl], v[:, sl], lr[:, sl], decay[:, sl],
                beta[:, sl] if beta is not None else None,
                gate[:, sl] if gate is not None else None,
                S_ref, S, Z, b, e, scan)
            ys.append(y)
            S = S_end if (end < T or clamp_final) else S_raw
            Z = Z_end
        return torch.cat(ys, dim=1), S, Z, b
    y, S_end, Z_end, b, S_raw, _ = _vectorised_impl(phi_k, phi_q, v, lr, decay, beta, gate, S_ref, S0,
                                                    Z0, buf, e, scan)
    return y, (S_end if clamp_final else S_raw), Z_end, b


# -----------------------------------------------------------------------------
# Matrix-affine scan: affine_scan.py:7-158.  H_t = H_{t-1} @ A_t + B_t.
# -----------------------------------------------------------------------------

def affine_scan_sequential(A: Tensor, B: Tensor, prev: Tensor | None = None, remove_prev: bool = False) -> Tensor:
    N, T, D, _ = A.shape
    R = B.shape[2]
    H = prev if prev is not None else A.new_zeros(N, R, D)
    outs = []
    for t in range(T):
        H = H @ A[:, t] + B[:, t]
        outs.append(H)
    out = torch.stack(outs, dim=1)
    if prev is not None and not remove_prev:
        out = torch.cat([prev[:, None], out], dim=1)
    return out


def affine_associative_scan(A: Tensor, B: Tensor, prev: Tensor | None = None, remove_prev: bool = False) -> Tensor:
    """Odd/even recursion over right-affine transforms (affine_scan.py:36-158), then
    H_t = H_0 A_pref[t] + B_pref[t] (affine_scan.py:148-150)."""
    N, T, D, _ = A.shape
    R = B.shape[2]

    def compose(l, r):                 # affine_scan.py:7-33
        return l[0] @ r[0], l[1] @ r[0] + r[1]

    def scan(Ae, Be):
        t = Ae.shape[1]
        if t < 2:
            return Ae, Be
        A_red, B_red = compose((Ae[:, :-1:2], Be[:, :-1:2]), (Ae[:, 1::2], Be[:, 1::2]))
        A_odd, B_odd = scan(A_red, B_red)
        if t % 2 == 0:
            A_ev, B_ev = compose((A_odd[:, :-1], B_odd[:, :-1]), (Ae[:, 2::2], Be[:, 2::2]))
        else:
            A_ev, B_ev = compose((A_odd, B_odd), (Ae[:, 2::2], Be[:, 2::2]))
        A_ev = torch.cat([Ae[:, :1], A_ev], dim=1)
        B_ev = torch.cat([Be[:, :1], B_ev], dim=1)
        A_out = torch.empty_like(Ae)
        B_out = torch.empty_like(Be)
        A_out[:, 0::2], A_out[:, 1::2] = A_ev, A_odd
        B_out[:, 0::2], B_out[:, 1::2] = B_ev, B_odd
        return A_out, B_out

    A_pref, B_pref = scan(A, B)
    H0 = prev if prev is not None else A.new_zeros(N, R, D)
    H = torch.einsum('nrd,ntde->ntre', H0, A_pref) + B_pref
    if prev is not None and not remove_prev:
        H = torch.cat([prev[:, None], H], dim=1)
    if prev is not None and remove_prev:
        H = H[:, :T]
    return H
