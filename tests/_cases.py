"""Seeded problem generation and the two sides of a parity check (test helper).

Inputs follow BASELINE.json's distributions: q, k, v ~ N(0, 1) with keys L2-normalised per
token, alpha = sigmoid(N(2, 0.5)), eta = 0.1 * sigmoid(N(0, 1)), beta = sigmoid(N(1, 0.5)),
per-lag gates softmax(N(0, 1)) over the window, per-token gates sigmoid(N(0, 1)).
Inputs are drawn in fp32 on the CPU, rounded to the test dtype, and the oracle runs in fp64
on exactly those rounded values.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from oracle import memory_recurrence_vectorised, poly_feature_map

F64 = torch.float64


@dataclass
class Case:
    name: str
    BH: int
    T: int
    d: int                           # d_k
    e: int = 1
    gate: str | None = None          # None | 'token' | 'lag'
    momentum: bool = True
    buffer: bool = False
    states: float = 0.0              # scale of random S_ref / S0 / Z0 (0 -> zeros)
    map_degree: int = 1
    clamp_every: int | None = None
    clamp_final: bool = True
    dtype: torch.dtype = torch.float32
    seed: int = 0
    decay_shift: float = 2.0
    beta_shift: float = 1.0          # momentum decay beta = sigmoid(N(0, 1) / 2 + beta_shift)
    backward: bool = True
    dv: int | None = None            # d_v (None: d_v = d_k)
    grad_buffer: bool = True         # the loss includes buffer_out (False: no buffer_out gradient)
    buffer_scale: float = 0.1        # carried buffer ~ buffer_scale * N(0, 1) (0: a zero buffer, as the cells pass)
    extra: dict = field(default_factory=dict)


def make_inputs(c: Case) -> dict:
    g = torch.Generator().manual_seed(1000 + c.seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)
    BH, T, d, e = c.BH, c.T, c.d, c.e
    dv = c.dv or d
    k = r(BH, T, d)
    k = k / k.norm(dim=-1, keepdim=True)
    p = dict(k=k, q=r(BH, T, d), v=r(BH, T, dv),
             decay=torch.sigmoid(r(BH, T) * 0.5 + c.decay_shift), lr=0.1 * torch.sigmoid(r(BH, T)))
    p["beta"] = torch.sigmoid(r(BH, T) * 0.5 + c.beta_shift) if c.momentum else None
    if c.gate == 'token':
        p["gate"] = torch.sigmoid(r(BH, T))
    elif c.gate == 'lag':
        p["gate"] = torch.softmax(r(BH, T, e), dim=-1)
    else:
        p["gate"] = None
    s = c.states
    z = lambda: torch.zeros(BH, dv, d)
    p["S_ref"] = s * r(BH, dv, d) if s else z()
    p["S0"] = s * r(BH, dv, d) if s else z()
    p["Z0"] = (s * r(BH, dv, d) if s else z()) if c.momentum else None
    p["buffer"] = (c.buffer_scale * r(BH, e - 1, dv, d)) if (c.buffer and e > 1) else None
    # upstream gradients
    p["gy"] = r(BH, T, dv)
    p["gS"] = r(BH, dv, d)
    p["gZ"] = r(BH, dv, d) if c.momentum else None
    p["gB"] = r(BH, e - 1, dv, d) if e > 1 else None
    if not c.grad_buffer:
        p["gB"] = None
    # round the dtype-carried tensors
    for key in ("k", "q", "v", "decay", "lr", "beta", "gate", "gy"):
        if p[key] is not None:
            p[key] = p[key].to(c.dtype).to(torch.float32)
    return p


TENSOR_INPUTS = ("k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buffer")


def _loss(out, p):
    y, S_T, Z_T, B = out
    loss = (y * p["gy"]).sum() + (S_T * p["gS"]).sum()
    if Z_T is not None:
        loss = loss + (Z_T * p["gZ"]).sum()
    if B is not None and p["gB"] is not None:
        loss = loss + (B * p["gB"]).sum()
    return loss


def run_oracle(c: Case, p: dict):
    """fp64 oracle outputs and gradients (autograd through the vectorised restatement)."""
    x = {kk: (p[kk].to(F64).clone().requires_grad_(c.backward) if p[kk] is not None else None)
         for kk in TENSOR_INPUTS}
    # S_ref and S0 are separate leaves here (the cell passes the same tensor for both)
    phi_k = poly_feature_map(x["k"], c.map_degree, 'elementwise' if c.map_degree > 1 else 'off')
    phi_q = poly_feature_map(x["q"], c.map_degree, 'elementwise' if c.map_degree > 1 else 'off')
    out = memory_recurrence_vectorised(phi_k, phi_q, x["v"], x["lr"], x["decay"], x["beta"], x["gate"],
                                       x["S_ref"], x["S0"], x["Z0"], x["buffer"], window=c.e,
                                       clamp_every=c.clamp_every, clamp_final=c.clamp_final)
    grads = {}
    if c.backward:
        q64 = {kk: (v.to(F64) if v is not None else None) for kk, v in p.items() if kk.startswith("g")}
        loss = _loss(out, q64)
        leaves = [kk for kk in TENSOR_INPUTS if x[kk] is not None]
        gs = torch.autograd.grad(loss, [x[kk] for kk in leaves], allow_unused=True)
        grads = {kk: (gg if gg is not None else torch.zeros_like(x[kk])) for kk, gg in zip(leaves, gs)}
    return [o.detach() if o is not None else None for o in out], grads


def run_gpu(c: Case, p: dict, device="cuda"):
    from atlas_rnn_amd.functional import memory_recurrence
    x = {}
    for kk in TENSOR_INPUTS:
        if p[kk] is None:
            x[kk] = None
            continue
        dt = c.dtype if kk in ("k", "q", "v", "lr", "decay", "beta", "gate") else torch.float32
        x[kk] = p[kk].to(device=device, dtype=dt).clone().requires_grad_(c.backward)
    out = memory_recurrence(x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"],
                            x["S_ref"], x["S0"], x["Z0"], x["buffer"], window=c.e,
                            map_mode='elementwise' if c.map_degree > 1 else 'off', map_degree=c.map_degree,
                            clamp_every=c.clamp_every, clamp_final=c.clamp_final)
    grads = {}
    if c.backward:
        gd = {kk: (v.to(device) if v is not None else None) for kk, v in p.items() if kk.startswith("g")}
        gd["gy"] = gd["gy"].to(c.dtype)
        loss = _loss([o.float() if o is not None else None for o in out], gd)
        leaves = [kk for kk in TENSOR_INPUTS if x[kk] is not None]
        gs = torch.autograd.grad(loss, [x[kk] for kk in leaves], allow_unused=True)
        grads = {kk: (gg if gg is not None else torch.zeros_like(x[kk])) for kk, gg in zip(leaves, gs)}
    torch.cuda.synchronize()
    return ([o.detach().float().cpu() if o is not None else None for o in out],
            {kk: v.float().cpu() for kk, v in grads.items()})


def run_oracle_rows(c: Case, p: dict, rows, block: int = 256):
    """fp64 oracle outputs and gradients for the head-batch rows `rows` only (rows are independent,
    so these equal the same rows of the full problem's). The sequence runs in blocks of `block`
    tokens carrying (S, Z, buffer), unclamped until the last block: the same recurrence as one call
    (the oracle's chunk invariance), with a fraction of the memory at long T. With clamp_every, the
    block length must be a multiple of it (every block end is then a clamp point)."""
    assert c.clamp_every is None or block % c.clamp_every == 0
    idx = torch.tensor(list(rows))
    sub = {kk: (v[idx] if v is not None else None) for kk, v in p.items()}
    x = {kk: (sub[kk].to(F64).clone().requires_grad_(c.backward) if sub[kk] is not None else None)
         for kk in TENSOR_INPUTS}
    mode = 'elementwise' if c.map_degree > 1 else 'off'
    phi_k = poly_feature_map(x["k"], c.map_degree, mode)
    phi_q = poly_feature_map(x["q"], c.map_degree, mode)
    ys, S, Z, B = [], x["S0"], x["Z0"], x["buffer"]
    for s0 in range(0, c.T, block):
        sl = slice(s0, min(c.T, s0 + block))
        sl_or_none = lambda t: t[:, sl] if t is not None else None
        last = s0 + block >= c.T
        y, S, Z, B = memory_recurrence_vectorised(
            phi_k[:, sl], phi_q[:, sl], x["v"][:, sl], x["lr"][:, sl], x["decay"][:, sl], sl_or_none(x["beta"]),
            sl_or_none(x["gate"]), x["S_ref"], S, Z, B, window=c.e, clamp_every=c.clamp_every,
            clamp_final=c.clamp_final if last else c.clamp_every is not None)
        ys.append(y)
    out = [torch.cat(ys, dim=1), S, Z, B]
    grads = {}
    if c.backward:
        q64 = {kk: (v.to(F64) if v is not None else None) for kk, v in sub.items() if kk.startswith("g")}
        loss = _loss(out, q64)
        leaves = [kk for kk in TENSOR_INPUTS if x[kk] is not None]
        gs = torch.autograd.grad(loss, [x[kk] for kk in leaves], allow_unused=True)
        grads = {kk: (gg if gg is not None else torch.zeros_like(x[kk])) for kk, gg in zip(leaves, gs)}
    return [o.detach() if o is not None else None for o in out], grads


def tol_for(c: Case) -> float:
    return 1e-4 if c.dtype == torch.float32 else 2e-2


# (name, normwise relative error, tol) of every compare() call in this process: the margin report
NORMWISE: list[tuple[str, float, float]] = []


def normwise_error(got: torch.Tensor, ref: torch.Tensor) -> float:
    """||got - ref||_F / ||ref||_F in fp64 (0 when both are zero)."""
    ref = ref.to(torch.float64)
    got = got.to(torch.float64)
    den = ref.norm().item()
    num = (got - ref).norm().item()
    return num / den if den > 0 else (0.0 if num == 0 else float("inf"))


def compare(name: str, got: torch.Tensor, ref: torch.Tensor, tol: float, normwise: bool = True):
    """Two checks: the normwise relative error ||got - ref|| / ||ref|| <= tol (normwise=True), and
    elementwise |got - ref| <= tol * |ref| + tol * max|ref| (rtol with an atol floor scaled by the
    tensor's largest magnitude). The normwise error is recorded in NORMWISE."""
    ref = ref.to(torch.float64)
    got = got.to(torch.float64)
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    nw = normwise_error(got, ref)
    NORMWISE.append((name, nw, tol))
    if normwise:
        assert nw <= tol, f"{name}: normwise relative error {nw:.3e} > {tol}"
    scale = ref.abs().max().item()
    atol = tol * max(scale, 1e-30)
    err = (got - ref).abs()
    bad = err > (tol * ref.abs() + atol)
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {bad.numel()} elements off (tol {tol}); max err "
            f"{err.max().item():.3e} vs max|ref| {scale:.3e}; first at {idx}: got "
            f"{got[tuple(idx)].item():.6e} ref {ref[tuple(idx)].item():.6e}")
