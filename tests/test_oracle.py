"""Pins the CPU oracle (oracle/recurrence.py) before it is trusted as the parity checker.

Every check here is independent of the oracle's own formulas: golden vectors from the
reference's tests, closed forms, brute-force finite differences, or agreement between two
independently written forms. A planted mistake (dropped term, wrong sign or index,
transposed operand) in either form fails at least one of these.
"""

import json
import os

import pytest
import torch

from oracle import (
    scalar_assoc_scan,
    scalar_assoc_scan_sequential,
    sliding_sum_along_time,
    poly_feature_map,
    memory_recurrence_loop,
    memory_recurrence_vectorised,
    affine_associative_scan,
    affine_scan_sequential,
)

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
D64 = torch.float64


def rand_problem(BH=3, T=9, dk=5, dv=4, e=3, gate="token", momentum=True, buf=True, seed=0,
                 state_scale=0.3, dtype=D64):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    p = dict(
        phi_k=r(BH, T, dk), phi_q=r(BH, T, dk), v=r(BH, T, dv),
        lr=0.5 * torch.sigmoid(r(BH, T)), decay=torch.sigmoid(r(BH, T) + 2),
        beta=torch.sigmoid(r(BH, T) + 1) if momentum else None,
        gate=None, S_ref=state_scale * r(BH, dv, dk), S0=state_scale * r(BH, dv, dk),
        Z0=state_scale * r(BH, dv, dk) if momentum else None,
        buf=state_scale * r(BH, e - 1, dv, dk) if (buf and e > 1) else None, window=e)
    if gate == "token":
        p["gate"] = torch.sigmoid(r(BH, T))
    elif gate == "lag":
        p["gate"] = torch.softmax(r(BH, T, e), dim=-1)
    return p


def assert_outs_close(a, b, rtol=1e-10, atol=1e-10):
    for x, y in zip(a, b):
        if x is None or y is None:
            assert x is None and y is None
            continue
        torch.testing.assert_close(x, y, rtol=rtol, atol=atol)


# ----------------------------------------------------------------------------- golden vectors

def test_sliding_sum_golden_1d():
    gv = GOLDEN["sliding_sum_1_to_6_w3"]
    x = torch.tensor(gv["x"], dtype=D64).view(1, -1, 1)
    out = sliding_sum_along_time(x, gv["window"])
    assert out.view(-1).tolist() == gv["expected"]


@pytest.mark.parametrize("w", ["1", "2", "3"])
def test_sliding_sum_golden_2x4x2(w):
    gv = GOLDEN["sliding_sum_2x4x2"]
    x = torch.tensor(gv["x"], dtype=D64)
    out = sliding_sum_along_time(x, int(w))
    assert out.tolist() == gv["expected"][w]


@pytest.mark.parametrize("scan", [scalar_assoc_scan, scalar_assoc_scan_sequential])
@pytest.mark.parametrize("name", ["assoc_scan_mixed", "assoc_scan_decay", "assoc_scan_additive"])
def test_assoc_scan_golden(scan, name):
    gv = GOLDEN[name]
    N, T, D1, D2 = gv["shape"]
    gates = torch.full((N, T), gv["gate"], dtype=D64)
    inputs = torch.full((N, T, D1, D2), gv["input"], dtype=D64)
    prev = torch.full((N, D1, D2), gv["prev"], dtype=D64)
    out = scan(gates, inputs, prev=prev)
    assert out.shape == inputs.shape
    for t, ex in enumerate(gv["expected_per_step"]):
        assert torch.allclose(out[:, t], torch.full_like(out[:, t], ex))


@pytest.mark.parametrize("scan", [scalar_assoc_scan, scalar_assoc_scan_sequential])
def test_assoc_scan_identity_and_chaining(scan):
    # tests/test_rnn_all.py:832-837 (identity) and tests/test_titans.py:681-711 (chaining with prev)
    g = torch.Generator().manual_seed(1)
    x0 = torch.randn(2, 4, 4, generator=g, dtype=D64)
    out = scan(torch.ones(2, 5, dtype=D64), torch.zeros(2, 5, 4, 4, dtype=D64), prev=x0)
    for t in range(5):
        assert torch.allclose(out[:, t], x0)
    gates = torch.sigmoid(torch.randn(2, 128, 16, generator=g, dtype=D64))
    inputs = torch.randn(2, 128, 16, generator=g, dtype=D64)
    full = scan(gates, inputs)
    first = scan(gates[:, :64], inputs[:, :64])
    second = scan(gates[:, 64:], inputs[:, 64:], prev=first[:, -1])
    assert second.shape == inputs[:, 64:].shape
    assert torch.allclose(full[:, -1], second[:, -1], atol=1e-12)


def test_assoc_scan_remove_prev_false_prepends_prev():
    # omega.py:315 uses remove_prev=False: T+1 outputs, the first one is prev
    g = torch.Generator().manual_seed(2)
    gates = torch.rand(3, 7, 1, generator=g, dtype=D64)
    inputs = torch.randn(3, 7, 5, generator=g, dtype=D64)
    prev = torch.randn(3, 5, generator=g, dtype=D64)
    for scan in (scalar_assoc_scan, scalar_assoc_scan_sequential):
        out = scan(gates, inputs, prev=prev, remove_prev=False)
        assert out.shape == (3, 8, 5)
        assert torch.equal(out[:, 0], prev)
        assert torch.allclose(out[:, 1:], scan(gates, inputs, prev=prev), atol=1e-12)


def test_assoc_scan_forms_agree_odd_lengths():
    g = torch.Generator().manual_seed(3)
    for T in (1, 2, 3, 5, 8, 13, 31):
        gates = torch.rand(2, T, generator=g, dtype=D64)
        inputs = torch.randn(2, T, 3, 2, generator=g, dtype=D64)
        prev = torch.randn(2, 3, 2, generator=g, dtype=D64)
        assert torch.allclose(scalar_assoc_scan(gates, inputs, prev=prev),
                              scalar_assoc_scan_sequential(gates, inputs, prev=prev), atol=1e-12)


def test_window_then_unit_scan_differences_equal_window_sums():
    # tests/test_atlas.py:217-309: with unit decay gate, diff(updates) == sliding_sum(surprises)
    surprises = -torch.arange(1, 5, dtype=D64).view(1, 4, 1)
    u = sliding_sum_along_time(surprises, 3)
    y = scalar_assoc_scan(torch.ones(1, 4, dtype=D64), u)
    assert torch.allclose(y[:, 1:] - y[:, :-1], u[:, 1:])
    assert u.view(-1).tolist() == [-1.0, -3.0, -6.0, -9.0]


# ----------------------------------------------------------------------------- feature maps

def test_poly_elementwise_closed_form():
    x = torch.linspace(-2, 2, 11, dtype=D64).view(1, 11)
    assert torch.allclose(poly_feature_map(x, 3, 'elementwise'), x + x ** 2 + x ** 3)
    assert torch.equal(poly_feature_map(x, 1, 'elementwise'), x)
    assert torch.equal(poly_feature_map(x, 3, 'off'), x)


def test_poly_tensor_matches_kronecker():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 3, generator=g, dtype=D64)
    P = torch.randn(3 + 9, 3, generator=g, dtype=D64)
    feats = torch.stack([torch.cat([xi, torch.kron(xi, xi)]) for xi in x])
    assert torch.allclose(poly_feature_map(x, 2, 'tensor', P), feats @ P)


# ----------------------------------------------------------------------------- recurrence closed forms

def test_gated_linear_attention_closed_form():
    """S_ref=0, S0=0, e=1, no momentum: y_t = sum_{s<t} (prod_{r=s+1}^{t-1} a_r) eta_s v_s (phi_s . psi_t)."""
    p = rand_problem(BH=2, T=7, dk=4, dv=3, e=1, gate=None, momentum=False, buf=False, seed=5)
    p["S_ref"].zero_()
    p["S0"].zero_()
    y, S_T, _, _ = memory_recurrence_loop(**p)
    y2, _, _, _ = memory_recurrence_vectorised(**p)
    phi, psi, v, a, eta = p["phi_k"], p["phi_q"], p["v"], p["decay"], p["lr"]
    ref = torch.zeros_like(y)
    for t in range(7):
        for s in range(t):
            coef = eta[:, s] * torch.prod(a[:, s + 1:t], dim=1)
            ref[:, t] += coef[:, None] * v[:, s] * (phi[:, s] * psi[:, t]).sum(-1, keepdim=True)
    assert torch.allclose(y, ref, atol=1e-12)
    assert torch.allclose(y2, ref, atol=1e-12)


def test_cumulative_linear_attention_alpha_one():
    p = rand_problem(BH=2, T=6, dk=4, dv=3, e=1, gate=None, momentum=False, buf=False, seed=6)
    p["S_ref"].zero_()
    p["S0"].zero_()
    p["decay"].fill_(1.0)
    p["lr"].fill_(0.25)
    y, S_T, _, _ = memory_recurrence_loop(**p)
    scores = torch.einsum('btk,bsk->bts', p["phi_q"], p["phi_k"])
    mask = torch.tril(torch.ones(6, 6, dtype=D64), diagonal=-1)
    ref = 0.25 * torch.einsum('bts,bsd->btd', scores * mask, p["v"])
    assert torch.allclose(y, ref, atol=1e-12)
    assert torch.allclose(S_T, 0.25 * torch.einsum('btd,btk->bdk', p["v"], p["phi_k"]), atol=1e-12)


@pytest.mark.parametrize("form", [memory_recurrence_loop, memory_recurrence_vectorised])
def test_gate_zero_no_update(form):
    # tests/test_rnn_all.py:917-932: u ~ 0 suppresses the update
    p = rand_problem(e=3, gate="token", momentum=True, buf=False, seed=7)
    p["gate"].zero_()
    p["Z0"].zero_()
    y, S_T, Z_T, buf_out = form(**p)
    ref_S = torch.prod(p["decay"], dim=1)[:, None, None] * p["S0"]
    assert torch.allclose(S_T, ref_S, atol=1e-12)
    assert torch.count_nonzero(Z_T) == 0 and torch.count_nonzero(buf_out) == 0


@pytest.mark.parametrize("form", [memory_recurrence_loop, memory_recurrence_vectorised])
def test_beta_zero_equals_no_momentum(form):
    p = rand_problem(e=2, gate="token", momentum=True, buf=True, seed=8)
    p["beta"].zero_()
    a = form(**p)
    q = dict(p, beta=None, Z0=None)
    b = form(**q)
    assert torch.allclose(a[0], b[0], atol=1e-12)
    assert torch.allclose(a[1], b[1], atol=1e-12)


def test_omega_e1_equals_titans():
    p = rand_problem(e=1, gate="token", momentum=True, buf=False, seed=9)
    p["gate"].fill_(1.0)
    a = memory_recurrence_loop(**p)
    b = memory_recurrence_vectorised(**dict(p, gate=None))
    assert_outs_close(a, b)


def test_lag_gate_generalises_token_gate_without_buffer():
    p = rand_problem(e=3, gate="token", momentum=True, buf=False, seed=10)
    u = p["gate"]
    BH, T = u.shape
    w = torch.zeros(BH, T, 3, dtype=D64)
    for j in range(3):
        w[:, j:, j] = u[:, :T - j]
    a = memory_recurrence_loop(**p)
    b = memory_recurrence_vectorised(**dict(p, gate=w))
    torch.testing.assert_close(a[0], b[0], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(a[1], b[1], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(a[2], b[2], rtol=1e-10, atol=1e-10)


def _prechange_titans(p):
    """tests/test_rnn_all.py:43-140: the pre-change G/B form, g = S0 G - B (valid with S_ref = S0)."""
    phi, psi, v = p["phi_k"], p["phi_q"], p["v"]
    G = torch.einsum('bti,btj->btij', phi, phi)
    B = torch.einsum('bti,btj->btij', v, phi)
    g = torch.einsum('bde,btef->btdf', p["S0"], G) - B
    Z_all = scalar_assoc_scan_sequential(p["beta"], g, prev=p["Z0"])
    S_all = scalar_assoc_scan_sequential(p["decay"], -p["lr"][..., None, None] * Z_all, prev=p["S0"])
    S_start = torch.cat([p["S0"].unsqueeze(1), S_all[:, :-1]], dim=1)
    y = torch.einsum('btdp,btp->btd', S_start, psi)
    return y, S_all[:, -1].clamp(-100, 100), Z_all[:, -1]


def test_delta_phi_identity_matches_prechange_G_B_form():
    p = rand_problem(e=1, gate=None, momentum=True, buf=False, seed=11)
    p["S_ref"] = p["S0"].clone()
    a = memory_recurrence_loop(**p)
    b = _prechange_titans(p)
    for x, y in zip(a[:3], b):
        torch.testing.assert_close(x, y, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("gate", [None, "token", "lag"])
@pytest.mark.parametrize("momentum", [False, True])
@pytest.mark.parametrize("e,T", [(1, 1), (1, 9), (2, 1), (3, 2), (3, 9), (4, 13), (5, 3)])
@pytest.mark.parametrize("buf", [False, True])
def test_loop_and_vectorised_forms_agree(gate, momentum, e, T, buf):
    p = rand_problem(T=T, e=e, gate=gate, momentum=momentum, buf=buf, seed=100 + e * 10 + T)
    assert_outs_close(memory_recurrence_loop(**p), memory_recurrence_vectorised(**p))


@pytest.mark.parametrize("gate", [None, "token", "lag"])
def test_clamp_every_chunk_loop_agrees(gate):
    """rnn_memory.py:584-601 chunk loop == per-token loop with clamps at chunk ends,
    including a case where the clamp is active."""
    for scale, seed in ((0.3, 12), (400.0, 13)):
        p = rand_problem(T=13, e=3, gate=gate, momentum=True, buf=True, seed=seed, state_scale=scale)
        a = memory_recurrence_loop(**p, clamp_every=4)
        b = memory_recurrence_vectorised(**p, clamp_every=4)
        assert_outs_close(a, b)
        if scale > 100:
            c = memory_recurrence_loop(**p)
            assert not torch.allclose(a[0], c[0])


def test_chunk_invariance_when_clamp_inactive():
    # tests/test_rnn_all.py:335-374
    p = rand_problem(T=13, e=3, gate="token", momentum=True, buf=True, seed=14)
    a = memory_recurrence_vectorised(**p)
    b = memory_recurrence_vectorised(**p, clamp_every=4)
    assert_outs_close(a, b)


def test_loop_gradcheck():
    """Brute-force finite differences pin the autograd backward of the loop form, which the
    GPU backward is compared against."""
    p = rand_problem(BH=1, T=5, dk=3, dv=2, e=3, gate="lag", momentum=True, buf=True, seed=15)
    names = ["phi_k", "phi_q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buf"]
    inputs = tuple(p[n].clone().requires_grad_(True) for n in names)

    def fn(*args):
        kw = dict(zip(names, args))
        y, S, Z, b = memory_recurrence_loop(**kw, window=3)
        return y, S, Z, b

    assert torch.autograd.gradcheck(fn, inputs, eps=1e-6, atol=1e-7)


def test_affine_scan_forms_agree_and_reduce_to_scalar_scan():
    g = torch.Generator().manual_seed(16)
    N, T, D, R = 2, 11, 4, 3
    A = 0.5 * torch.randn(N, T, D, D, generator=g, dtype=D64)
    B = torch.randn(N, T, R, D, generator=g, dtype=D64)
    prev = torch.randn(N, R, D, generator=g, dtype=D64)
    for rp in (False, True):
        torch.testing.assert_close(affine_associative_scan(A, B, prev=prev, remove_prev=rp),
                                   affine_scan_sequential(A, B, prev=prev, remove_prev=rp))
    torch.testing.assert_close(affine_associative_scan(A, B), affine_scan_sequential(A, B))
    alpha = torch.rand(N, T, generator=g, dtype=D64)
    A_diag = alpha[..., None, None] * torch.eye(D, dtype=D64)
    torch.testing.assert_close(affine_associative_scan(A_diag, B, prev=prev, remove_prev=True),
                               scalar_assoc_scan_sequential(alpha, B, prev=prev))
