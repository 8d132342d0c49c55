"""Pins of oracle/omega.py (the Omega section of OmegaNeuralMemory.store_memories, omega.py:262-318),
on the CPU in float64: the two forms agree; chunk invariance with the carried state; closed forms
of the decay scan, the momentum scan and the window; the gate short-circuit."""

import pytest
import torch

from oracle.omega import omega_store_chain, omega_store_chain_loop

F64 = torch.float64


def _inputs(BH=3, n=9, p=(4, 5), O=1, combine=False, gate=True, e=3, buf=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    x = dict(surprise=r(BH, n, *p), decay_factor=torch.sigmoid(r(BH, n)), last_update=r(BH, *p))
    if O:
        x["adaptive_momentum"] = torch.sigmoid(r(O, BH, n))
        x["last_momentum"] = r(O, BH, *p)
        if combine:
            x["combine_momentums"] = r(O, BH, n)
    if gate:
        x["omega_gate"] = torch.sigmoid(r(BH, n))
    x["omega_window"] = e
    if buf and e > 1:
        x["omega_buf"] = r(BH, e - 1, *p)
    return x


SETTINGS = [dict(), dict(O=0), dict(O=2), dict(O=2, combine=True), dict(gate=False), dict(e=1), dict(e=4, buf=False),
            dict(e=12, n=5), dict(p=()), dict(n=1, e=2)]


@pytest.mark.parametrize("kw", SETTINGS, ids=[str(s) for s in SETTINGS])
def test_forms_agree(kw):
    x = _inputs(**kw)
    a = omega_store_chain(**x)
    b = omega_store_chain_loop(**x)
    for u, v in zip(a, b):
        if u is None:
            assert v is None
            continue
        torch.testing.assert_close(u, v, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kw", [dict(), dict(O=2, combine=True), dict(e=5, n=12)])
def test_chunk_invariance(kw):
    """n chunks in one call == two calls carrying last_update, last_momentum and the omega buffer
    (the state past_state carries between store_memories calls)."""
    x = _inputs(**kw)
    n = x["surprise"].shape[1]
    full = omega_store_chain(**x)
    cut = n // 2
    per_t = ("surprise", "decay_factor", "omega_gate")
    first = dict(x)
    second = dict(x)
    for k in per_t:
        if k in x:
            first[k] = x[k][:, :cut]
            second[k] = x[k][:, cut:]
    for k in ("adaptive_momentum", "combine_momentums"):
        if k in x:
            first[k] = x[k][:, :, :cut]
            second[k] = x[k][:, :, cut:]
    u1, lu1, lm1, b1 = omega_store_chain(**first)
    second["last_update"] = lu1
    if lm1 is not None:
        second["last_momentum"] = lm1
    if b1 is not None:
        second["omega_buf"] = b1
    u2, lu2, lm2, b2 = omega_store_chain(**second)
    torch.testing.assert_close(torch.cat([u1, u2[:, 1:]], dim=1), full[0], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lu2, full[1])
    if lm2 is not None:
        torch.testing.assert_close(lm2, full[2])
    if b2 is not None:
        torch.testing.assert_close(b2, full[3])


def test_decay_scan_closed_form():
    """Window 1, no momentum, no gate, constant decay d and surprise c:
    u_t = (1-d)^(t+1) u_0 + c (1 - (1-d)^(t+1)) / d."""
    BH, n, d, c, u0 = 2, 7, 0.3, 1.5, -0.7
    upd, last, _, _ = omega_store_chain(torch.full((BH, n, 3), c, dtype=F64), torch.full((BH, n), d, dtype=F64),
                                        torch.full((BH, 3), u0, dtype=F64))
    t = torch.arange(n + 1, dtype=F64)
    a = (1 - d) ** t
    want = a * u0 + c * (1 - a) / d
    assert upd.shape == (BH, n + 1, 3)
    torch.testing.assert_close(upd[0, :, 0], want)
    torch.testing.assert_close(last, torch.full((BH, 3), want[-1].item(), dtype=F64))


def test_momentum_closed_form():
    """One momentum order with constant gate b and surprise x, decay 1 (the update is the momentum
    itself): m_t = b^(t+1) m_{-1} + x (1 - b^(t+1)) / (1 - b)."""
    BH, n, b, x, m0 = 2, 6, 0.6, 2.0, 0.25
    upd, _, lm, _ = omega_store_chain(torch.full((BH, n), x, dtype=F64), torch.ones(BH, n, dtype=F64),
                                      torch.zeros(BH, dtype=F64),
                                      adaptive_momentum=torch.full((1, BH, n), b, dtype=F64),
                                      last_momentum=torch.full((1, BH), m0, dtype=F64))
    t = torch.arange(1, n + 1, dtype=F64)
    want = b ** t * m0 + x * (1 - b ** t) / (1 - b)
    torch.testing.assert_close(upd[0, 1:], want)
    torch.testing.assert_close(lm[0, 0], want[-1])


def test_window_known_answer():
    """Window 3 over ones with a zero buffer and decay 1: the window sums 1, 2, 3, 3, ...; the next
    buffer is the last two chunks' gated surprises."""
    upd, _, _, buf = omega_store_chain(torch.ones(1, 6, dtype=F64), torch.ones(1, 6, dtype=F64),
                                       torch.zeros(1, dtype=F64), omega_window=3)
    assert upd[0].tolist() == [0.0, 1.0, 2.0, 3.0, 3.0, 3.0, 3.0]
    assert buf[0].tolist() == [1.0, 1.0]
    # a carried buffer enters the first e - 1 windows
    upd, _, _, _ = omega_store_chain(torch.ones(1, 3, dtype=F64), torch.ones(1, 3, dtype=F64),
                                     torch.zeros(1, dtype=F64), omega_window=3,
                                     omega_buf=torch.tensor([[10.0, 20.0]], dtype=F64))
    assert upd[0].tolist() == [0.0, 31.0, 22.0, 3.0]


def test_gate_short_circuit():
    x = _inputs(BH=3, n=5)
    x["omega_gate"] = torch.full((3, 5), 5e-4, dtype=F64)
    upd, last, lm, buf = omega_store_chain(**x)
    assert torch.count_nonzero(upd) == 0 and torch.count_nonzero(last) == 0
    assert buf is not None and torch.count_nonzero(buf) > 0     # the buffer still carries the gated surprises
    x["omega_gate"][1, 2] = 2e-3                                # one gate above the threshold: no short-circuit
    upd, _, _, _ = omega_store_chain(**x)
    assert torch.count_nonzero(upd) > 0


def test_newtonschulz5_acts_on_singular_values():
    """The quintic iteration maps X = U diag(s) V^T to U diag(p^5(s / ||s||)) V^T with
    p(x) = a x + b x^3 + c x^5 (the SVD closed form of the published iteration), for wide and tall
    matrices (tall ones are transposed and back); at most 3 dims pass through unchanged."""
    from oracle.omega import newtonschulz5
    g = torch.Generator().manual_seed(77)
    a, b, c = 3.4445, -4.7750, 2.0315
    for shape in [(2, 3, 6, 9), (2, 3, 9, 6), (1, 1, 5, 5)]:
        x = torch.randn(*shape, generator=g, dtype=F64)
        U, s, Vh = torch.linalg.svd(x, full_matrices=False)
        sn = s / s.norm(dim=-1, keepdim=True)
        for _ in range(5):
            sn = a * sn + b * sn ** 3 + c * sn ** 5
        want = U @ torch.diag_embed(sn) @ Vh
        torch.testing.assert_close(newtonschulz5(x), want, rtol=1e-9, atol=1e-9)
    y = torch.randn(3, 4, 5, generator=g, dtype=F64)
    assert newtonschulz5(y) is y


def test_newton_schulz_points_and_reference_shapes():
    """spectral_norm acts on the windowed update before the scan, muon on the scanned result;
    with every gate below 1e-3 reference_shapes gives the reference's n zero steps."""
    from oracle.omega import newtonschulz5
    x = _inputs(p=(4, 6))
    base = omega_store_chain(**x)
    sn = omega_store_chain(**x, spectral_norm=newtonschulz5)
    mu = omega_store_chain(**x, muon=newtonschulz5)
    # muon: the scanned result orthogonalised (next_last_update taken after it)
    torch.testing.assert_close(mu[0], newtonschulz5(base[0]))
    torch.testing.assert_close(mu[1], newtonschulz5(base[0])[:, -1])
    # spectral_norm: the scan over orthogonalised updates, differs from the plain chain
    assert not torch.allclose(sn[0], base[0])
    xo = dict(x, omega_gate=torch.full_like(x["omega_gate"], 5e-4))
    z = omega_store_chain(**xo, reference_shapes=True)
    assert z[0].shape[1] == x["surprise"].shape[1] and not z[0].any() and not z[1].any()
    z2 = omega_store_chain(**xo)
    assert z2[0].shape[1] == x["surprise"].shape[1] + 1 and not z2[0].any()
