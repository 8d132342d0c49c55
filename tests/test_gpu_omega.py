"""GPU parity of atlas_rnn_amd.omega (the Omega section of OmegaNeuralMemory.store_memories,
omega.py:262-318, and its feature map omega.py:90-118) against oracle/omega.py in float64: every
output and the gradients of every input (surprise, decay, last update, momentum gates and state,
combine weights, omega gate, carried buffer). fp32 rtol 1e-4, bf16 rtol 2e-2 (normwise and
elementwise, tests/_cases.compare)."""

import sys

import pytest
import torch

from _cases import compare
from atlas_rnn_amd.omega import OmegaPolyFeatures, apply_poly_features, omega_store_chain
from oracle import poly_feature_map
from oracle.omega import omega_store_chain as oracle_chain

pytestmark = pytest.mark.gpu

F64 = torch.float64
BF16 = torch.bfloat16


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(BH, n, p, O, combine, gate, e, buf, seed, dt):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    x = dict(surprise=r(BH, n, *p), decay_factor=torch.sigmoid(r(BH, n) - 2), last_update=r(BH, *p))
    if O:
        x["adaptive_momentum"] = torch.sigmoid(r(O, BH, n) + 1)
        x["last_momentum"] = r(O, BH, *p)
        if combine:
            x["combine_momentums"] = r(O, BH, n)
    if gate:
        x["omega_gate"] = torch.sigmoid(r(BH, n))
    if buf and e > 1:
        x["omega_buf"] = 0.5 * r(BH, e - 1, *p)
    return {k: v.to(dt).to(torch.float32) for k, v in x.items()}


CASES = [
    # (name, BH, n, param shape, momentum order, combine, gate, window, buffer, dtype)
    ("fp32_w4_mom1_gate_buf", 6, 16, (32, 16), 1, False, True, 4, True, torch.float32),
    ("fp32_w1_nomom_nogate", 4, 9, (8,), 0, False, False, 1, False, torch.float32),
    ("fp32_w3_mom2_combine", 5, 12, (16, 16), 2, True, True, 3, True, torch.float32),
    ("fp32_w8_longer_than_n", 3, 5, (4, 8), 1, False, True, 8, True, torch.float32),
    ("fp32_scalar_params", 8, 7, (), 1, False, True, 2, True, torch.float32),
    ("bf16_w4_mom1_gate_buf", 6, 16, (32, 16), 1, False, True, 4, True, BF16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_omega_store_chain_parity(case):
    name, BH, n, p, O, combine, gate, e, buf, dt = case
    _say(f"omega chain {name}")
    x = _inputs(BH, n, p, O, combine, gate, e, buf, seed=sum(map(ord, name)), dt=dt)
    xr = {k: v.to(F64).requires_grad_() for k, v in x.items()}
    ref = oracle_chain(**xr, omega_window=e)
    xd = {k: v.to("cuda", dt).requires_grad_() for k, v in x.items()}
    got = omega_store_chain(**xd, omega_window=e)
    g = torch.Generator().manual_seed(7)
    weights = [torch.randn(r.shape, generator=g, dtype=F64) if r is not None else None for r in ref]
    loss_r = sum((r * w).sum() for r, w in zip(ref, weights) if r is not None)
    loss_d = sum((o.float() * w.to("cuda", torch.float32)).sum() for o, w in zip(got, weights) if o is not None)
    names = sorted(x)
    gr = torch.autograd.grad(loss_r, [xr[k] for k in names])
    gd = torch.autograd.grad(loss_d, [xd[k] for k in names])
    torch.cuda.synchronize()
    tol = 1e-4 if dt == torch.float32 else 2e-2
    for nm, o, r in zip(("update", "next_last_update", "next_last_momentum", "next_buf"), got, ref):
        if r is None:
            assert o is None, nm
            continue
        assert o.shape == r.shape, nm
        compare(f"{name}.{nm}", o.detach().float().cpu(), r.detach(), tol)
    for k, a, b in zip(names, gd, gr):
        compare(f"{name}.d{k}", a.float().cpu(), b, tol)


def test_omega_gate_short_circuit_on_device():
    """All gates below 1e-3: zero updates and zero next_last_update, chosen without a host sync;
    the buffer still carries the gated surprises."""
    _say("omega gate short-circuit")
    BH, n, p = 4, 6, (8, 4)
    g = torch.Generator().manual_seed(3)
    s = torch.randn(BH, n, *p, generator=g).cuda()
    gate = torch.full((BH, n), 5e-4).cuda()
    upd, last, _, buf = omega_store_chain(s, torch.full((BH, n), 0.1).cuda(), torch.randn(BH, *p).cuda(),
                                          omega_gate=gate, omega_window=3)
    assert upd.shape == (BH, n + 1, *p)
    assert torch.count_nonzero(upd).item() == 0 and torch.count_nonzero(last).item() == 0
    ref_buf = oracle_chain(s.cpu().double(), torch.full((BH, n), 0.1, dtype=F64), torch.zeros(BH, *p, dtype=F64),
                           omega_gate=gate.cpu().double(), omega_window=3)[3]
    compare("short_circuit.buf", buf.cpu(), ref_buf, 1e-5)


@pytest.mark.parametrize("mode,degree,dt", [("elementwise", 3, torch.float32), ("tensor", 2, BF16),
                                            ("tensor", 2, torch.float32)])
def test_omega_poly_features(mode, degree, dt):
    """omega.py:90-118 on the GPU: the elementwise polynomial, and the tensor map with the cached
    projection (the fused kernel) against the oracle's closed form with the same projection."""
    _say(f"omega poly features {mode} {degree} {dt}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 37, 64, generator=g).to(dt)
    fm = OmegaPolyFeatures(degree, mode)
    out = fm(x.cuda())
    if mode == "tensor":
        (proj,) = fm._poly_proj_cache.values()
        assert proj.shape == (64 + 64 * 64, 64)
        again = apply_poly_features(x.cuda(), degree, mode, fm._poly_proj_cache)   # cached: the same projection
        assert torch.equal(out, again)
        ref = poly_feature_map(x.double(), 2, 'tensor', proj.cpu().double())
    else:
        ref = poly_feature_map(x.double(), degree, 'elementwise')
    compare(f"omega_poly.{mode}", out.float().cpu(), ref, 1e-4 if dt == torch.float32 else 2e-2)


@pytest.mark.parametrize("point", ["spectral_norm", "muon", "both"])
def test_omega_newton_schulz_points(point):
    """The reference's two Newton-Schulz points (omega.py:304-305, :317-318) with the library's
    newtonschulz5 on the GPU against the oracle's fp64 restatement at the same points: every output
    and every input gradient (fp32, rtol 1e-4 on outputs; gradients through five NS steps 1e-3)."""
    from atlas_rnn_amd.omega import newtonschulz5
    from oracle.omega import newtonschulz5 as ns_ref
    _say(f"omega chain with Newton-Schulz at {point}")
    BH, n, p, e = 4, 10, (8, 12), 3
    x = _inputs(BH, n, p, 1, False, True, e, True, seed=91, dt=torch.float32)
    kw_r = dict(spectral_norm=ns_ref if point in ("spectral_norm", "both") else None,
                muon=ns_ref if point in ("muon", "both") else None)
    kw_d = dict(spectral_norm=newtonschulz5 if point in ("spectral_norm", "both") else None,
                muon=newtonschulz5 if point in ("muon", "both") else None)
    xr = {k: v.to(F64).requires_grad_() for k, v in x.items()}
    ref = oracle_chain(**xr, omega_window=e, **kw_r)
    xd = {k: v.to("cuda").requires_grad_() for k, v in x.items()}
    got = omega_store_chain(**xd, omega_window=e, **kw_d)
    g = torch.Generator().manual_seed(8)
    weights = [torch.randn(r.shape, generator=g, dtype=F64) for r in ref]
    loss_r = sum((r * w).sum() for r, w in zip(ref, weights))
    loss_d = sum((o.float() * w.to("cuda", torch.float32)).sum() for o, w in zip(got, weights))
    names = sorted(x)
    gr = torch.autograd.grad(loss_r, [xr[k] for k in names])
    gd = torch.autograd.grad(loss_d, [xd[k] for k in names])
    torch.cuda.synchronize()
    for nm, o, r in zip(("update", "next_last_update", "next_last_momentum", "next_buf"), got, ref):
        compare(f"ns_{point}.{nm}", o.detach().float().cpu(), r.detach(), 1e-4)
    for k, a, b in zip(names, gd, gr):
        compare(f"ns_{point}.d{k}", a.float().cpu(), b, 1e-3)


def test_omega_reference_shapes_zero_branch():
    """reference_shapes=True: with every gate below 1e-3 the reference's n zero steps (a host
    decision, as omega.py:311-313 makes it); otherwise the scanned n + 1 steps as by default."""
    _say("omega chain with the reference's zero-branch shape")
    BH, n, p = 3, 5, (4, 4)
    g = torch.Generator().manual_seed(9)
    s = torch.randn(BH, n, *p, generator=g).cuda()
    dec = torch.full((BH, n), 0.1).cuda()
    last = torch.randn(BH, *p, generator=g).cuda()
    upd, nl, _, _ = omega_store_chain(s, dec, last, omega_gate=torch.full((BH, n), 5e-4).cuda(), omega_window=2,
                                      reference_shapes=True)
    assert upd.shape == (BH, n, *p) and torch.count_nonzero(upd).item() == 0
    assert torch.count_nonzero(nl).item() == 0
    gate = torch.full((BH, n), 0.5).cuda()
    a = omega_store_chain(s, dec, last, omega_gate=gate, omega_window=2, reference_shapes=True)
    b = omega_store_chain(s, dec, last, omega_gate=gate, omega_window=2)
    assert a[0].shape == (BH, n + 1, *p)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
