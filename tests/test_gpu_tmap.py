"""GPU parity of the fused tensor feature map (atlas_tensor_map_fwd / _bwd) against the fp64
oracle map `poly_feature_map(x, 2, 'tensor', proj)` (rnn_memory.py:125-130), on inputs rounded to
the kernel's dtype: the map's output and the gradient of x for a seeded upstream gradient, bf16
rtol 2e-2 and fp32 rtol 1e-4 (normwise and elementwise, tests/_cases.compare). bf16 at the fast
kernels' sizes (d_in 32 / 64, d_out 32 / 64 / 128) and at others (the general kernels, which also
run every fp32 size). Then the BASELINE C4 composition at a reduced size: the tensor map
(64 + 4096 -> 128) into the d_k = 128 / d_v = 64 recurrence with the elementwise map of degree 3,
window 8, lag gates and momentum, against the oracle end to end (outputs and every input gradient).
"""

import sys

import pytest
import torch

from _cases import compare
from oracle import memory_recurrence_vectorised, poly_feature_map

pytestmark = pytest.mark.gpu

F64 = torch.float64
BF16 = torch.bfloat16
F32 = torch.float32
TOL = 2e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


MAP_CASES = [
    # (n, d_in, d_out, degree, dtype): the fast bf16 kernels
    (300, 64, 128, 1, BF16), (129, 64, 64, 1, BF16), (77, 32, 32, 1, BF16), (1, 32, 128, 1, BF16),
    (256, 64, 32, 1, BF16), (1000, 32, 64, 1, BF16), (300, 64, 128, 3, BF16), (65, 32, 64, 2, BF16),
    # the general kernels: bf16 at other sizes, fp32 at every size
    (70, 16, 16, 1, BF16), (129, 64, 48, 2, BF16), (33, 32, 112, 1, BF16),
    (300, 64, 128, 1, F32), (129, 64, 64, 3, F32), (77, 32, 32, 1, F32), (40, 16, 16, 2, F32),
    (1, 16, 128, 1, F32), (200, 32, 80, 1, F32),
]


@pytest.mark.parametrize("n,d,m,deg,dt", MAP_CASES, ids=[f"{c[4]}-{c[0]}x{c[1]}-{c[2]}-g{c[3]}".replace("torch.", "")
                                                          for c in MAP_CASES])
def test_tensor_map_parity(n, d, m, deg, dt):
    from atlas_rnn_amd.functional import _TensorMapFn
    _say(f"tensor map n={n} d={d} m={m} degree={deg} {dt}")
    g = torch.Generator().manual_seed(n * 7 + d + m)
    x = torch.randn(n, d, generator=g)
    x = (x / x.norm(dim=-1, keepdim=True)).to(dt)
    bound = (6.0 / (d + d * d + m)) ** 0.5
    P = ((torch.rand(d + d * d, m, generator=g) * 2 - 1) * bound).to(dt)
    gy = torch.randn(n, m, generator=g).to(dt)
    # oracle
    x64 = x.to(F64).requires_grad_(True)
    ref = poly_feature_map(poly_feature_map(x64, 2, 'tensor', P.to(F64)), deg, 'elementwise')
    (dref,) = torch.autograd.grad((ref * gy.to(F64)).sum(), [x64])
    # kernels (through the autograd function)
    xg = x.cuda().requires_grad_(True)
    out = _TensorMapFn.apply(xg, P.cuda(), deg)
    assert out.dtype == dt
    (dx,) = torch.autograd.grad((out.float() * gy.cuda().float()).sum(), [xg])
    torch.cuda.synchronize()
    tol = TOL if dt == BF16 else 1e-4
    compare("phi", out.detach().float().cpu(), ref.detach(), tol)
    compare("dx", dx.float().cpu(), dref, tol)


@pytest.mark.parametrize("dt,m", [(BF16, 128), (F32, 128), (BF16, 64), (BF16, 32)],
                         ids=["bf16_m128", "fp32_m128", "bf16_m64", "bf16_m32"])
def test_symmetrized_table_and_both_forwards(dt, m):
    """atlas_tensor_map_symmetrize against the table formed on the CPU (P's linear rows, then
    P[a][b] + P[b][a] above the diagonal, P[a][a] on it, zeros below; bit-exact after rounding the
    fp32 sum to the dtype) and its transpose; then atlas_tensor_map_fwd on P^T and
    atlas_tensor_map_fwd_sym on the symmetrised table against the oracle map, and the gradient of x
    from atlas_tensor_map_bwd on P and atlas_tensor_map_bwd_sym on the symmetrised table against the
    oracle's (fp64 autograd)."""
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import _ptr, _stream
    d, n = 64, 257
    _say(f"symmetrised tensor-map table {dt} m={m}")
    g = torch.Generator().manual_seed(777)
    bound = (6.0 / (d + d * d + m)) ** 0.5
    P = ((torch.rand(d + d * d, m, generator=g) * 2 - 1) * bound).to(dt)
    Pq = P[d:].float().reshape(d, d, m)
    ref_q = Pq + Pq.transpose(0, 1)
    a = torch.arange(d).view(d, 1)
    b = torch.arange(d).view(1, d)
    ref_q = torch.where((b > a).unsqueeze(-1), ref_q, torch.where((b == a).unsqueeze(-1), Pq, torch.zeros_like(Pq)))
    ref = torch.cat([P[:d].float(), ref_q.reshape(d * d, m)]).to(dt)
    lib = _lib.load()
    dev = torch.device("cuda:0")
    code = _lib.DT_BF16 if dt == BF16 else _lib.DT_F32
    Pd = P.to(dev)
    ps = torch.empty_like(Pd)
    pst = torch.empty(m, d + d * d, device=dev, dtype=dt)
    _lib.check(lib.atlas_tensor_map_symmetrize(code, d, m, _ptr(Pd), _ptr(ps), _ptr(pst), _stream(dev)), "symmetrize")
    torch.cuda.synchronize()
    assert torch.equal(ps.cpu(), ref)
    assert torch.equal(pst.cpu(), ref.t().contiguous())
    x = torch.randn(n, d, generator=g)
    x = (x / x.norm(dim=-1, keepdim=True)).to(dt)
    oracle = poly_feature_map(x.to(F64), 2, 'tensor', P.to(F64))
    xd = x.to(dev)
    pt = Pd.t().contiguous()
    tol = TOL if dt == BF16 else 1e-4
    for name, fn, table in (("fwd", lib.atlas_tensor_map_fwd, pt), ("fwd_sym", lib.atlas_tensor_map_fwd_sym, pst)):
        out = torch.empty(n, m, device=dev, dtype=dt)
        _lib.check(fn(code, n, d, m, 1, _ptr(xd), _ptr(table), _ptr(out), None, _stream(dev)), name)
        torch.cuda.synchronize()
        compare(f"tmap.{name}", out.float().cpu(), oracle, tol)
    # backward: atlas_tensor_map_bwd on P and atlas_tensor_map_bwd_sym on the symmetrised table
    dout = torch.randn(n, m, generator=g).to(dt)
    xo = x.to(F64).requires_grad_()
    (poly_feature_map(xo, 2, 'tensor', P.to(F64)) * dout.to(F64)).sum().backward()
    dd = dout.to(dev)
    for name, fn, table in (("bwd", lib.atlas_tensor_map_bwd, Pd), ("bwd_sym", lib.atlas_tensor_map_bwd_sym, ps)):
        dx = torch.empty(n, d, device=dev, dtype=dt)
        _lib.check(fn(code, n, d, m, 1, _ptr(xd), _ptr(table), None, _ptr(dd), _ptr(dx), _stream(dev)), name)
        torch.cuda.synchronize()
        compare(f"tmap.{name}", dx.float().cpu(), xo.grad, tol)


def test_c4_composition_reduced():
    """tensor map -> d_k 128 / d_v 64 recurrence (block path, elementwise map g = 3), fwd + bwd."""
    from atlas_rnn_amd.functional import memory_recurrence, tensor_feature_map
    BH, T, d, dk, dv, e = 4, 160, 64, 128, 64, 8
    _say(f"c4 composition BH={BH} T={T}")
    g = torch.Generator().manual_seed(4004)
    r = lambda *s: torch.randn(*s, generator=g)
    k = r(BH, T, d)
    k = k / k.norm(dim=-1, keepdim=True)
    q = r(BH, T, d)
    q = q / q.norm(dim=-1, keepdim=True)
    bound = (6.0 / (d + d * d + dk)) ** 0.5
    P = ((torch.rand(d + d * d, dk, generator=g) * 2 - 1) * bound).to(BF16)
    x = dict(k=k, q=q, v=r(BH, T, dv), lr=0.1 * torch.sigmoid(r(BH, T)), decay=torch.sigmoid(r(BH, T) * 0.5 + 2.0),
             beta=torch.sigmoid(r(BH, T) * 0.5 + 1.0), gate=torch.softmax(r(BH, T, e), -1))
    x = {kk: v.to(BF16) for kk, v in x.items()}
    S0 = 0.1 * r(BH, dv, dk)
    gy = r(BH, T, dv).to(BF16)
    gS = r(BH, dv, dk)
    names = list(x)

    # oracle: fp64 on the bf16 values; the map rounds its output to bf16 like the kernels' input
    x64 = {kk: v.to(F64).requires_grad_(True) for kk, v in x.items()}
    S064 = S0.to(F64)
    pk = poly_feature_map(poly_feature_map(x64["k"], 2, 'tensor', P.to(F64)), 3, 'elementwise')
    pq = poly_feature_map(poly_feature_map(x64["q"], 2, 'tensor', P.to(F64)), 3, 'elementwise')
    y, S_T, Z_T, B = memory_recurrence_vectorised(pk, pq, x64["v"], x64["lr"], x64["decay"], x64["beta"], x64["gate"],
                                                  S064, S064, torch.zeros_like(S064), None, window=e)
    loss = (y * gy.to(F64)).sum() + (S_T * gS.to(F64)).sum()
    ref_g = dict(zip(names, torch.autograd.grad(loss, [x64[kk] for kk in names])))

    xg = {kk: v.cuda().requires_grad_(True) for kk, v in x.items()}
    Sg = S0.cuda()
    Pg = P.cuda()
    fk = tensor_feature_map(xg["k"], Pg, degree=3)
    fq = tensor_feature_map(xg["q"], Pg, degree=3)
    yg, STg, ZTg, Bg = memory_recurrence(fk, fq, xg["v"], xg["lr"], xg["decay"], xg["beta"], xg["gate"], Sg, Sg,
                                         torch.zeros_like(Sg), None, window=e)
    lg = (yg.float() * gy.cuda().float()).sum() + (STg * gS.cuda()).sum()
    got_g = dict(zip(names, torch.autograd.grad(lg, [xg[kk] for kk in names])))
    torch.cuda.synchronize()
    compare("c4.y", yg.detach().float().cpu(), y.detach(), TOL)
    compare("c4.S_T", STg.detach().float().cpu(), S_T.detach(), TOL)
    for kk in names:
        compare(f"c4.d{kk}", got_g[kk].float().cpu(), ref_g[kk], TOL)


def test_symmetrised_tables_follow_in_place_changes_of_proj():
    """The symmetrised tables are kept per projection; an in-place change of proj (its version)
    forms them again, so the map always uses the current proj."""
    from atlas_rnn_amd.functional import tensor_feature_map
    _say("tensor map after an in-place change of proj")
    g = torch.Generator().manual_seed(778)
    d, m, n = 64, 128, 200
    bound = (6.0 / (d + d * d + m)) ** 0.5
    P = ((torch.rand(d + d * d, m, generator=g) * 2 - 1) * bound).to(BF16)
    x = torch.randn(n, d, generator=g)
    x = (x / x.norm(dim=-1, keepdim=True)).to(BF16)
    dev = torch.device("cuda:0")
    Pd, xd = P.to(dev), x.to(dev)
    out1 = tensor_feature_map(xd, Pd, 1)
    out2 = tensor_feature_map(xd, Pd, 1)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    Pd.mul_(2.0)   # exact in bf16
    out3 = tensor_feature_map(xd, Pd, 1)
    torch.cuda.synchronize()
    compare("tmap.after_inplace", out3.float().cpu(), poly_feature_map(x.to(F64), 2, 'tensor', 2.0 * P.to(F64)), TOL)
