"""GPU parity of BASELINE config C4 at its full geometry, against the fp64 oracle on a subset of rows.

C4: B=2, H=8 (BH = 16), T = 8192; raw keys and queries [16, 8192, 64] (L2-normalised) go through
the tensor feature map [x; vec(x x^T)] P with P [4160, 128] Xavier-uniform (rnn_memory.py:125-130),
then the elementwise polynomial of degree 3; the recurrence then runs with d_k = 128, d_v = 64,
e = 8 per-lag gates and momentum (rnn_memory.py:605-730), as two stacked 64 x 64 state blocks.

The GPU runs the whole problem: the fused map over all 131,072 tokens of k and of q, the block
recurrence at its full segment plan, and the backward through both. Rows are independent, so the
oracle (fp64, the map included, in 256-token blocks carrying the state) runs rows 0, 7 and 15 only,
and those rows of y, S_T, Z_T, buffer_out and of the gradients of k and q (through the map), v, the
scalars, the gates, S_ref, S0 and Z0 are compared.

Tolerances: bf16 inputs with fp32 state 2e-2, fp32 inputs 1e-4 (normwise and elementwise with an
atol floor, `_cases.compare`).
"""

import sys

import pytest
import torch

from _cases import compare
from oracle import memory_recurrence_vectorised, poly_feature_map

pytestmark = pytest.mark.gpu

F64 = torch.float64
BH, T, D_IN, DK, DV, E = 16, 8192, 64, 128, 64, 8
ROWS = (0, 7, 15)
BLOCK = 256


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32)
    k = r(BH, T, D_IN)
    k = k / k.norm(dim=-1, keepdim=True)
    q = r(BH, T, D_IN)
    q = q / q.norm(dim=-1, keepdim=True)
    bound = (6.0 / (D_IN + D_IN * D_IN + DK)) ** 0.5
    P = (torch.rand(D_IN + D_IN * D_IN, DK, generator=g) * 2 - 1) * bound
    x = dict(k=k, q=q, v=r(BH, T, DV), lr=0.1 * torch.sigmoid(r(BH, T)),
             decay=torch.sigmoid(r(BH, T) * 0.5 + 2.0), beta=torch.sigmoid(r(BH, T) * 0.5 + 1.0),
             gate=torch.softmax(r(BH, T, E), dim=-1))
    x = {kk: v.to(dtype) for kk, v in x.items()}
    st = dict(S_ref=0.1 * r(BH, DV, DK), S0=0.1 * r(BH, DV, DK), Z0=0.05 * r(BH, DV, DK))
    loss_w = dict(gy=r(BH, T, DV).to(dtype), gS=r(BH, DV, DK), gZ=r(BH, DV, DK), gB=r(BH, E - 1, DV, DK))
    return x, P.to(dtype), st, loss_w


def _oracle_rows(x, P, st, lw, rows):
    """fp64 map + recurrence on `rows`, in BLOCK-token blocks carrying (S, Z, buffer); autograd
    through the map gives dk and dq."""
    idx = torch.tensor(rows)
    xs = {kk: v[idx].to(F64).requires_grad_(True) for kk, v in x.items()}
    ss = {kk: v[idx].to(F64).requires_grad_(True) for kk, v in st.items()}
    P64 = P.to(F64)
    ys = []
    S, Z, B = ss["S0"], ss["Z0"], None
    for s0 in range(0, T, BLOCK):
        sl = slice(s0, s0 + BLOCK)
        fk = poly_feature_map(poly_feature_map(xs["k"][:, sl], 2, 'tensor', P64), 3, 'elementwise')
        fq = poly_feature_map(poly_feature_map(xs["q"][:, sl], 2, 'tensor', P64), 3, 'elementwise')
        if x["k"].dtype == torch.bfloat16:   # the map's output is rounded to the recurrence's input dtype
            fk = fk + (fk.detach().to(torch.bfloat16).to(F64) - fk.detach())
            fq = fq + (fq.detach().to(torch.bfloat16).to(F64) - fq.detach())
        last = s0 + BLOCK >= T
        y, S, Z, B = memory_recurrence_vectorised(fk, fq, xs["v"][:, sl], xs["lr"][:, sl], xs["decay"][:, sl],
                                                  xs["beta"][:, sl], xs["gate"][:, sl], ss["S_ref"], S, Z, B,
                                                  window=E, clamp_every=None, clamp_final=last)
        ys.append(y)
    y = torch.cat(ys, dim=1)
    lw64 = {kk: v[idx].to(F64) for kk, v in lw.items()}
    loss = (y * lw64["gy"]).sum() + (S * lw64["gS"]).sum() + (Z * lw64["gZ"]).sum() + (B * lw64["gB"]).sum()
    names = list(xs) + list(ss)
    grads = torch.autograd.grad(loss, [xs[n] for n in xs] + [ss[n] for n in ss])
    return [y.detach(), S.detach(), Z.detach(), B.detach()], dict(zip(names, grads))


def _gpu(x, P, st, lw):
    from atlas_rnn_amd.functional import memory_recurrence, tensor_feature_map
    dev = torch.device("cuda:0")
    xg = {kk: v.to(dev).requires_grad_(True) for kk, v in x.items()}
    sg = {kk: v.to(dev).requires_grad_(True) for kk, v in st.items()}
    Pg = P.to(dev)
    fk = tensor_feature_map(xg["k"], Pg, degree=3)
    fq = tensor_feature_map(xg["q"], Pg, degree=3)
    y, S_T, Z_T, B = memory_recurrence(fk, fq, xg["v"], xg["lr"], xg["decay"], xg["beta"], xg["gate"], sg["S_ref"],
                                       sg["S0"], sg["Z0"], None, window=E)
    lwg = {kk: v.to(dev) for kk, v in lw.items()}
    loss = ((y.float() * lwg["gy"].float()).sum() + (S_T * lwg["gS"]).sum() + (Z_T * lwg["gZ"]).sum()
            + (B * lwg["gB"]).sum())
    names = list(xg) + list(sg)
    grads = torch.autograd.grad(loss, [xg[n] for n in xg] + [sg[n] for n in sg])
    torch.cuda.synchronize()
    out = [t.detach().float().cpu() for t in (y, S_T, Z_T, B)]
    return out, {n: gr.float().cpu() for n, gr in zip(names, grads)}


@pytest.mark.parametrize("dtype,tol,seed", [(torch.bfloat16, 2e-2, 4101), (torch.float32, 1e-4, 4102)],
                         ids=["c4_full_bf16", "c4_full_fp32"])
def test_c4_full_geometry_rows_match_oracle(dtype, tol, seed):
    _say(f"C4 full geometry ({dtype}): BH={BH} T={T} tensor map {D_IN}+{D_IN * D_IN}->{DK} g=3, dv={DV}, e={E}")
    x, P, st, lw = _inputs(dtype, seed)
    got_out, got_grads = _gpu(x, P, st, lw)
    _say(f"  gpu done; oracle on rows {ROWS}")
    ref_out, ref_grads = _oracle_rows(x, P, st, lw, ROWS)
    idx = torch.tensor(ROWS)
    for name, g, r in zip(("y", "S_T", "Z_T", "buffer_out"), got_out, ref_out):
        compare(f"c4_full.{name}", g[idx], r, tol)
    for name, r in ref_grads.items():
        compare(f"c4_full.d{name}", got_grads[name][idx], r, tol)
    _say(f"  C4 rows {ROWS}: 4 outputs and {len(ref_grads)} gradients match")
