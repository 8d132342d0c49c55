"""The state-block decomposition for head sizes the kernels are not built for (d_k = 128 after a
tensor feature map with d_v = 64 is BASELINE config C4), checked on the CPU as algebra: the
decomposition `functional.block_recurrence` runs on the GPU (64 x 64 blocks S[i, j] stacked along
the row axis, each with S_ref = 0 and v = -delta[rows of i], y = sum_j of the blocks' outputs) is
restated here with torch ops around the fp64 oracle as the 64-wide recurrence, and must equal the
oracle run on the full state, outputs and every input gradient (exact algebra: the bar is fp64
round-off). The GPU kernels of the split (atlas_block_split / _merge) are checked end to end
against the oracle in tests/test_gpu_parity.py (the c4_reduced and d_k != d_v cases)."""

from __future__ import annotations

import pytest
import torch

from oracle import memory_recurrence_vectorised, poly_feature_map

F64 = torch.float64
BLK = 64


def block_decomposition(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, *, window, map_mode, map_degree,
                        clamp_every, clamp_final, inner):
    """The block algebra of functional.block_recurrence with torch ops (fp64 reference)."""
    bh, T, dk = k.shape
    dv = v.shape[-1]
    nbk, nbv = -(-dk // BLK), -(-dv // BLK)
    Dk, Dv = nbk * BLK, nbv * BLK
    F = torch.nn.functional
    padf = lambda t, pads: t if t is None or not any(pads) else F.pad(t, pads)
    if map_mode == 'elementwise' and map_degree > 1:
        k, q = poly_feature_map(k, map_degree, 'elementwise'), poly_feature_map(q, map_degree, 'elementwise')
    phi, psi, vv = padf(k, (0, Dk - dk)), padf(q, (0, Dk - dk)), padf(v, (0, Dv - dv))
    pst = lambda t: padf(t, (0, Dk - dk, 0, Dv - dv))
    S_ref, S0, Z0, buffer = pst(S_ref), pst(S0), pst(Z0), pst(buffer)
    nv = vv - torch.matmul(phi, S_ref.transpose(-1, -2))       # v - S_ref phi = -delta
    nb = nbv * nbk

    def cols(x, i_major):   # [BH, T, n*64] -> [(i, j, bh), T, 64]
        n = x.shape[-1] // BLK
        x = x.reshape(bh, T, n, BLK).permute(2, 0, 1, 3)
        if i_major:   # row blocks i of nv, the same for every j
            x = x.unsqueeze(1).expand(nbv, nbk, bh, T, BLK)
        else:         # column blocks j of phi / psi, the same for every i
            x = x.unsqueeze(0).expand(nbv, nbk, bh, T, BLK)
        return x.reshape(nb * bh, T, BLK)

    def stack_state(x):
        if x is None:
            return None
        mid = x.shape[1:-2]
        x = x.reshape(bh, *mid, nbv, BLK, nbk, BLK)
        m = len(mid)
        return x.permute(m + 1, m + 3, 0, *range(1, m + 1), m + 2, m + 4).reshape(nb * bh, *mid, BLK, BLK)

    rep = lambda t: None if t is None else t.unsqueeze(0).expand(nb, *t.shape).reshape(nb * bh, *t.shape[1:])
    S0b = stack_state(S0)
    y, S_T, Z_T, B = inner(cols(phi, False), cols(psi, False), cols(nv, True), rep(lr), rep(decay), rep(beta),
                           rep(gate), torch.zeros_like(S0b), S0b, stack_state(Z0), stack_state(buffer),
                           window=window, map_mode='off', map_degree=1, clamp_every=clamp_every,
                           clamp_final=clamp_final)
    y = y.reshape(nbv, nbk, bh, T, BLK).sum(dim=1).permute(1, 2, 0, 3).reshape(bh, T, Dv)

    def unblock(x):
        if x is None:
            return None
        mid = x.shape[1:-2]
        m = len(mid)
        x = x.reshape(nbv, nbk, bh, *mid, BLK, BLK)
        return x.permute(2, *range(3, m + 3), 0, m + 3, 1, m + 4).reshape(bh, *mid, Dv, Dk)[..., :dv, :dk]

    return y[..., :dv], unblock(S_T), unblock(Z_T), unblock(B)


def _oracle_inner(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, *, window, map_mode, map_degree,
                  clamp_every, clamp_final):
    assert map_mode == 'off' and k.shape[-1] == 64 and v.shape[-1] == 64
    return memory_recurrence_vectorised(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, window=window,
                                        clamp_every=clamp_every, clamp_final=clamp_final)


def _inputs(BH, T, dk, dv, e, gate, momentum, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=F64)
    k = r(BH, T, dk)
    k = k / k.norm(dim=-1, keepdim=True)
    x = dict(k=k, q=r(BH, T, dk), v=r(BH, T, dv), lr=0.1 * torch.sigmoid(r(BH, T)),
             decay=torch.sigmoid(r(BH, T) * 0.5 + 2.0),
             beta=torch.sigmoid(r(BH, T) * 0.5 + 1.0) if momentum else None,
             gate=(torch.softmax(r(BH, T, e), -1) if gate == 'lag' else
                   torch.sigmoid(r(BH, T)) if gate == 'token' else None),
             S_ref=0.1 * r(BH, dv, dk), S0=0.1 * r(BH, dv, dk), Z0=0.1 * r(BH, dv, dk) if momentum else None,
             buffer=0.1 * r(BH, e - 1, dv, dk) if e > 1 else None)
    up = dict(gy=r(BH, T, dv), gS=r(BH, dv, dk), gZ=r(BH, dv, dk), gB=r(BH, max(e - 1, 1), dv, dk))
    return x, up


def _loss(out, up):
    y, S_T, Z_T, B = out
    loss = (y * up["gy"]).sum() + (S_T * up["gS"]).sum()
    if Z_T is not None:
        loss = loss + (Z_T * up["gZ"]).sum()
    if B is not None:
        loss = loss + (B * up["gB"][:, :B.shape[1]]).sum()
    return loss


@pytest.mark.parametrize("dk,dv,e,gate,momentum,degree,clamp_every", [
    (128, 64, 8, 'lag', True, 3, None),      # C4 shape class (d_k 128 after the tensor map, d_v 64)
    (128, 64, 4, 'token', True, 1, None),
    (96, 80, 4, 'lag', True, 1, None),       # both padded
    (64, 128, 3, None, False, 2, None),      # row blocks only
    (128, 128, 2, 'token', True, 1, 16),     # 2 x 2 blocks with the scan_chunk_len clamp
])
def test_block_recurrence_matches_full_oracle(dk, dv, e, gate, momentum, degree, clamp_every):
    BH, T = 2, 40
    x, up = _inputs(BH, T, dk, dv, e, gate, momentum, seed=dk * 7 + dv + e)
    if clamp_every:
        x["S0"] = x["S0"] * 2000.0      # large enough for the clamp at +-100 to act
    names = [n for n in x if x[n] is not None]

    def run(fn):
        leaves = {n: x[n].clone().requires_grad_(True) for n in names}
        a = {n: leaves.get(n) for n in x}
        out = fn(a)
        gs = torch.autograd.grad(_loss(out, up), [leaves[n] for n in names])
        return [o.detach() if o is not None else None for o in out], dict(zip(names, gs))

    mode = 'elementwise' if degree > 1 else 'off'
    ref_out, ref_g = run(lambda a: memory_recurrence_vectorised(
        poly_feature_map(a["k"], degree, mode), poly_feature_map(a["q"], degree, mode), a["v"], a["lr"],
        a["decay"], a["beta"], a["gate"], a["S_ref"], a["S0"], a["Z0"], a["buffer"], window=e,
        clamp_every=clamp_every, clamp_final=True))
    got_out, got_g = run(lambda a: block_decomposition(
        a["k"], a["q"], a["v"], a["lr"], a["decay"], a["beta"], a["gate"], a["S_ref"], a["S0"], a["Z0"],
        a["buffer"], window=e, map_mode=mode, map_degree=degree, clamp_every=clamp_every, clamp_final=True,
        inner=_oracle_inner))
    for name, g_, r_ in zip(("y", "S_T", "Z_T", "buffer_out"), got_out, ref_out):
        if r_ is None:
            assert g_ is None, name
            continue
        assert g_.shape == r_.shape, name
        torch.testing.assert_close(g_, r_, rtol=1e-10, atol=1e-10 * r_.abs().max().item(), msg=name)
    for n in names:
        torch.testing.assert_close(got_g[n], ref_g[n], rtol=1e-9, atol=1e-9 * ref_g[n].abs().max().item(),
                                   msg="d" + n)
