"""The bf16 drop-in cell end to end at BASELINE config C5's layer shape, against an fp64 composition.

`OmegaRNNMemoryCell(dim=512, dim_head=64, heads=8, omega_window=4)` (rnn_memory.py:415-730) in
bf16, batch 8, T = 2048, called with a carried state (S, Z and the omega buffer from an earlier
call). The GPU runs the whole batch through the library's path: the fused prologue kernels, the
batched projection products and weight gradients, the recurrence walks and `to_out`. Batch rows are
independent through every layer, so the loss is taken on batch row 0 only (its output and the next
state of its 8 heads); then every parameter gradient is row 0's, and the reference runs row 0 alone.

Reference: the cell's own layers in fp64 on the same (bf16-valued) parameters, composed as
rnn_memory.py:556-730 with the fp64 oracle recurrence (in 256-token blocks carrying the state). The
bf16 tensors the GPU materialises between layers (the convolved inputs, the projections, the
normalised q / k, the gate heads' products and sigmoids, y, the output) are rounded to bf16 in the
reference, as are the gradients flowing back through them (bf16 tensors have bf16 gradients), and a
gate sigmoid's backward uses its stored bf16 output as torch's bf16 sigmoid does (s (1 - s) with s
near 1 is where bf16 storage matters most), so the comparison measures the kernels' arithmetic
rather than the storage format.
Tolerance: 2e-2 (bf16 inputs), normwise and elementwise with an atol floor (`_cases.compare`).
"""

import copy
import sys

import pytest
import torch
from einops import rearrange

import atlas_rnn_amd as am
from _cases import compare
from oracle import memory_recurrence_vectorised

pytestmark = pytest.mark.gpu

F64 = torch.float64
BF16 = torch.bfloat16
DIM, DH, HEADS, E, BATCH, T = 512, 64, 8, 4, 8, 2048
BLOCK = 256
TOL = 2e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class _Bf16Point(torch.autograd.Function):
    """A tensor the GPU holds in bf16: its value is rounded to bf16, and so is the gradient that
    flows back through it (autograd keeps a bf16 tensor's gradient in bf16)."""

    @staticmethod
    def forward(ctx, t):
        return t.to(BF16).to(t.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(BF16).to(g.dtype)


def _r(t):
    return _Bf16Point.apply(t)


class _GateSigmoid(torch.autograd.Function):
    """A gate head's sigmoid as the GPU (and torch's own bf16 sigmoid) computes it: the output is
    stored in bf16 and the backward forms dz = dg s (1 - s) from that stored s, in bf16."""

    @staticmethod
    def forward(ctx, z):
        s = torch.sigmoid(z).to(BF16).to(z.dtype)
        ctx.save_for_backward(s)
        return s

    @staticmethod
    def backward(ctx, g):
        (s,) = ctx.saved_tensors
        return (g.to(BF16).to(g.dtype) * s * (1 - s)).to(BF16).to(g.dtype)


def _reference_row(cell, x, state):
    """rnn_memory.py:556-730 for one batch row with fp64 layers and the oracle recurrence."""
    batch, n, _ = x.shape
    x_act = _r(cell.activation(cell.pre_norm(x)))
    q_in = _r(cell.q_conv(x_act.transpose(1, 2)).transpose(1, 2))
    k_in = _r(cell.k_conv(x_act.transpose(1, 2)).transpose(1, 2))
    v_in = _r(cell.v_conv(x_act.transpose(1, 2)).transpose(1, 2))
    q = cell.split_heads(_r(cell.to_q(q_in)))[:, :, :n]
    k = cell.split_heads(_r(cell.to_k(k_in)))[:, :, :n]
    v = cell.split_heads(_r(cell.to_v(v_in)))[:, :, :n]
    q, k = _r(cell.q_norm(q)), _r(cell.k_norm(k))
    flat = lambda t: rearrange(t, 'b h n d -> (b h) n d')
    k, q, v = flat(k), flat(q), flat(v)
    # a gate head: the product (bf16), its bias, the sigmoid stored in bf16
    heads = lambda lin: rearrange(_GateSigmoid.apply(_r(x_act @ lin[0].weight.t()) + lin[0].bias),
                                  'b n h -> (b h) n')
    lr, decay, beta, gate = (heads(cell.to_lr), heads(cell.to_decay), heads(cell.to_momentum),
                             heads(cell.to_omega_gate))
    S_ref, S, Z, B = state.S, state.S, state.Z, state.omega_buffer
    ys = []
    for s0 in range(0, n, BLOCK):
        sl = slice(s0, min(n, s0 + BLOCK))
        y, S, Z, B = memory_recurrence_vectorised(k[:, sl], q[:, sl], v[:, sl], lr[:, sl], decay[:, sl], beta[:, sl],
                                                  gate[:, sl], S_ref, S, Z, B, window=E, clamp_every=None,
                                                  clamp_final=s0 + BLOCK >= n)
        ys.append(y)
    y = _r(torch.cat(ys, dim=1))
    y = rearrange(y, '(b h) t d -> b h t d', b=batch, h=cell.heads)
    out = _r(cell.to_out(cell.merge_heads(y)))
    return out, (S, Z, B)


def test_bf16_cell_c5_layer_shape_row0_matches_fp64_composition():
    _say(f"bf16 cell dim={DIM} heads={HEADS}x{DH} e={E} batch={BATCH} T={T}, carried state, loss on row 0")
    torch.manual_seed(51)
    cell = am.OmegaRNNMemoryCell(dim=DIM, dim_head=DH, heads=HEADS, omega_window=E)
    with torch.no_grad():   # non-trivial gate heads (zero-weight init makes every gate constant)
        for p in cell.parameters():
            if p.ndim == 2 and p.shape[0] == cell.heads:
                p.normal_(0, 0.05)
    gcell = copy.deepcopy(cell).to(BF16).cuda()
    ref_cell = copy.deepcopy(gcell).cpu().double()    # the same bf16 parameter values, in fp64

    g = torch.Generator().manual_seed(52)
    BH = BATCH * HEADS
    x = torch.randn(BATCH, T, DIM, generator=g).to(BF16)
    st = am.RNNMemState(seq_index=2048, S=(0.05 * torch.randn(BH, DH, DH, generator=g)).to(BF16),
                        Z=(0.05 * torch.randn(BH, DH, DH, generator=g)).to(BF16),
                        omega_buffer=(0.02 * torch.randn(BH, E - 1, DH, DH, generator=g)).to(BF16))
    gy = torch.randn(T, DIM, generator=g)
    gS = torch.randn(HEADS, DH, DH, generator=g)

    xd = x.cuda().requires_grad_()
    out, nst = gcell(xd, am.RNNMemState(st.seq_index, *[t.cuda() for t in st[1:]]))
    assert nst.seq_index == st.seq_index + T
    loss = (out[0].float() * gy.cuda()).sum() + (nst.S[:HEADS].float() * gS.cuda()).sum()
    names = ["x"] + [n for n, _ in gcell.named_parameters()]
    grads = torch.autograd.grad(loss, [xd] + [p for _, p in gcell.named_parameters()])
    torch.cuda.synchronize()
    got = {n: gr.float().cpu() for n, gr in zip(names, grads)}
    got["x"] = got["x"][:1]
    _say("  gpu done; fp64 composition on batch row 0")

    xr = x[:1].to(F64).requires_grad_()
    st_r = am.RNNMemState(st.seq_index, *[t[:HEADS].to(F64) for t in st[1:]])
    out_r, (S_r, Z_r, B_r) = _reference_row(ref_cell, xr, st_r)
    loss_r = (out_r[0] * gy.to(F64)).sum() + (S_r * gS.to(F64)).sum()
    grads_r = torch.autograd.grad(loss_r, [xr] + [p for _, p in ref_cell.named_parameters()])

    compare("cell_c5.out", out[:1].detach().float().cpu(), out_r.detach(), TOL)
    compare("cell_c5.S", nst.S[:HEADS].detach().float().cpu(), S_r.detach(), TOL)
    compare("cell_c5.Z", nst.Z[:HEADS].detach().float().cpu(), Z_r.detach(), TOL)
    compare("cell_c5.buffer", nst.omega_buffer[:HEADS].detach().float().cpu(), B_r.detach(), TOL)
    for n, r in zip(names, grads_r):
        compare(f"cell_c5.d{n}", got[n], r, TOL)
    _say(f"  out, next state and {len(names)} gradients match")
