"""GPU parity of the scan primitives and of the module API against the CPU oracle.

* assoc_scan (atlas_scan_fwd/bwd) vs oracle.scalar_assoc_scan_sequential, values and gradients,
  plus the reference's scan known answers (tests/golden).
* window_sum (atlas_window_sum) vs oracle.sliding_sum_along_time and the reference's
  sliding-sum known answers.
* affine_associative_scan (atlas_affine_scan_fwd/bwd) vs oracle.affine_scan_sequential.
* RNNMemoryCell / OmegaRNNMemoryCell on the GPU vs the reference cell's op sequence
  (rnn_memory.py:250-408, :556-730, :732-814) composed on the CPU in fp64 from the same
  module's prologue layers and the oracle recurrence: outputs, next state and the gradients of
  every parameter and of the input.

Tolerances: fp32 rtol 1e-4, bf16 rtol 2e-2, each with an atol floor of tol * max|ref|.
"""

import copy
import json
import os
import sys

import pytest
import torch
from einops import rearrange

import atlas_rnn_amd as am
from _cases import compare
from oracle import (affine_scan_sequential, memory_recurrence_vectorised, poly_feature_map,
                    scalar_assoc_scan_sequential, sliding_sum_along_time)

pytestmark = pytest.mark.gpu

F64 = torch.float64
BF16 = torch.bfloat16
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _tol(dt):
    return 1e-4 if dt == torch.float32 else 2e-2


# ----------------------------------------------------------------------------- assoc_scan

@pytest.mark.parametrize("name", ["assoc_scan_mixed", "assoc_scan_decay", "assoc_scan_additive"])
def test_assoc_scan_known_answers(name):
    gv = GOLDEN[name]
    _say(f"assoc_scan golden {name}")
    shape = gv["shape"]
    N, T = shape[:2]
    gates = torch.full((N, T), gv["gate"], device="cuda")
    x = torch.full(shape, gv["input"], device="cuda")
    prev = torch.full((N, *shape[2:]), gv["prev"], device="cuda")
    out = am.assoc_scan(gates, x, prev=prev).cpu()
    for t, want in enumerate(gv["expected_per_step"]):
        assert torch.allclose(out[:, t], torch.full_like(out[:, t], want), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dt", [torch.float32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("with_prev,remove_prev", [(False, None), (True, None), (True, False), (True, True)])
def test_assoc_scan_parity(dt, with_prev, remove_prev):
    _say(f"assoc_scan {dt} prev={with_prev} remove_prev={remove_prev}")
    g = torch.Generator().manual_seed(21)
    N, T, shape = 3, 67, (5, 7)
    gates = torch.sigmoid(torch.randn(N, T, generator=g) + 1).to(dt)
    x = torch.randn(N, T, *shape, generator=g).to(dt)
    prev = torch.randn(N, *shape, generator=g).to(dt) if with_prev else None
    T_out = T + (1 if (with_prev and remove_prev is False) else 0)
    gout = torch.randn(N, T_out, *shape, generator=g)
    # oracle: fp64 on the rounded inputs
    ins = [t.to(F64).requires_grad_() if t is not None else None for t in (gates, x, prev)]
    ref = scalar_assoc_scan_sequential(ins[0], ins[1], prev=ins[2], remove_prev=remove_prev)
    rg = torch.autograd.grad((ref * gout.to(F64)).sum(), [t for t in ins if t is not None])
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (gates, x, prev)]
    out = am.assoc_scan(dev[0], dev[1], prev=dev[2], remove_prev=remove_prev)
    assert out.shape == ref.shape and out.dtype == dt
    gg = torch.autograd.grad((out.float() * gout.cuda()).sum(), [t for t in dev if t is not None])
    tol = _tol(dt)
    compare("scan.out", out.float().cpu(), ref.detach(), tol)
    for nm, a, b in zip(("dgates", "dx", "dprev"), gg, rg):
        compare(f"scan.{nm}", a.float().cpu(), b, tol)


def test_assoc_scan_module_and_broadcast_gates():
    _say("AssocScan module, gates [N, T, 1, 1]")
    g = torch.Generator().manual_seed(22)
    gates = torch.rand(2, 9, 1, 1, generator=g)
    x = torch.randn(2, 9, 3, 4, generator=g)
    ref = scalar_assoc_scan_sequential(gates.to(F64), x.to(F64))
    out = am.AssocScan(use_accelerated=False)(gates.cuda(), x.cuda())
    compare("AssocScan", out.cpu(), ref, 1e-4)


# ----------------------------------------------------------------------------- window sum

def test_window_sum_known_answers():
    _say("window_sum golden")
    gv = GOLDEN["sliding_sum_1_to_6_w3"]
    x = torch.tensor(gv["x"], dtype=torch.float32, device="cuda").view(1, -1, 1)
    assert am.window_sum(x, gv["window"]).view(-1).cpu().tolist() == gv["expected"]
    gv = GOLDEN["sliding_sum_2x4x2"]
    x = torch.tensor(gv["x"], dtype=torch.float32, device="cuda")
    for w, want in gv["expected"].items():
        assert am.window_sum(x, int(w)).cpu().tolist() == want


@pytest.mark.parametrize("dt", [torch.float32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("window", [1, 2, 5, 16, 200])
def test_window_sum_parity(dt, window):
    _say(f"window_sum {dt} w={window}")
    g = torch.Generator().manual_seed(23 + window)
    x = torch.randn(3, 90, 4, 6, generator=g).to(dt)
    gy = torch.randn(3, 90, 4, 6, generator=g)
    xr = x.to(F64).requires_grad_()
    ref = sliding_sum_along_time(xr, window)
    (rgx,) = torch.autograd.grad((ref * gy.to(F64)).sum(), [xr])
    xd = x.cuda().requires_grad_()
    out = am.window_sum(xd, window)
    (gx,) = torch.autograd.grad((out.float() * gy.cuda()).sum(), [xd])
    compare("window.out", out.float().cpu(), ref.detach(), _tol(dt))
    compare("window.dx", gx.float().cpu(), rgx, _tol(dt))
    # the omega.py name of the same primitive
    from atlas_rnn_amd.omega import _sliding_sum_along_n
    assert torch.equal(_sliding_sum_along_n(x.cuda(), window), out.detach())


# ----------------------------------------------------------------------------- affine scan

@pytest.mark.parametrize("N,T,R,D,with_prev,remove_prev", [
    (3, 50, 16, 32, True, False),
    (2, 33, 64, 64, True, True),
    (4, 1, 5, 7, False, False),
    (1, 129, 1, 64, True, False),
    # chunks of 64 steps, 16 chunks: the compose / chain / apply passes at full tile size
    (2, 1024, 64, 64, True, False),
    # sizes off the 16-wide tiles, a ragged last chunk, no prev
    (3, 301, 20, 50, False, False),
])
def test_affine_scan_parity(N, T, R, D, with_prev, remove_prev):
    _say(f"affine scan N={N} T={T} R={R} D={D} prev={with_prev} remove_prev={remove_prev}")
    g = torch.Generator().manual_seed(N * 1000 + T)
    A = 0.95 * torch.eye(D) + 0.3 * torch.randn(N, T, D, D, generator=g) / D ** 0.5
    B = torch.randn(N, T, R, D, generator=g)
    prev = torch.randn(N, R, D, generator=g) if with_prev else None
    T_out = T + (1 if (with_prev and not remove_prev) else 0)
    gout = torch.randn(N, T_out, R, D, generator=g)
    ins = [t.to(F64).requires_grad_() if t is not None else None for t in (A, B, prev)]
    ref = affine_scan_sequential(ins[0], ins[1], prev=ins[2], remove_prev=remove_prev)
    rg = torch.autograd.grad((ref * gout.to(F64)).sum(), [t for t in ins if t is not None])
    dev = [t.cuda().requires_grad_() if t is not None else None for t in (A, B, prev)]
    out = am.affine_associative_scan(dev[0], dev[1], prev=dev[2], remove_prev=remove_prev)
    assert out.shape == ref.shape
    gg = torch.autograd.grad((out * gout.cuda()).sum(), [t for t in dev if t is not None])
    compare("affine.out", out.detach().cpu(), ref.detach(), 1e-4)
    for nm, a, b in zip(("dA", "dB", "dprev"), gg, rg):
        compare(f"affine.{nm}", a.cpu(), b, 1e-4)


# ----------------------------------------------------------------------------- module API

def _ste_bf16(t):
    """Round to bf16 in the forward, identity in the backward (as a .to(bfloat16) cast is)."""
    return t + (t.to(BF16).to(t.dtype) - t).detach()


def _reference_cell_forward(cell, x, state):
    """The reference cell forward (rnn_memory.py:250-408 / :556-730, and :732-814 when the cell
    runs the window-16 kernel path), composed from `cell`'s own prologue layers and the oracle
    recurrence. `cell` is a float64 CPU copy."""
    batch, T, _ = x.shape
    x_act = cell.activation(cell.pre_norm(x))
    q_in = k_in = v_in = x_act
    if cell.q_conv is not None:
        q_in = cell.q_conv(q_in.transpose(1, 2)).transpose(1, 2)
        k_in = cell.k_conv(k_in.transpose(1, 2)).transpose(1, 2)
        v_in = cell.v_conv(v_in.transpose(1, 2)).transpose(1, 2)
    q = cell.split_heads(cell.to_q(q_in))[:, :, :T]
    k = cell.split_heads(cell.to_k(k_in))[:, :, :T]
    v = cell.split_heads(cell.to_v(v_in))[:, :, :T]
    q, k = cell.q_norm(q), cell.k_norm(k)
    fm = cell.phi   # the oracle's feature map with the cell's own projection buffer
    phi = lambda t: poly_feature_map(t, fm.degree, fm.mode, getattr(fm, 'proj', None))
    phi_k = rearrange(phi(rearrange(k, 'b h n d -> (b h n) d')), '(b h n) d -> (b h) n d', b=batch,
                      h=cell.heads, n=T)
    phi_q = rearrange(phi(rearrange(q, 'b h n d -> (b h n) d')), '(b h n) d -> (b h) n d', b=batch,
                      h=cell.heads, n=T)
    v = rearrange(v, 'b h n d -> (b h) n d')
    lr = rearrange(cell.to_lr(x_act), 'b n h -> (b h) n')
    decay = rearrange(cell.to_decay(x_act), 'b n h -> (b h) n')
    beta = rearrange(cell.to_momentum(x_act), 'b n h -> (b h) n') if cell.use_momentum else None
    gate = None
    if getattr(cell, 'use_omega_gate', None):
        gate = rearrange(cell.to_omega_gate(x_act), 'b n h -> (b h) n')
    e = cell.omega_window
    chunk = cell.scan_chunk_len if (cell.scan_chunk_len is not None and T > cell.scan_chunk_len) else None
    if getattr(cell, 'use_cuda', False) and cell.cuda_available:
        # window-16 kernel path: bf16 operands, beta/gate default 1, no clamp, empty window per chunk
        beta = beta if beta is not None else torch.ones_like(lr)
        gate = gate if gate is not None else torch.ones_like(lr)
        ops = [_ste_bf16(t) for t in (phi_k, phi_q, v, lr, decay, beta, gate)]
        S_ref = _ste_bf16(state.S)
        # the next chunk starts from the returned Z only with momentum; otherwise the reference's
        # state carries Z = None and each chunk starts from zeros (rnn_memory.py:781, :810)
        zeros = torch.zeros_like(state.S)
        S = state.S
        Z = state.Z if (cell.use_momentum and state.Z is not None) else zeros
        ys = []
        step = chunk or T
        for s0 in range(0, T, step):
            sl = slice(s0, min(T, s0 + step))
            y, S, Z_T, _ = memory_recurrence_vectorised(*[o[:, sl] for o in ops], S_ref, _ste_bf16(S),
                                                        _ste_bf16(Z), None, window=16, clamp_final=False)
            Z = Z_T if cell.use_momentum else zeros
            ys.append(y)
        y = torch.cat(ys, dim=1)
        Z = Z if cell.use_momentum else None
        buf = None
    else:
        Z0 = state.Z if cell.use_momentum else None
        buf = state.omega_buffer if e > 1 else None
        y, S, Z, buf = memory_recurrence_vectorised(phi_k, phi_q, v, lr, decay, beta, gate, state.S, state.S, Z0,
                                                    buf, window=e, clamp_every=chunk, clamp_final=True)
    y = rearrange(y, '(b h) t d -> b h t d', b=batch, h=cell.heads)
    out = cell.to_out(cell.merge_heads(y))
    return out, (S, Z, buf)


CELLS = [
    ("titans", dict(kind="titans", dim=64, dim_head=32, heads=2), 70, None),
    ("titans_nomom_chunk32", dict(kind="titans", dim=48, dim_head=16, heads=3, use_momentum=False,
                                  scan_chunk_len=32), 75, None),
    ("omega_w4", dict(kind="omega", dim=64, dim_head=32, heads=2, omega_window=4), 70, None),
    ("omega_w3_chunk16_map2", dict(kind="omega", dim=32, dim_head=32, heads=1, omega_window=3, poly_degree=2,
                                   poly_mode='elementwise', scan_chunk_len=16), 50, None),
    ("omega_tensor_map_nogate", dict(kind="omega", dim=32, dim_head=16, heads=2, omega_window=2,
                                     use_omega_gate=False, poly_degree=2, poly_mode='tensor',
                                     qkv_conv_kernel=None), 40, None),
    ("omega_cuda_w16_chunk32", dict(kind="omega", dim=64, dim_head=64, heads=1, omega_window=16, use_cuda=True,
                                    scan_chunk_len=32), 80, BF16),
    # without momentum every scan chunk of the window-16 path starts from Z = 0
    ("omega_cuda_w16_nomom_chunk32", dict(kind="omega", dim=64, dim_head=64, heads=1, omega_window=16,
                                          use_cuda=True, use_momentum=False, scan_chunk_len=32), 80, BF16),
]


def _make_cell(spec):
    spec = dict(spec)
    kind = spec.pop("kind")
    cls = am.RNNMemoryCell if kind == "titans" else am.OmegaRNNMemoryCell
    return cls(**spec)


@pytest.mark.parametrize("name,spec,T,kernel_dt", CELLS, ids=[c[0] for c in CELLS])
def test_cell_parity(name, spec, T, kernel_dt):
    _say(f"cell {name}: T={T} {spec}")
    torch.manual_seed(31)
    cell = _make_cell(spec)
    # non-trivial gate heads (their zero-weight init would make every gate constant)
    with torch.no_grad():
        for p in cell.parameters():
            if p.ndim == 2 and p.shape[0] == cell.heads:
                p.normal_(0, 0.2)
    batch = 2
    g = torch.Generator().manual_seed(32)
    x = torch.randn(batch, T, cell.dim, generator=g)
    st = cell.init_state(batch)
    BH, d = batch * cell.heads, cell.dim_head
    # a non-zero carried state
    st = am.RNNMemState(seq_index=3, S=0.05 * torch.randn(BH, d, d, generator=g),
                        Z=0.05 * torch.randn(BH, d, d, generator=g) if st.Z is not None else None,
                        omega_buffer=0.02 * torch.randn(*st.omega_buffer.shape, generator=g)
                        if st.omega_buffer is not None else None)
    if kernel_dt is not None:
        st = am.RNNMemState(3, st.S, st.Z, None)
    gy = torch.randn(batch, T, cell.dim, generator=g)
    gS = torch.randn(BH, d, d, generator=g)

    ref_cell = copy.deepcopy(cell).double()
    xr = x.to(F64).requires_grad_()
    st_r = am.RNNMemState(st.seq_index, *[t.to(F64) if t is not None else None for t in st[1:]])
    out_r, (S_r, Z_r, B_r) = _reference_cell_forward(ref_cell, xr, st_r)
    loss_r = (out_r * gy.to(F64)).sum() + (S_r * gS.to(F64)).sum()
    params_r = [p for _, p in ref_cell.named_parameters()]
    grads_r = torch.autograd.grad(loss_r, [xr] + params_r)

    gcell = copy.deepcopy(cell).cuda()
    xd = x.cuda().requires_grad_()
    st_d = am.RNNMemState(st.seq_index, *[t.cuda() if t is not None else None for t in st[1:]])
    out, nst = gcell(xd, st_d)
    assert nst.seq_index == st.seq_index + T
    loss = (out.float() * gy.cuda()).sum() + (nst.S.float() * gS.cuda()).sum()
    params = [p for _, p in gcell.named_parameters()]
    grads = torch.autograd.grad(loss, [xd] + params)
    torch.cuda.synchronize()

    tol = _tol(kernel_dt or torch.float32)
    compare(f"{name}.out", out.detach().float().cpu(), out_r.detach(), tol)
    compare(f"{name}.S", nst.S.detach().float().cpu(), S_r.detach(), tol)
    if Z_r is not None:
        compare(f"{name}.Z", nst.Z.detach().float().cpu(), Z_r.detach(), tol)
    if B_r is not None:
        compare(f"{name}.buffer", nst.omega_buffer.detach().float().cpu(), B_r.detach(), tol)
    else:
        assert nst.omega_buffer is None
    names = ["x"] + [n for n, _ in gcell.named_parameters()]
    for n, a, b in zip(names, grads, grads_r):
        compare(f"{name}.d{n}", a.float().cpu(), b, tol)


@pytest.mark.parametrize("name,spec", [CELLS[0][:2], CELLS[2][:2]], ids=[CELLS[0][0], CELLS[2][0]])
def test_cell_decode_steps(name, spec):
    """Generation: the cell called one token at a time without autograd (the decode step kernel)
    carries its state like the reference cell called the same way."""
    _say(f"cell decode {name}: {spec}")
    torch.manual_seed(33)
    cell = _make_cell(spec)
    with torch.no_grad():
        for p in cell.parameters():
            if p.ndim == 2 and p.shape[0] == cell.heads:
                p.normal_(0, 0.2)
    batch, steps = 2, 6
    g = torch.Generator().manual_seed(34)
    x = torch.randn(batch, steps, cell.dim, generator=g)
    ref_cell = copy.deepcopy(cell).double()
    gcell = copy.deepcopy(cell).cuda()
    st_r = ref_cell.init_state(batch)
    st_r = am.RNNMemState(st_r.seq_index, *[t.to(F64) if t is not None else None for t in st_r[1:]])
    st_d = gcell.init_state(batch)
    st_d = am.RNNMemState(st_d.seq_index, *[t.cuda() if t is not None else None for t in st_d[1:]])
    with torch.no_grad():
        for t in range(steps):
            out_r, (S_r, Z_r, B_r) = _reference_cell_forward(ref_cell, x[:, t:t + 1].to(F64), st_r)
            st_r = am.RNNMemState(st_r.seq_index + 1, S_r, Z_r, B_r)
            out, st_d = gcell(x[:, t:t + 1].cuda(), st_d)
            compare(f"{name}.out[{t}]", out.float().cpu(), out_r, 1e-4)
    torch.cuda.synchronize()
    compare(f"{name}.S", st_d.S.float().cpu(), st_r.S, 1e-4)
    if st_r.Z is not None:
        compare(f"{name}.Z", st_d.Z.float().cpu(), st_r.Z, 1e-4)
    if st_r.omega_buffer is not None:
        compare(f"{name}.buffer", st_d.omega_buffer.float().cpu(), st_r.omega_buffer, 1e-4)


@pytest.mark.parametrize("spec", [dict(kind="omega", dim=128, dim_head=64, heads=2, omega_window=4, scan_chunk_len=64),
                                  dict(kind="titans", dim=64, dim_head=32, heads=2)],
                         ids=["omega_w4_chunk64", "titans"])
def test_cell_fresh_state_matches_explicit_zero_state(spec):
    """cell(x) with no state passes its zero Z and omega buffer as absent (the specialised walks);
    cell(x, cell.init_state(b)) passes them as tensors (the general kernels). Outputs, next states
    and parameter gradients agree (fp32: rtol 1e-4; the explicit zero-state path is the one the
    oracle pins in test_cell_parity)."""
    _say(f"cell fresh state vs zero state: {spec}")
    torch.manual_seed(41)
    cell = _make_cell(spec).cuda()
    with torch.no_grad():
        for p in cell.parameters():
            if p.ndim == 2 and p.shape[0] == cell.heads:
                p.normal_(0, 0.2)
    g = torch.Generator().manual_seed(42)
    x = torch.randn(2, 300, cell.dim, generator=g).cuda()
    gy = torch.randn(2, 300, cell.dim, generator=g).cuda()
    res = []
    for state in (None, cell.init_state(2)):
        out, st = cell(x, state)
        grads = torch.autograd.grad((out * gy).sum(), list(cell.parameters()))
        res.append((out, st, grads))
    torch.cuda.synchronize()
    (o1, s1, g1), (o2, s2, g2) = res
    compare("fresh.out", o1.detach().cpu(), o2.detach().cpu().double(), 1e-4)
    for a, b in zip(s1[1:], s2[1:]):
        if a is None:
            assert b is None
            continue
        compare("fresh.state", a.cpu(), b.cpu().double(), 1e-4)
    for (n, _), a, b in zip(cell.named_parameters(), g1, g2):
        compare(f"fresh.d{n}", a.cpu(), b.cpu().double(), 1e-4)
