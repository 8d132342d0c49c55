"""Autograd functions over libatlas_mem.so.

* `memory_recurrence(...)`: the memory-layer recurrence of the Titans/OmegaNet RNN cells
  (atlas_pytorch/rnn_memory.py:300-406 and :605-730), forward and backward on the GPU.
* `AtlasOmegaFunction` / `atlas_omega_forward`: drop-in for the reference's CUDA autograd
  function (atlas_pytorch/cuda/atlas_omega_autograd.py:87-211): window 16, per-token gate,
  no buffer, no clamp.
* `assoc_scan` / `window_sum`: the scalar-gated scan and window sum primitives.

Every op requires ROCm GPU tensors and raises on CPU tensors; there is no fallback path.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib

_DTYPES = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16}
_KERNEL_DIMS = (32, 64)       # head dims the kernels are compiled for; smaller ones are zero-padded


def _ptr(t: Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device):
    """The current HIP stream of device as a raw handle (the raw query costs ~0.1 us of host time
    against ~2 us for building torch's Stream object; every library call passes one)."""
    if _RAW_STREAM is not None:
        return ctypes.c_void_p(_RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*ts: Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("atlas_rnn_amd runs on ROCm GPU tensors only (got a CPU tensor); "
                               "there is no CPU implementation in the product path")
        dev = t.device if dev is None else dev
    if dev is None:
        raise RuntimeError("no tensor inputs")
    return dev


def check_operands(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, *, window: int,
                   dtype: torch.dtype | None = None, contiguous: bool = False) -> None:
    """Raises ValueError unless the recurrence operands have consistent shapes, one device and
    (when given) the input dtype, before any pointer reaches the C ABI:
    k, q [BH, T, d_k]; v [BH, T, d_v]; lr, decay, beta [BH, T]; gate [BH, T] (per token) or
    [BH, T, window] (per lag); S_ref, S0, Z0 [BH, d_v, d_k]; buffer [BH, window - 1, d_v, d_k]
    (fp32 states). contiguous=True also requires row-major storage (the raw-pointer calls)."""
    if k.dim() != 3:
        raise ValueError(f"k must be [BH, T, d_k], got shape {tuple(k.shape)}")
    bh, T, dk = k.shape
    if v.dim() != 3 or v.shape[:2] != (bh, T):
        raise ValueError(f"v must be [BH={bh}, T={T}, d_v], got {tuple(v.shape)}")
    dv = v.shape[2]
    if tuple(q.shape) != (bh, T, dk):
        raise ValueError(f"q must have k's shape {(bh, T, dk)}, got {tuple(q.shape)}")
    if not 1 <= window:
        raise ValueError(f"window must be >= 1, got {window}")
    expect = {"lr": (lr, (bh, T)), "decay": (decay, (bh, T)), "beta": (beta, (bh, T)),
              "S_ref": (S_ref, (bh, dv, dk)), "S0": (S0, (bh, dv, dk)), "Z0": (Z0, (bh, dv, dk)),
              "buffer": (buffer if window > 1 else None, (bh, window - 1, dv, dk))}
    if gate is not None:
        if gate.dim() == 2:
            expect["gate"] = (gate, (bh, T))
        elif gate.dim() == 3:
            expect["gate"] = (gate, (bh, T, window))
        else:
            raise ValueError(f"gate must be [BH, T] (per token) or [BH, T, window] (per lag), got {tuple(gate.shape)}")
    for name, (t, shape) in expect.items():
        if t is not None and tuple(t.shape) != shape:
            raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    dev = k.device
    named = dict(k=k, q=q, v=v, lr=lr, decay=decay, beta=beta, gate=gate, S_ref=S_ref, S0=S0, Z0=Z0, buffer=buffer)
    for name, t in named.items():
        if t is None:
            continue
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, k on {dev}")
        if contiguous and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if dtype is not None:
            want = dtype if name in ("k", "q", "v", "lr", "decay", "beta", "gate") else torch.float32
            if t.dtype != want:
                raise ValueError(f"{name} must be {want}, got {t.dtype}")


@dataclass(frozen=True)
class RecurrenceConfig:
    window: int = 1
    map_mode: str = 'off'         # 'off' | 'elementwise'
    map_degree: int = 1
    clamp_every: int | None = None
    clamp_final: bool = True


def _problem(cfg: RecurrenceConfig, bh, T, dk, dv, momentum, gate, has_buffer, dtype) -> _lib.Problem:
    p = _lib.Problem()
    p.abi_version = _lib.ABI_VERSION
    p.bh, p.seq_len, p.d_k, p.d_v = bh, T, dk, dv
    p.window = cfg.window
    p.momentum = int(momentum)
    if gate is None:
        p.gate_mode = _lib.GATE_NONE
    else:
        p.gate_mode = _lib.GATE_TOKEN if gate.dim() == 2 else _lib.GATE_LAG
    elementwise = cfg.map_mode == 'elementwise' and cfg.map_degree > 1
    p.map_mode = _lib.MAP_ELEMENTWISE if elementwise else _lib.MAP_OFF
    p.map_degree = cfg.map_degree if elementwise else 1
    p.has_buffer = int(has_buffer)
    p.clamp_every = int(cfg.clamp_every or 0)
    p.clamp_final = int(cfg.clamp_final)
    p.dtype = _DTYPES[dtype]
    return p


class MemoryRecurrenceFn(torch.autograd.Function):
    """y, S_T, Z_T, buffer_out = recurrence(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer).

    k, q, v, lr, decay, beta, gate: same dtype (fp32 or bf16), contiguous; states fp32.
    Z_T / buffer_out are empty tensors when momentum is off / window == 1.
    """

    @staticmethod
    def forward(ctx, k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf, cfg: RecurrenceConfig):
        # outputs a loss does not use get no gradient tensor (the kernels treat a missing dS_T,
        # dZ_T or buffer_out gradient as zero without reading one)
        ctx.set_materialize_grads(False)
        lib = _lib.load()
        check_operands(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf, window=cfg.window, dtype=k.dtype,
                       contiguous=True)
        bh, T, dk = k.shape
        dv = v.shape[-1]
        momentum = beta is not None
        prob = _problem(cfg, bh, T, dk, dv, momentum, gate, buf is not None, k.dtype)
        _lib.check(lib.atlas_mem_validate(ctypes.byref(prob)), "atlas_mem_validate")
        dev = k.device
        y = torch.empty(bh, T, dv, device=dev, dtype=k.dtype)
        S_T = torch.empty(bh, dv, dk, device=dev, dtype=torch.float32)
        Z_T = torch.empty(bh, dv, dk, device=dev, dtype=torch.float32) if momentum else None
        e = cfg.window
        buf_out = torch.empty(bh, e - 1, dv, dk, device=dev, dtype=torch.float32) if e > 1 else None
        # segment-start states and aggregates: the forward writes them (it needs them for its own
        # second pass) and the backward re-reads them
        nbytes = lib.atlas_mem_saved_bytes(ctypes.byref(prob))
        saved = torch.empty(nbytes // 4, device=dev, dtype=torch.float32)
        a = _lib.FwdArgs(k=_ptr(k), q=_ptr(q), v=_ptr(v), lr=_ptr(lr), decay=_ptr(decay), beta=_ptr(beta),
                         gate=_ptr(gate), S_ref=_ptr(S_ref), S0=_ptr(S0), Z0=_ptr(Z0), buffer_in=_ptr(buf),
                         y=_ptr(y), S_T=_ptr(S_T), Z_T=_ptr(Z_T), buffer_out=_ptr(buf_out))
        _lib.check(lib.atlas_mem_fwd(ctypes.byref(prob), ctypes.byref(a), _ptr(saved), _stream(dev)), "atlas_mem_fwd")
        ctx.cfg = cfg
        ctx.prob = prob
        ctx.momentum = momentum
        ctx.save_for_backward(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf, saved)
        empty = torch.empty(0, device=dev)
        return y, S_T, (Z_T if Z_T is not None else empty), (buf_out if buf_out is not None else empty)

    @staticmethod
    def backward(ctx, dy, dS_T, dZ_T, dbuf_out):
        lib = _lib.load()
        k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf, saved = ctx.saved_tensors
        prob = ctx.prob
        dev = k.device
        bh, T, dk = k.shape
        dv_ = v.shape[-1]
        f32 = torch.float32
        dy = _aligned(dy.to(k.dtype)) if dy is not None else None
        dS_T = _aligned(dS_T.float()) if dS_T is not None else None
        dZ_T = _aligned(dZ_T.float()) if (dZ_T is not None and ctx.momentum and dZ_T.numel() > 0) else None
        dbuf_out = _aligned(dbuf_out.float()) if (dbuf_out is not None and dbuf_out.numel() > 0) else None
        dk_ = torch.empty_like(k)
        dq_ = torch.empty_like(q)
        dv_t = torch.empty_like(v)
        dlr = torch.empty_like(lr)
        ddecay = torch.empty_like(decay)
        dbeta = torch.empty_like(beta) if beta is not None else None
        dgate = torch.empty_like(gate) if gate is not None else None
        dS_ref = torch.empty(bh, dv_, dk, device=dev, dtype=f32)
        dS0 = torch.empty(bh, dv_, dk, device=dev, dtype=f32)
        dZ0 = torch.empty(bh, dv_, dk, device=dev, dtype=f32) if ctx.momentum else None
        dbuf_in = torch.empty_like(buf) if buf is not None else None
        ws_bytes = lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(prob))
        ws = torch.empty((ws_bytes + 3) // 4, device=dev, dtype=f32)
        a = _lib.BwdArgs(k=_ptr(k), q=_ptr(q), v=_ptr(v), lr=_ptr(lr), decay=_ptr(decay), beta=_ptr(beta),
                         gate=_ptr(gate), S_ref=_ptr(S_ref), S0=_ptr(S0), Z0=_ptr(Z0), buffer_in=_ptr(buf),
                         dy=_ptr(dy), dS_T=_ptr(dS_T), dZ_T=_ptr(dZ_T), dbuffer_out=_ptr(dbuf_out),
                         dk=_ptr(dk_), dq=_ptr(dq_), dv=_ptr(dv_t), dlr=_ptr(dlr), ddecay=_ptr(ddecay),
                         dbeta=_ptr(dbeta), dgate=_ptr(dgate), dS_ref=_ptr(dS_ref), dS0=_ptr(dS0),
                         dZ0=_ptr(dZ0), dbuffer_in=_ptr(dbuf_in))
        _lib.check(lib.atlas_mem_bwd(ctypes.byref(prob), ctypes.byref(a), _ptr(saved), _ptr(ws),
                                     ctypes.c_size_t(ws_bytes), _stream(dev)), "atlas_mem_bwd")
        return (dk_, dq_, dv_t, dlr, ddecay, dbeta, dgate, dS_ref, dS0,
                dZ0 if Z0 is not None else None, dbuf_in, None)


def _aligned(x: Tensor | None) -> Tensor | None:
    """x contiguous with a 16-byte aligned start (the C ABI rejects other pointers)."""
    if x is None:
        return None
    x = x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _canon(x: Tensor | None, dtype) -> Tensor | None:
    return None if x is None else _aligned(x.to(dtype))


# ---------------------------------------------------------------------------------------------
# Tensor polynomial feature map (rnn_memory.py:125-130): [x; vec(x x^T)] @ P, fused on the GPU
# ---------------------------------------------------------------------------------------------

_TMAP_DIN = (16, 32, 64)
_TMAP_DOUT = tuple(range(16, 129, 16))


def _tmap_check(x: Tensor, proj: Tensor, degree: int) -> None:
    """Raises for operands the kernels do not take (no other implementation exists)."""
    d, m = x.shape[-1], proj.shape[-1]
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"tensor_feature_map: dtype {x.dtype} (the kernels take bfloat16 or float32)")
    if d not in _TMAP_DIN or m not in _TMAP_DOUT:
        raise ValueError(f"tensor_feature_map: d_in {d} / d_out {m} (the kernels take d_in in {_TMAP_DIN}, "
                         "d_out a multiple of 16 up to 128)")
    if tuple(proj.shape) != (d + d * d, m):
        raise ValueError(f"tensor_feature_map: proj {tuple(proj.shape)}, expected ({d + d * d}, {m})")
    if proj.requires_grad:
        raise NotImplementedError("tensor_feature_map: proj is a constant (a registered buffer in the reference); "
                                  "the kernels form no gradient for it")
    if not 1 <= int(degree) <= 16:
        raise ValueError(f"tensor_feature_map: degree {degree} (1 .. 16)")


def symmetrized_tables(proj: Tensor, d: int, dtype) -> tuple[Tensor, Tensor]:
    """The symmetrised table of proj [d + d*d, m] in both layouts, in `dtype`
    (atlas_tensor_map_symmetrize: one launch in place of a transposition; the forward and the
    backward skip the products over its zero lower triangle). x x^T is symmetric, so
    [x; vec(x x^T)] proj = [x; vec(x x^T)] P' with P'[a][b] = proj[a][b] + proj[b][a] above the
    diagonal, proj[a][a] on it and zeros below. Nothing is cached here: the owner of proj keeps the
    tables (PolynomialFeatureMap does, per dtype and device) and passes them to tensor_feature_map."""
    lib = _lib.load()
    dev = proj.device
    m = proj.shape[1]
    p = _aligned(proj.detach().to(dtype))
    ps = torch.empty_like(p)
    pst = torch.empty(m, p.shape[0], device=dev, dtype=p.dtype)
    _lib.check(lib.atlas_tensor_map_symmetrize(_dt_code(p), d, m, _ptr(p), _ptr(ps), _ptr(pst), _stream(dev)),
               "atlas_tensor_map_symmetrize")
    return ps, pst


class _TensorMapFn(torch.autograd.Function):
    """atlas_tensor_map_fwd / _bwd: x [n, d] and P [d + d*d, m] (bf16 or fp32, P in x's dtype as the
    reference casts it) -> phi [n, m], followed by the elementwise polynomial of `degree` (1: none);
    P is a constant (a registered buffer in the reference, so it has no gradient)."""

    @staticmethod
    def forward(ctx, x, proj, degree, tables=None):
        dev = _require_gpu(x, proj)
        lib = _lib.load()
        lead, d, m = x.shape[:-1], x.shape[-1], proj.shape[-1]
        x2 = _aligned(x.reshape(-1, d))
        ps, pst = tables if tables is not None else symmetrized_tables(proj, d, x.dtype)
        n = x2.shape[0]
        out = torch.empty(n, m, device=dev, dtype=x.dtype)
        pre = torch.empty(n, m, device=dev, dtype=x.dtype) if degree > 1 else None
        _lib.check(lib.atlas_tensor_map_fwd_sym(_dt_code(x2), n, d, m, degree, _ptr(x2), _ptr(pst), _ptr(out),
                                                _ptr(pre), _stream(dev)), "atlas_tensor_map_fwd_sym")
        p = ps
        ctx.save_for_backward(x2, p, pre)
        ctx.lead = lead
        ctx.degree = degree
        return out.reshape(*lead, m)

    @staticmethod
    def backward(ctx, dout):
        x2, p, pre = ctx.saved_tensors
        dev = x2.device
        lib = _lib.load()
        n, d = x2.shape
        m = p.shape[-1]
        g = _aligned(dout.reshape(-1, m).to(x2.dtype))
        dx = torch.empty_like(x2)
        _lib.check(lib.atlas_tensor_map_bwd_sym(_dt_code(x2), n, d, m, ctx.degree, _ptr(x2), _ptr(p), _ptr(pre),
                                                _ptr(g), _ptr(dx), _stream(dev)), "atlas_tensor_map_bwd_sym")
        return dx.reshape(*ctx.lead, d), None, None, None


def _tables_ok(tables, proj: Tensor, dtype) -> bool:
    ps, pst = tables
    m = proj.shape[-1]
    return (ps.dtype == dtype and pst.dtype == dtype and ps.device == proj.device and pst.device == proj.device
            and tuple(ps.shape) == tuple(proj.shape) and tuple(pst.shape) == (m, proj.shape[0])
            and ps.is_contiguous() and pst.is_contiguous())


def tensor_feature_map(x: Tensor, proj: Tensor, degree: int = 1,
                       tables: tuple[Tensor, Tensor] | None = None) -> Tensor:
    """[x; vec(x x^T)] @ proj (rnn_memory.py:125-130) in x's dtype, then (degree > 1) the elementwise
    polynomial sum_{i=1..degree} phi^i (BASELINE C4's composition), on the fused kernels: the
    Kronecker features are never materialised and the polynomial is applied on the fp32 accumulator.
    x: bf16 or fp32 GPU tensor [..., d], d in (16, 32, 64); proj [d + d*d, m], m a multiple of 16 up
    to 128, constant. Anything else raises (CPU tensors included).
    tables: proj's symmetrised tables in x's dtype (`symmetrized_tables`), when the caller keeps
    them across calls; formed by this call otherwise (one extra launch)."""
    _tmap_check(x, proj, degree)
    if tables is not None and not _tables_ok(tables, proj, x.dtype):
        raise ValueError("tensor_feature_map: tables do not match proj (shape, dtype, device) and x's dtype")
    return _TensorMapFn.apply(x, proj, int(degree), tables)


_BLOCK = 64    # block width of the decomposition for head sizes the kernels are not built for


def _poly_map(x: Tensor, degree: int) -> Tensor:
    """sum_{i=1..degree} x^i in (at least) fp32, rounded back to x's dtype (what the kernels apply
    to each input element before its matrix products)."""
    xf = x.to(torch.promote_types(x.dtype, torch.float32))
    out, pw = xf, xf
    for _ in range(2, degree + 1):
        pw = pw * xf
        out = out + pw
    return out.to(x.dtype)


class _BlockSplitFn(torch.autograd.Function):
    """phi, psi [BH, T, Dk], v [BH, T, Dv], S_ref [BH, Dv, Dk] -> the stacked 64-wide operands of the
    state blocks (atlas_block_split / atlas_block_merge): phi_b, psi_b, nv_b [NB BH, T, 64] with
    nv = v - S_ref phi, block r = (i * Dk/64 + j) * BH + bh."""

    @staticmethod
    def forward(ctx, phi, psi, v, S_ref):
        lib = _lib.load()
        bh, T, dk = phi.shape
        dv = v.shape[-1]
        nb = (dk // _BLOCK) * (dv // _BLOCK)
        phi, psi, v, S_ref = _aligned(phi), _aligned(psi), _aligned(v), _aligned(S_ref.float())
        out = [torch.empty(nb * bh, T, _BLOCK, device=phi.device, dtype=phi.dtype) for _ in range(3)]
        _lib.check(lib.atlas_block_split(_dt_code(phi), bh, T, dk, dv, _ptr(phi), _ptr(psi), _ptr(v), _ptr(S_ref),
                                         _ptr(out[0]), _ptr(out[1]), _ptr(out[2]), _stream(phi.device)),
                   "atlas_block_split")
        ctx.save_for_backward(phi, S_ref)
        ctx.dv = dv
        return tuple(out)

    @staticmethod
    def backward(ctx, dphi_b, dpsi_b, dnv_b):
        lib = _lib.load()
        phi, S_ref = ctx.saved_tensors
        bh, T, dk = phi.shape
        dv = ctx.dv
        z = lambda g: torch.zeros(dk // _BLOCK * (dv // _BLOCK) * bh, T, _BLOCK, device=phi.device,
                                  dtype=phi.dtype) if g is None else _aligned(g.to(phi.dtype))
        dphi_b, dpsi_b, dnv_b = z(dphi_b), z(dpsi_b), z(dnv_b)
        dphi = torch.empty_like(phi)
        dpsi = torch.empty_like(phi)
        dvv = torch.empty(bh, T, dv, device=phi.device, dtype=phi.dtype)
        parts = torch.empty(bh, lib.atlas_block_parts(T), dv, dk, device=phi.device, dtype=torch.float32)
        _lib.check(lib.atlas_block_merge(_dt_code(phi), bh, T, dk, dv, _ptr(phi), _ptr(S_ref), _ptr(dphi_b),
                                         _ptr(dpsi_b), _ptr(dnv_b), _ptr(dphi), _ptr(dpsi), _ptr(dvv), _ptr(parts),
                                         _stream(phi.device)), "atlas_block_merge")
        return dphi, dpsi, dvv, parts.sum(dim=1)


_REPLICATE, _REPLICA_SUM = 0, 1


def _replicas(op: int, nrep: int, xs):
    """atlas_replicas over a list of tensors (one launch per dtype, up to four arrays each):
    _REPLICATE gives [nrep * x.shape[0], ...] (x repeated along the first axis), _REPLICA_SUM the
    sum of the nrep replicas stacked along the first axis of x."""
    lib = _lib.load()
    xs = [x.contiguous() for x in xs]
    if op == _REPLICA_SUM:
        for x in xs:
            if x.shape[0] % nrep != 0:
                raise ValueError(f"replica sum: first axis {x.shape[0]} is not a multiple of {nrep} replicas")
    outs = [torch.empty(((nrep * x.shape[0]) if op == _REPLICATE else (x.shape[0] // nrep),) + tuple(x.shape[1:]),
                        device=x.device, dtype=x.dtype) for x in xs]
    for dt in {x.dtype for x in xs}:
        idx = [i for i, x in enumerate(xs) if x.dtype == dt]
        for c0 in range(0, len(idx), 4):
            grp = idx[c0:c0 + 4]
            cnt = len(grp)
            n64 = (ctypes.c_int64 * cnt)(*[(xs[i] if op == _REPLICATE else outs[i]).numel() for i in grp])
            vp = ctypes.c_void_p * cnt
            _lib.check(lib.atlas_replicas(op, _DTYPES[dt], cnt, nrep, n64, vp(*[xs[i].data_ptr() for i in grp]),
                                          vp(*[outs[i].data_ptr() for i in grp]), _stream(xs[0].device)),
                       "atlas_replicas")
    return outs


class _ReplicateFn(torch.autograd.Function):
    """Each tensor repeated nrep times along its first axis; the adjoint sums the replicas."""

    @staticmethod
    def forward(ctx, nrep, *xs):
        ctx.nrep = nrep
        return tuple(_replicas(_REPLICATE, nrep, xs))

    @staticmethod
    def backward(ctx, *gs):
        return (None,) + tuple(_replicas(_REPLICA_SUM, ctx.nrep, gs))


class _ReplicaSumFn(torch.autograd.Function):
    """The sum of the nrep replicas stacked along each tensor's first axis; the adjoint repeats."""

    @staticmethod
    def forward(ctx, nrep, *xs):
        ctx.nrep = nrep
        return tuple(_replicas(_REPLICA_SUM, nrep, xs))

    @staticmethod
    def backward(ctx, *gs):
        return (None,) + tuple(_replicas(_REPLICATE, ctx.nrep, gs))


def block_recurrence(k: Tensor, q: Tensor, v: Tensor, lr: Tensor, decay: Tensor,
                     beta: Tensor | None, gate: Tensor | None, S_ref: Tensor, S0: Tensor, Z0: Tensor | None,
                     buffer: Tensor | None, *, window: int, map_mode: str, map_degree: int,
                     clamp_every: int | None, clamp_final: bool):
    """The recurrence for head sizes above 64 or d_k != d_v, as 64 x 64 state blocks.

    With the state split into blocks S[i, j] (rows 64 i .. of d_v, columns 64 j .. of d_k):
      * delta_t = S_ref phi_t - v_t couples the column blocks only through delta, so delta is
        formed once and every block runs the 64-wide recurrence with S_ref = 0 and
        v = -delta[rows of i] (its own delta is then 0 . phi - v = delta);
      * the block's update delta_i phi_j^T, decay, momentum, window and clamp are blockwise;
      * y[rows of i] = sum_j S[i, j] psi_j.
    The blocks are stacked along the head-batch axis ((i, j, bh) order) into ONE call of the
    64-wide kernels; the per-token scalars are shared by all blocks. The column / row blocks of
    phi, psi and v - S_ref phi are formed in one pass by atlas_block_split (its adjoint
    atlas_block_merge); the states are stacked by small copies, the scalars by one launch of
    atlas_replicas (and y summed over the column blocks by another). Head sizes that are not
    a multiple of 64 are zero-padded (the padded rows / columns of every state stay zero).
    """
    bh, T, dk = k.shape
    dv = v.shape[-1]
    nbk, nbv = -(-dk // _BLOCK), -(-dv // _BLOCK)
    Dk, Dv = nbk * _BLOCK, nbv * _BLOCK
    pad_k, pad_v = Dk - dk, Dv - dv
    if Dk > 256 or Dv > 256:
        raise ValueError(f"head sizes up to 256 are supported (got d_k={dk}, d_v={dv})")
    # the elementwise map is applied here (delta needs the mapped keys)
    if map_mode == 'elementwise' and map_degree > 1:
        k, q = _poly_map(k, map_degree), _poly_map(q, map_degree)
    F = torch.nn.functional
    padf = lambda t, pads: t if t is None or not any(pads) else F.pad(t, pads)   # F.pad copies even at 0
    phi, psi = padf(k, (0, pad_k)), padf(q, (0, pad_k))
    vv = padf(v, (0, pad_v))
    pst = lambda t: padf(t, (0, pad_k, 0, pad_v))
    S_ref, S0, Z0, buffer = pst(S_ref), pst(S0), pst(Z0), pst(buffer)
    nb = nbv * nbk
    kb, qb, vb = _BlockSplitFn.apply(phi, psi, vv, S_ref)

    def stack_state(x):        # [BH, ..., Dv, Dk] -> [(i, j, bh), ..., 64, 64]
        if x is None:
            return None
        mid = x.shape[1:-2]
        x = x.reshape(bh, *mid, nbv, _BLOCK, nbk, _BLOCK)
        m = len(mid)
        x = x.permute(m + 1, m + 3, 0, *range(1, m + 1), m + 2, m + 4)
        return x.reshape(nb * bh, *mid, _BLOCK, _BLOCK)

    # the per-token scalars of every block: one replicating launch (its adjoint: one summing launch)
    scal = [t for t in (lr, decay, beta, gate) if t is not None]
    reps = iter(_ReplicateFn.apply(nb, *scal))
    lr_b, decay_b, beta_b, gate_b = [None if t is None else next(reps) for t in (lr, decay, beta, gate)]
    S0b, Z0b, Bb = stack_state(S0), stack_state(Z0), stack_state(buffer)
    Sref0 = torch.zeros_like(S0b)
    y, S_T, Z_T, B = memory_recurrence(kb, qb, vb, lr_b, decay_b, beta_b, gate_b, Sref0, S0b, Z0b, Bb,
                                       window=window, map_mode='off', map_degree=1, clamp_every=clamp_every,
                                       clamp_final=clamp_final)
    # y: sum over the column blocks of each row block (one launch); states: blocks back in place
    if nbv == 1:   # a plain view, so that the adjoint hands the replicated gradient over without a copy
        (y,) = _ReplicaSumFn.apply(nbk, y)
    else:
        yr = _ReplicaSumFn.apply(nbk, *y.reshape(nbv, nbk * bh, T, _BLOCK).unbind(0))
        y = torch.stack(yr, dim=2).reshape(bh, T, Dv)

    def unblock(x):            # [(i, j, bh), ..., 64, 64] -> [bh, ..., Dv, Dk]
        if x is None:
            return None
        mid = x.shape[1:-2]
        m = len(mid)
        x = x.reshape(nbv, nbk, bh, *mid, _BLOCK, _BLOCK)
        x = x.permute(2, *range(3, m + 3), 0, m + 3, 1, m + 4).reshape(bh, *mid, Dv, Dk)
        return x[..., :dv, :dk]

    return y[..., :dv], unblock(S_T), unblock(Z_T), unblock(B)


def _memory_step(cfg: RecurrenceConfig, args, states):
    """One token without autograd (atlas_mem_step): the generation step of
    atlas_pytorch/rnn_transformer.py:863-900 through the cell's recurrence at T = 1."""
    k, q, v, lr, decay, beta, gate = args
    S_ref, S0, Z0, buf = states
    lib = _lib.load()
    bh, _, dk = k.shape
    dv = v.shape[-1]
    dev = k.device
    momentum = beta is not None
    e = cfg.window
    prob = _problem(cfg, bh, 1, dk, dv, momentum, gate, buf is not None, k.dtype)
    y = torch.empty(bh, 1, dv, device=dev, dtype=k.dtype)
    S_T = torch.empty(bh, dv, dk, device=dev, dtype=torch.float32)
    Z_T = torch.empty_like(S_T) if momentum else None
    buf_out = torch.empty(bh, e - 1, dv, dk, device=dev, dtype=torch.float32) if e > 1 else None
    a = _lib.FwdArgs(k=_ptr(k), q=_ptr(q), v=_ptr(v), lr=_ptr(lr), decay=_ptr(decay), beta=_ptr(beta),
                     gate=_ptr(gate), S_ref=_ptr(S_ref), S0=_ptr(S0), Z0=_ptr(Z0), buffer_in=_ptr(buf),
                     y=_ptr(y), S_T=_ptr(S_T), Z_T=_ptr(Z_T), buffer_out=_ptr(buf_out))
    _lib.check(lib.atlas_mem_step(ctypes.byref(prob), ctypes.byref(a), _stream(dev)), "atlas_mem_step")
    return y, S_T, Z_T, buf_out


# ---------------------------------------------------------------------------------------------
# The carried buffer as rank-1 factors (decode): factors [BH, e-1, d_v + d_k] fp32, slot m =
# (g delta | phi) of the token whose product g delta phi^T the dense slot holds
# ---------------------------------------------------------------------------------------------

def _factor_dims(k: Tensor, v: Tensor) -> tuple[int, int, int]:
    if k.dim() != 3 or v.dim() != 3:
        raise ValueError(f"k and v must be [BH, T, d], got {tuple(k.shape)} and {tuple(v.shape)}")
    bh, _, dk = k.shape
    dv = v.shape[-1]
    if dk != dv or dk not in _KERNEL_DIMS:
        raise ValueError(f"the factored buffer takes d_k == d_v in {_KERNEL_DIMS}, got {dk} / {dv}")
    return bh, dk, dv


def _check_factors(factors: Tensor | None, bh: int, window: int, d: int, name: str) -> None:
    if factors is None:
        return
    want = (bh, window - 1, 2 * d)
    if tuple(factors.shape) != want or factors.dtype != torch.float32:
        raise ValueError(f"{name} must be fp32 {want}, got {factors.dtype} {tuple(factors.shape)}")


def memory_step_factored(k: Tensor, q: Tensor, v: Tensor, lr: Tensor, decay: Tensor,
                         beta: Tensor | None = None, gate: Tensor | None = None,
                         S_ref: Tensor | None = None, S0: Tensor | None = None, Z0: Tensor | None = None,
                         factors: Tensor | None = None, *, window: int = 1, map_mode: str = 'off',
                         map_degree: int = 1, clamp_final: bool = True):
    """One decode token (T = 1, no autograd) with the carried buffer as rank-1 factors
    (atlas_mem_step_factored): the recurrence step of memory_recurrence at T = 1
    (rnn_memory.py:659-728, the generation loop of rnn_transformer.py:863-900), reading and writing
    factors [BH, e-1, 2d] instead of the dense [BH, e-1, d, d]. Returns (y [BH, 1, d], S_T,
    Z_T or None, factors_out or None); expand_buffer_factors(factors_out) is the dense buffer_out."""
    dev = _require_gpu(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, factors)
    bh, dk, dv = _factor_dims(k, v)
    if k.shape[1] != 1:
        raise ValueError(f"memory_step_factored takes one token, got T = {k.shape[1]}")
    dt = k.dtype if k.dtype in _DTYPES else torch.float32
    if S0 is None:
        S0 = torch.zeros(bh, dv, dk, device=dev, dtype=torch.float32)
    if S_ref is None:
        S_ref = S0
    check_operands(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, None, window=window)
    _check_factors(factors, bh, window, dk, "factors")
    e = window
    cfg = RecurrenceConfig(window=e, map_mode=map_mode, map_degree=map_degree, clamp_final=clamp_final)
    kk, qq, vv, lr_, dc, bt, gt = [_canon(t, dt) for t in (k, q, v, lr, decay, beta, gate)]
    S_ref_, S0_ = _canon(S_ref, torch.float32), _canon(S0, torch.float32)
    Z0_ = _canon(Z0, torch.float32) if beta is not None else None
    f_in = _canon(factors, torch.float32) if e > 1 else None
    lib = _lib.load()
    prob = _problem(cfg, bh, 1, dk, dv, beta is not None, gt, f_in is not None, dt)
    y = torch.empty(bh, 1, dv, device=dev, dtype=dt)
    S_T = torch.empty(bh, dv, dk, device=dev, dtype=torch.float32)
    Z_T = torch.empty_like(S_T) if beta is not None else None
    f_out = torch.empty(bh, e - 1, dv + dk, device=dev, dtype=torch.float32) if e > 1 else None
    a = _lib.FwdArgs(k=_ptr(kk), q=_ptr(qq), v=_ptr(vv), lr=_ptr(lr_), decay=_ptr(dc), beta=_ptr(bt), gate=_ptr(gt),
                     S_ref=_ptr(S_ref_), S0=_ptr(S0_), Z0=_ptr(Z0_), y=_ptr(y), S_T=_ptr(S_T), Z_T=_ptr(Z_T))
    _lib.check(lib.atlas_mem_step_factored(ctypes.byref(prob), ctypes.byref(a), _ptr(f_in), _ptr(f_out),
                                           _stream(dev)), "atlas_mem_step_factored")
    return y, S_T, Z_T, f_out


def buffer_factors(k: Tensor, v: Tensor, gate: Tensor | None, S_ref: Tensor, factors: Tensor | None = None, *,
                   window: int, map_mode: str = 'off', map_degree: int = 1) -> Tensor:
    """The factored form of the buffer memory_recurrence returns after these T tokens (the last
    e-1 of [factors; tokens], atlas_buffer_factors): prefill -> factored decode state."""
    dev = _require_gpu(k, v, gate, S_ref, factors)
    bh, dk, dv = _factor_dims(k, v)
    if window < 2:
        raise ValueError("the buffer exists for window >= 2")
    T = k.shape[1]
    dt = k.dtype if k.dtype in _DTYPES else torch.float32
    check_operands(k, k, v, v[..., 0], v[..., 0], None, gate, S_ref, S_ref, None, None, window=window)
    _check_factors(factors, bh, window, dk, "factors")
    cfg = RecurrenceConfig(window=window, map_mode=map_mode, map_degree=map_degree)
    kk, vv, gt = [_canon(t, dt) for t in (k, v, gate)]
    S_ref_ = _canon(S_ref, torch.float32)
    f_in = _canon(factors, torch.float32)
    prob = _problem(cfg, bh, T, dk, dv, False, gt, f_in is not None, dt)
    out = torch.empty(bh, window - 1, dv + dk, device=dev, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.atlas_buffer_factors(ctypes.byref(prob), _ptr(kk), _ptr(vv), _ptr(gt), _ptr(S_ref_), _ptr(f_in),
                                        _ptr(out), _stream(dev)), "atlas_buffer_factors")
    return out


def expand_buffer_factors(factors: Tensor, d_v: int | None = None) -> Tensor:
    """factors [BH, e-1, d_v + d_k] -> the dense buffer [BH, e-1, d_v, d_k] (atlas_buffer_expand), the
    RNNMemState.omega_buffer / memory_recurrence buffer format. d_v defaults to half the width."""
    dev = _require_gpu(factors)
    if factors.dim() != 3 or factors.dtype != torch.float32:
        raise ValueError(f"factors must be fp32 [BH, e-1, d_v + d_k], got {factors.dtype} {tuple(factors.shape)}")
    bh, slots, width = factors.shape
    dv = width // 2 if d_v is None else d_v
    dk = width - dv
    if dv < 1 or dk < 1:
        raise ValueError(f"d_v {dv} does not split width {width}")
    f = _aligned(factors)
    out = torch.empty(bh, slots, dv, dk, device=dev, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(lib.atlas_buffer_expand(bh, slots, dv, dk, _ptr(f), _ptr(out), _stream(dev)), "atlas_buffer_expand")
    return out


def memory_recurrence(k: Tensor, q: Tensor, v: Tensor, lr: Tensor, decay: Tensor,
                      beta: Tensor | None = None, gate: Tensor | None = None,
                      S_ref: Tensor | None = None, S0: Tensor | None = None, Z0: Tensor | None = None,
                      buffer: Tensor | None = None, *, window: int = 1, map_mode: str = 'off',
                      map_degree: int = 1, clamp_every: int | None = None, clamp_final: bool = True):
    """Memory-layer recurrence over [BH, T, d] inputs (atlas_pytorch/rnn_memory.py:605-730).

    The kernels are built for d_k == d_v in {32, 64}; smaller equal head sizes are zero-padded,
    and larger or unequal ones (e.g. d_k = 128 after a tensor feature map, d_v = 64) run as
    64 x 64 state blocks through `block_recurrence`.
    k, q: raw keys / queries [BH, T, d_k] (the elementwise polynomial map is applied inside);
    v [BH, T, d_v]; lr (eta), decay (alpha), beta [BH, T]; gate None | [BH, T] (per-token,
    reference omega_gate) | [BH, T, e] (per-lag); S_ref, S0, Z0 [BH, d_v, d_k];
    buffer [BH, e-1, d_v, d_k]. Returns (y [BH,T,d_v] in the input dtype, S_T, Z_T or None,
    buffer_out or None) with fp32 states.
    """
    dev = _require_gpu(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer)
    dt = k.dtype if k.dtype in _DTYPES else torch.float32
    if k.dim() != 3 or v.dim() != 3:
        raise ValueError(f"k and v must be [BH, T, d], got {tuple(k.shape)} and {tuple(v.shape)}")
    bh, T, dk = k.shape
    dv = v.shape[-1]
    if S0 is None:
        S0 = torch.zeros(bh, dv, dk, device=dev, dtype=torch.float32)
    if S_ref is None:
        S_ref = S0
    check_operands(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, window=window)
    if dk != dv or dk > max(_KERNEL_DIMS):
        return block_recurrence(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, window=window,
                                map_mode=map_mode, map_degree=map_degree, clamp_every=clamp_every,
                                clamp_final=clamp_final)
    if dk == dv and dk < 64 and dk not in _KERNEL_DIMS:
        # Zero feature columns leave the recurrence exact: the padded rows / columns of every
        # state stay zero, the padded entries of y are zero and their gradients are dropped.
        D = next(x for x in _KERNEL_DIMS if x > dk)
        pad = D - dk
        pv = lambda t: None if t is None else torch.nn.functional.pad(t, (0, pad))
        pm = lambda t: None if t is None else torch.nn.functional.pad(t, (0, pad, 0, pad))
        y, S_T, Z_T, B = memory_recurrence(pv(k), pv(q), pv(v), lr, decay, beta, gate, pm(S_ref), pm(S0), pm(Z0),
                                           pm(buffer), window=window, map_mode=map_mode, map_degree=map_degree,
                                           clamp_every=clamp_every, clamp_final=clamp_final)
        return (y[..., :dk], S_T[..., :dk, :dk], None if Z_T is None else Z_T[..., :dk, :dk],
                None if B is None else B[..., :dk, :dk])
    e = window
    if clamp_every is not None and clamp_every >= T:
        clamp_every = None        # no clamp point before the last token (the final clamp is clamp_final's)
    cfg = RecurrenceConfig(window=e, map_mode=map_mode, map_degree=map_degree,
                           clamp_every=clamp_every, clamp_final=clamp_final)
    args = [_canon(t, dt) for t in (k, q, v, lr, decay, beta, gate)]
    states = [_canon(t, torch.float32) for t in (S_ref, S0, Z0 if beta is not None else None,
                                                  buffer if e > 1 else None)]
    if T == 1 and not (torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (*args, *states))):
        return _memory_step(cfg, args, states)   # decode: one launch, no saved buffer
    # window - 1 longer than the chunk implied by clamp_every, or clamp_every without a divisor
    # usable as a chunk: run one call per scan chunk (atlas_pytorch/rnn_memory.py:584-601),
    # carrying S, Z and the buffer, S_ref fixed.
    lib = _lib.load()
    prob = _problem(cfg, bh, T, dk, dv, beta is not None, gate, states[3] is not None, dt)
    status = lib.atlas_mem_validate(ctypes.byref(prob))
    if status == _lib.ERR_UNSUPPORTED and clamp_every and T > clamp_every:
        ys = []
        S_ref_f, S, Z, B = states
        for start in range(0, T, clamp_every):
            end = min(T, start + clamp_every)
            sl = slice(start, end)
            y, S, Z, B = memory_recurrence(
                args[0][:, sl], args[1][:, sl], args[2][:, sl], args[3][:, sl], args[4][:, sl],
                args[5][:, sl] if args[5] is not None else None,
                args[6][:, sl] if args[6] is not None else None,
                S_ref_f, S, Z, B, window=e, map_mode=map_mode, map_degree=map_degree,
                clamp_every=None, clamp_final=(end < T) or clamp_final)
            ys.append(y)
        return torch.cat(ys, dim=1), S, Z, B
    _lib.check(status, "atlas_mem_validate")
    y, S_T, Z_T, buf_out = MemoryRecurrenceFn.apply(*args, *states, cfg)
    return y, S_T, (Z_T if beta is not None else None), (buf_out if e > 1 else None)


class AtlasOmegaFunction:
    """Drop-in for atlas_pytorch/cuda/atlas_omega_autograd.py:87-204.

    apply(phi_k, phi_q, v, S_ref, lr, decay, beta, gate, S0, Z0) -> (y, S_T, Z_T): window 16,
    per-token gate, momentum, zero buffer, no clamp. phi_k / phi_q are already feature-mapped.
    Unlike the reference CUDA kernel, alpha and beta are not clamped to >= 1e-4 and states stay
    in fp32 (the PyTorch-path semantics); y and the states are returned in phi_k's dtype.
    """

    WINDOW = 16

    @staticmethod
    def apply(phi_k, phi_q, v, S_ref, lr, decay, beta, gate, S0, Z0):
        y, S_T, Z_T, _ = memory_recurrence(phi_k, phi_q, v, lr, decay, beta, gate, S_ref, S0, Z0, None,
                                           window=AtlasOmegaFunction.WINDOW, clamp_final=False)
        return y, S_T.to(phi_k.dtype), Z_T.to(phi_k.dtype)


def atlas_omega_forward(phi_k, phi_q, v, S_ref, lr, decay, beta, gate, S0, Z0):
    """atlas_pytorch/cuda/atlas_omega_autograd.py:207-211."""
    return AtlasOmegaFunction.apply(phi_k, phi_q, v, S_ref, lr, decay, beta, gate, S0, Z0)


def check_cuda_availability():
    """atlas_pytorch/cuda/atlas_omega_autograd.py:214-228: (available, message)."""
    if not torch.cuda.is_available():
        return False, "no ROCm GPU visible"
    try:
        _lib.load()
    except Exception as exc:  # noqa: BLE001
        return False, f"libatlas_mem.so not loaded: {exc}"
    props = torch.cuda.get_device_properties(0)
    return True, f"atlas_rnn_amd ready (GPU: {props.name}, library: {_lib.LIB_PATH})"


def get_cuda_status() -> dict:
    """atlas_pytorch/cuda/atlas_omega_autograd.py:16-22: the backend's load status for logging, with
    the reference's keys. `available`: libatlas_mem.so is loaded (its ABI version checked);
    `loaded_via`: the library's path, or "none"; `error`: why it could not be loaded ("" when
    available). Touches no GPU (it loads the library only)."""
    try:
        _lib.load()
    except Exception as exc:  # noqa: BLE001
        return {"available": False, "loaded_via": "none", "error": str(exc)}
    return {"available": True, "loaded_via": _lib.LIB_PATH, "error": ""}


# ------------------------------------------------------------------------------------------
# Scan primitives
# ------------------------------------------------------------------------------------------

class _ScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gates, x, prev):
        lib = _lib.load()
        n, t = gates.shape
        d = x.numel() // (n * t)
        out = torch.empty_like(x)
        _lib.check(lib.atlas_scan_fwd(_DTYPES[x.dtype], n, t, d, _ptr(gates), _ptr(x), _ptr(prev), _ptr(out),
                                      _stream(x.device)), "atlas_scan_fwd")
        ctx.save_for_backward(gates, out, prev)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        gates, out, prev = ctx.saved_tensors
        n, t = gates.shape
        d = out.numel() // (n * t)
        dout = dout.contiguous()
        dx = torch.empty_like(out)
        dg = torch.empty_like(gates)
        dprev = torch.empty_like(prev) if prev is not None else None
        _lib.check(lib.atlas_scan_bwd(_DTYPES[out.dtype], n, t, d, _ptr(gates), _ptr(out), _ptr(prev),
                                      _ptr(dout), _ptr(dx), _ptr(dg), _ptr(dprev), _stream(out.device)),
                   "atlas_scan_bwd")
        return dg, dx, dprev


def assoc_scan(gates: Tensor, inputs: Tensor, prev: Tensor | None = None, remove_prev: bool | None = None) -> Tensor:
    """AssocScan contract: out_t = gates_t * out_{t-1} + inputs_t (gates [N, T] or [N, T, 1...]
    broadcast over the trailing dims of inputs [N, T, ...]); prev is out_{-1}. With prev and
    remove_prev=False the result has T+1 steps and starts with prev."""
    _require_gpu(gates, inputs, prev)
    dt = inputs.dtype if inputs.dtype in _DTYPES else torch.float32
    N, T = inputs.shape[:2]
    g = gates.reshape(N, T, -1)
    if g.shape[-1] != 1:
        raise ValueError("gates must be scalar per (n, t)")
    g = g.reshape(N, T).to(dt).contiguous()
    x = inputs.to(dt).contiguous()
    pv = prev.to(dt).contiguous() if prev is not None else None
    out = _ScanFn.apply(g, x, pv)
    if remove_prev is None:
        remove_prev = prev is not None
    if prev is not None and not remove_prev:
        out = torch.cat([pv.unsqueeze(1), out], dim=1)
    return out


class AssocScan(torch.nn.Module):
    """Module form of the scan (constructor kwargs of assoc_scan.AssocScan are accepted)."""

    def __init__(self, use_accelerated: bool = False, **kwargs):
        super().__init__()

    def forward(self, gates, inputs, prev=None, remove_prev=None):
        return assoc_scan(gates, inputs, prev=prev, remove_prev=remove_prev)


class _WindowSumFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, window):
        lib = _lib.load()
        n, t = x.shape[:2]
        d = x.numel() // (n * t)
        y = torch.empty_like(x)
        _lib.check(lib.atlas_window_sum(_DTYPES[x.dtype], n, t, d, window, 0, _ptr(x), _ptr(y), _stream(x.device)),
                   "atlas_window_sum")
        ctx.window = window
        return y

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.load()
        dy = dy.contiguous()
        n, t = dy.shape[:2]
        d = dy.numel() // (n * t)
        dx = torch.empty_like(dy)
        _lib.check(lib.atlas_window_sum(_DTYPES[dy.dtype], n, t, d, ctx.window, 1, _ptr(dy), _ptr(dx),
                                        _stream(dy.device)), "atlas_window_sum")
        return dx, None


def window_sum(x: Tensor, window: int) -> Tensor:
    """Inclusive window sum along dim 1 (the contract of _sliding_sum_along_time)."""
    if window <= 1:
        return x
    _require_gpu(x)
    dt = x.dtype if x.dtype in _DTYPES else torch.float32
    return _WindowSumFn.apply(x.to(dt).contiguous(), int(window))


def _affine_workspace(lib, n, t, r, d, device) -> tuple[Tensor, int]:
    nbytes = lib.atlas_affine_scan_workspace_bytes(n, t, r, d)
    return torch.empty((nbytes + 3) // 4, device=device, dtype=torch.float32), nbytes


class _AffineScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, A, B, prev):
        lib = _lib.load()
        n, t, d = A.shape[0], A.shape[1], A.shape[2]
        r = B.shape[2]
        out = torch.empty_like(B)
        ws, nbytes = _affine_workspace(lib, n, t, r, d, A.device)
        _lib.check(lib.atlas_affine_scan_fwd(n, t, r, d, _ptr(A), _ptr(B), _ptr(prev), _ptr(out), _ptr(ws), nbytes,
                                             _stream(A.device)), "atlas_affine_scan_fwd")
        ctx.save_for_backward(A, out, prev)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        A, out, prev = ctx.saved_tensors
        n, t, d = A.shape[0], A.shape[1], A.shape[2]
        r = out.shape[2]
        dout = dout.contiguous().float()
        dA = torch.empty_like(A)
        dB = torch.empty_like(out)
        dprev = torch.empty_like(prev) if prev is not None else None
        ws, nbytes = _affine_workspace(lib, n, t, r, d, A.device)
        _lib.check(lib.atlas_affine_scan_bwd(n, t, r, d, _ptr(A), _ptr(out), _ptr(prev), _ptr(dout), _ptr(dA), _ptr(dB),
                                             _ptr(dprev), _ptr(ws), nbytes, _stream(A.device)), "atlas_affine_scan_bwd")
        return dA, dB, dprev


def affine_associative_scan(A: Tensor, B: Tensor, *, prev: Tensor | None = None, remove_prev: bool = False) -> Tensor:
    """H_t = H_{t-1} A_t + B_t (atlas_pytorch/affine_scan.py:36-158): A [N,T,D,D], B [N,T,R,D],
    prev [N,R,D]. Returns [N,T,R,D], or [N,T+1,R,D] led by prev when prev is given and not
    remove_prev. Computed in fp32 on the matrix cores, chunked (D, R <= 64); the result has B's dtype."""
    _require_gpu(A, B, prev)
    if A.dim() != 4 or A.shape[2] != A.shape[3] or B.dim() != 4 or B.shape[:2] != A.shape[:2] or B.shape[3] != A.shape[2]:
        raise ValueError(f"A must be [N, T, D, D] and B [N, T, R, D], got {tuple(A.shape)} and {tuple(B.shape)}")
    if prev is not None and tuple(prev.shape) != (B.shape[0], B.shape[2], B.shape[3]):
        raise ValueError(f"prev must be [N, R, D] = {(B.shape[0], B.shape[2], B.shape[3])}, got {tuple(prev.shape)}")
    dt = B.dtype
    A32 = A.float().contiguous()
    B32 = B.float().contiguous()
    p32 = prev.float().contiguous() if prev is not None else None
    H = _AffineScanFn.apply(A32, B32, p32)
    if prev is not None and not remove_prev:
        H = torch.cat([p32[:, None], H], dim=1)
    return H.to(dt)


# ------------------------------------------------------------------------------------------
# Cell prologue (rnn_memory.py:567-653): fused kernels around the projection GEMMs
# ------------------------------------------------------------------------------------------

def _dt_code(t: Tensor) -> int:
    if t.dtype not in _DTYPES:
        raise ValueError(f"the fused prologue takes fp32 or bf16 tensors, got {t.dtype}")
    return _DTYPES[t.dtype]


def _sum_partials(items):
    """atlas_partials_sum: items of (partials [rows, ...] fp32, out dtype, out shape) -> the sums over
    the rows, one launch for all of them (deterministic order)."""
    lib = _lib.load()
    parts = [_aligned(p.reshape(p.shape[0], -1)) for p, _, _ in items]
    outs = [torch.empty(p.shape[1], device=p.device, dtype=dt) for p, (_, dt, _) in zip(parts, items)]
    cnt = len(parts)
    I32, VP = ctypes.c_int * cnt, ctypes.c_void_p * cnt
    _lib.check(lib.atlas_partials_sum(cnt, parts[0].shape[0], I32(*[p.shape[1] for p in parts]),
                                      VP(*[p.data_ptr() for p in parts]), VP(*[o.data_ptr() for o in outs]),
                                      I32(*[_DTYPES[o.dtype] for o in outs]), _stream(parts[0].device)),
               "atlas_partials_sum")
    return [o.reshape(shape) for o, (_, _, shape) in zip(outs, items)]


class _PrologueFn:
    """xn = RMSNorm(x) and the three depthwise convolutions of xn (atlas_prologue_fwd / _bwd), called
    by hand from _CellPrologueFn (ctx is a _HandCtx); the backward returns its parameter gradients as
    per-workgroup partials for one _sum_partials call."""

    @staticmethod
    def forward(ctx, x, norm_w, wq, wk, wv, conv_k, eps):
        lib = _lib.load()
        B, T, dim = x.shape
        x = _aligned(x)
        conv = conv_k > 1
        xn = torch.empty_like(x)
        qi = torch.empty_like(x) if conv else None
        ki = torch.empty_like(x) if conv else None
        vi = torch.empty_like(x) if conv else None
        inv = torch.empty(B, T, device=x.device, dtype=torch.float32)
        taps = [_aligned(w.reshape(dim, conv_k)) if conv else None for w in (wq, wk, wv)]
        _lib.check(lib.atlas_prologue_fwd(_dt_code(x), B, T, dim, conv_k, float(eps), _ptr(x), _ptr(norm_w),
                                          _ptr(taps[0]), _ptr(taps[1]), _ptr(taps[2]), _ptr(xn), _ptr(qi), _ptr(ki),
                                          _ptr(vi), _ptr(inv), _stream(x.device)), "atlas_prologue_fwd")
        ctx.save_for_backward(x, norm_w, *(t if t is not None else torch.empty(0) for t in taps), inv)
        ctx.conv_k = conv_k
        ctx.wshape = tuple(wq.shape) if conv else None
        if not conv:
            return xn          # the caller uses xn for q_in, k_in and v_in
        return xn, qi, ki, vi

    @staticmethod
    def backward(ctx, dxn, *dconv):
        lib = _lib.load()
        x, norm_w, tq, tk, tv, inv = ctx.saved_tensors
        B, T, dim = x.shape
        K = ctx.conv_k
        conv = K > 1
        z = lambda t: torch.zeros_like(x) if t is None else _aligned(t.to(x.dtype))
        dxn = z(dxn)
        dqi, dki, dvi = (z(g) for g in dconv) if conv else (None, None, None)
        nwg = lib.atlas_prologue_num_workgroups(B, T)
        dx = torch.empty_like(x)
        dnw = torch.empty(nwg, dim, device=x.device, dtype=torch.float32)
        dcv = torch.empty(nwg, 3, dim, K, device=x.device, dtype=torch.float32) if conv else None
        _lib.check(lib.atlas_prologue_bwd(_dt_code(x), B, T, dim, K, _ptr(x), _ptr(norm_w),
                                          _ptr(tq if conv else None), _ptr(tk if conv else None),
                                          _ptr(tv if conv else None), _ptr(inv), _ptr(dxn), _ptr(dqi), _ptr(dki),
                                          _ptr(dvi), _ptr(dx), _ptr(dnw), _ptr(dcv), _stream(x.device)),
                   "atlas_prologue_bwd")
        parts = [(dnw, norm_w.dtype, tuple(norm_w.shape))]
        if conv:
            parts.append((dcv, x.dtype, (3, *ctx.wshape)))
        return dx, parts


class _HeadsFn:
    """Head split, MultiheadRMSNorm of q / k and the gate sigmoids (atlas_heads_fwd / _bwd), called by
    hand from _CellPrologueFn; the backward returns its parameter gradients as partials."""

    @staticmethod
    def forward(ctx, ql, kl, vl, zl, q_gamma, k_gamma, bias, heads, d):
        lib = _lib.load()
        B, T, _ = ql.shape
        nG = bias.numel() // heads if bias is not None else 0
        dev = ql.device
        ql, kl, vl = _aligned(ql), _aligned(kl), _aligned(vl)
        zl = _aligned(zl) if nG else None
        qg = _aligned(q_gamma.reshape(heads, d)) if q_gamma is not None else None
        kg = _aligned(k_gamma.reshape(heads, d)) if k_gamma is not None else None
        q = torch.empty(B * heads, T, d, device=dev, dtype=ql.dtype)
        k = torch.empty_like(q)
        v = torch.empty_like(q)
        gates = torch.empty(nG, B * heads, T, device=dev, dtype=ql.dtype) if nG else None
        _lib.check(lib.atlas_heads_fwd(_dt_code(ql), B, T, heads, d, nG, _ptr(ql), _ptr(kl), _ptr(vl), _ptr(zl),
                                       _ptr(qg), _ptr(kg), _ptr(bias), _ptr(q), _ptr(k), _ptr(v), _ptr(gates),
                                       _stream(dev)), "atlas_heads_fwd")
        e0 = torch.empty(0, device=dev)
        ctx.save_for_backward(ql, kl, qg if qg is not None else e0, kg if kg is not None else e0,
                              gates if gates is not None else e0)
        ctx.meta = (heads, d, nG, q_gamma is not None, None if q_gamma is None else tuple(q_gamma.shape),
                    None if bias is None else bias.dtype)
        if nG:
            return (q, k, v, *gates.unbind(0))
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv, *dgates):
        lib = _lib.load()
        ql, kl, qg, kg, gates = ctx.saved_tensors
        heads, d, nG, norm, gshape, bdt = ctx.meta
        B, T, _ = ql.shape
        dev = ql.device
        z = lambda t: torch.zeros(B * heads, T, d, device=dev, dtype=ql.dtype) if t is None else _aligned(t.to(ql.dtype))
        dq, dk, dv = z(dq), z(dk), z(dv)
        dg = None
        if nG:
            dg = torch.stack([g.to(ql.dtype) if g is not None else torch.zeros(B * heads, T, device=dev, dtype=ql.dtype)
                              for g in dgates])
        nwg = lib.atlas_prologue_num_workgroups(B, T)
        dql, dkl, dvl = torch.empty_like(ql), torch.empty_like(kl), torch.empty_like(ql)
        dzl = torch.empty(B, T, nG * heads, device=dev, dtype=ql.dtype) if nG else None
        dqg = torch.empty(nwg, heads, d, device=dev, dtype=torch.float32) if norm else None
        dkg = torch.empty_like(dqg) if norm else None
        dbias = torch.empty(nwg, nG * heads, device=dev, dtype=torch.float32) if nG else None
        _lib.check(lib.atlas_heads_bwd(_dt_code(ql), B, T, heads, d, nG, _ptr(ql), _ptr(kl),
                                       _ptr(qg if norm else None), _ptr(kg if norm else None),
                                       _ptr(gates if nG else None), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dg), _ptr(dql),
                                       _ptr(dkl), _ptr(dvl), _ptr(dzl), _ptr(dqg), _ptr(dkg), _ptr(dbias), _stream(dev)),
                   "atlas_heads_bwd")
        parts = {}
        if norm:
            parts["qg"] = (dqg, qg.dtype, gshape)
            parts["kg"] = (dkg, kg.dtype, gshape)
        if nG:
            parts["b"] = (dbias, bdt, (nG * heads,))
        return dql, dkl, dvl, dzl, parts


def _wgrads(pairs, dtype) -> list:
    """dW = dy^T x over every leading axis of dy [..., o] and x [..., i], for each (dy, x) of pairs
    (the same token count). bf16 operands go to atlas_linear_wgrad_batch, all layers in one launch
    (both activations read as stored, the token axis split over the matrix cores, fp32 partials
    summed in a fixed order): 16384 tokens x 512 x 512 took 67 us through a transposed copy and a
    batched hipBLASLt product, whose plain form (one product with K = 16384 on few output tiles)
    took 100 us. fp32 operands keep torch's product over token slices."""
    dys = [dy.reshape(-1, dy.shape[-1]) for dy, _ in pairs]
    xs = [x.reshape(-1, x.shape[-1]) for _, x in pairs]
    n = dys[0].shape[0]
    if all(d.dtype == torch.bfloat16 and x.dtype == torch.bfloat16 and d.shape[-1] % 8 == 0 and x.shape[-1] % 8 == 0
           and d.shape[0] == n and x.shape[0] == n for d, x in zip(dys, xs)) and dtype in _DTYPES:
        lib = _lib.load()
        dys, xs = [_aligned(d) for d in dys], [_aligned(x) for x in xs]
        dev = dys[0].device
        cnt = len(dys)
        I32, VP = ctypes.c_int * cnt, ctypes.c_void_p * cnt
        os_, is_ = I32(*[d.shape[1] for d in dys]), I32(*[x.shape[1] for x in xs])
        ws_bytes = lib.atlas_linear_wgrad_batch_workspace_bytes(cnt, n, os_, is_)
        ws = torch.empty(max(ws_bytes, 16) // 4, device=dev, dtype=torch.float32)
        dws = [torch.empty(d.shape[1], x.shape[1], device=dev, dtype=dtype) for d, x in zip(dys, xs)]
        _lib.check(lib.atlas_linear_wgrad_batch(_DTYPES[dtype], cnt, n, os_, is_, VP(*[d.data_ptr() for d in dys]),
                                                VP(*[x.data_ptr() for x in xs]), VP(*[w.data_ptr() for w in dws]),
                                                _ptr(ws), ws_bytes, _stream(dev)), "atlas_linear_wgrad_batch")
        return dws
    out = []
    for dy2, x2 in zip(dys, xs):
        o, i = dy2.shape[-1], x2.shape[-1]
        S = next((c for c in (8, 4, 2) if n % c == 0 and n // c >= 1024), 1)
        if S == 1:
            out.append((dy2.t() @ x2).to(dtype))
            continue
        a = dy2.view(S, n // S, o).transpose(1, 2).contiguous()   # both operands row-major (no transposed views)
        out.append(torch.bmm(a, x2.view(S, n // S, i).contiguous()).float().sum(0).to(dtype))
    return out


def _wgrad(dy: Tensor, x: Tensor, dtype) -> Tensor:
    """One layer's weight gradient (_wgrads)."""
    return _wgrads([(dy, x)], dtype)[0]


_GEMM_NT, _GEMM_NN = 0, 1


def _products(layout: int, acts, weights):
    """atlas_linear_batch: up to four bf16 products in one launch. NT: acts[i] [..., k] x
    weights[i] [n, k] -> [..., n] (y = x W^T); NN: acts[i] [..., k] x weights[i] [k, n] -> [..., n]
    (dx = dy W). Falls back to torch for other dtypes or sizes that are not multiples of 8."""
    ok = all(a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and a.shape[-1] % 8 == 0
             and w.shape[0] % 8 == 0 and w.shape[1] % 8 == 0 for a, w in zip(acts, weights))
    m = acts[0].numel() // acts[0].shape[-1]
    if not ok or any(a.numel() // a.shape[-1] != m for a in acts):
        if layout == _GEMM_NT:
            return [torch.nn.functional.linear(a, w) for a, w in zip(acts, weights)]
        return [a @ w for a, w in zip(acts, weights)]
    lib = _lib.load()
    dev = acts[0].device
    a2 = [_aligned(a.reshape(m, a.shape[-1])) for a in acts]
    w2 = [_aligned(w) for w in weights]
    ns = [w.shape[0] if layout == _GEMM_NT else w.shape[1] for w in w2]
    ks = [a.shape[-1] for a in a2]
    outs = [torch.empty(m, nn, device=dev, dtype=torch.bfloat16) for nn in ns]
    cnt = len(a2)
    I32 = ctypes.c_int * cnt
    VP = ctypes.c_void_p * cnt
    _lib.check(lib.atlas_linear_batch(layout, cnt, m, I32(*ns), I32(*ks), VP(*[a.data_ptr() for a in a2]),
                                      VP(*[w.data_ptr() for w in w2]), VP(*[o.data_ptr() for o in outs]),
                                      _stream(dev)), "atlas_linear_batch")
    return [o.reshape(*a.shape[:-1], nn) for o, a, nn in zip(outs, acts, ns)]


class _LinearFn(torch.autograd.Function):
    """y = x W^T with its input gradient on atlas_linear_batch and the weight gradient of _wgrad."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return _products(_GEMM_NT, [x], [w])[0]

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = _products(_GEMM_NN, [dy], [w])[0] if ctx.needs_input_grad[0] else None
        dw = _wgrad(dy, x, w.dtype) if ctx.needs_input_grad[1] else None
        return dx, dw


def linear(x: Tensor, w: Tensor) -> Tensor:
    """x W^T without bias, with the token-split weight gradient of _LinearFn."""
    return _LinearFn.apply(x, w)


class _HandCtx:
    """Stands in for autograd's ctx where one Function composes other Functions' forward and
    backward by hand."""

    def set_materialize_grads(self, value):
        pass

    def save_for_backward(self, *tensors):
        self.saved_tensors = tensors


class _CellPrologueFn(torch.autograd.Function):
    """The whole prologue as ONE autograd node: the RMSNorm / conv kernel, the four projections
    (one atlas_linear_batch launch), the head-split kernel, and in the backward their adjoints in
    reverse order (the four input gradients in one launch) with the weight gradients of _wgrad.
    One node and batched products keep the host's per-step work down (the prologue is bound by
    host issue at C5's layer shape, not by its kernels)."""

    @staticmethod
    def forward(ctx, x, norm_w, wq, wk, wv, Wq, Wk, Wv, Wg, bg, qg, kg, conv_k, eps, heads, d):
        cp, ch = _HandCtx(), _HandCtx()
        conv = conv_k > 1
        if conv:
            xn, qi, ki, vi = _PrologueFn.forward(cp, x, norm_w, wq, wk, wv, conv_k, eps)
        else:
            xn = _PrologueFn.forward(cp, x, norm_w, None, None, None, 0, eps)
            qi = ki = vi = xn
        if Wg is not None:
            ql, kl, vl, zl = _products(_GEMM_NT, [qi, ki, vi, xn], [Wq, Wk, Wv, Wg])
        else:
            (ql, kl, vl), zl = _products(_GEMM_NT, [qi, ki, vi], [Wq, Wk, Wv]), None
        outs = _HeadsFn.forward(ch, ql, kl, vl, zl, qg, kg, bg, heads, d)
        e0 = torch.empty(0, device=x.device)
        ctx.save_for_backward(qi, ki, vi, xn, Wq, Wk, Wv, Wg if Wg is not None else e0)
        ctx.cp, ctx.ch, ctx.conv, ctx.has_g = cp, ch, conv, Wg is not None
        return (xn, *outs)

    @staticmethod
    def backward(ctx, dxn, dq, dk, dv, *dgates):
        qi, ki, vi, xn, Wq, Wk, Wv, Wg = ctx.saved_tensors
        dql, dkl, dvl, dzl, hparts = _HeadsFn.backward(ctx.ch, dq, dk, dv, *dgates)
        if ctx.has_g:
            dqi, dki, dvi, dxg = _products(_GEMM_NN, [dql, dkl, dvl, dzl], [Wq, Wk, Wv, Wg])
        else:
            dqi, dki, dvi = _products(_GEMM_NN, [dql, dkl, dvl], [Wq, Wk, Wv])
        pairs = [(dql, qi), (dkl, ki), (dvl, vi)] + ([(dzl, xn)] if ctx.has_g else [])
        dws = _wgrads(pairs, Wq.dtype)
        dWq, dWk, dWv = dws[:3]
        dWg = dws[3] if ctx.has_g else None
        dsum = dxn
        if ctx.has_g:
            dsum = dxg if dsum is None else dsum + dxg
        if ctx.conv:
            dx, pparts = _PrologueFn.backward(ctx.cp, dsum, dqi, dki, dvi)
        else:
            dsum = dqi + dki + dvi + (dsum if dsum is not None else 0)
            dx, pparts = _PrologueFn.backward(ctx.cp, dsum)
        # every parameter gradient of the two kernels from their partials, in one launch
        names = [n for n in ("qg", "kg", "b") if n in hparts]
        sums = _sum_partials(pparts + [hparts[n] for n in names])
        dnorm = sums[0]
        dtq = dtk = dtv = None
        if ctx.conv:
            dtq, dtk, dtv = sums[1].unbind(0)
        got = dict(zip(names, sums[len(pparts):]))
        return (dx, dnorm, dtq, dtk, dtv, dWq, dWk, dWv, dWg, got.get("b"), got.get("qg"), got.get("kg"),
                None, None, None, None)


def cell_prologue(x: Tensor, norm_weight: Tensor, eps: float, conv_weights, proj_weights, gate_weights, gate_biases,
                  q_gamma: Tensor | None, k_gamma: Tensor | None, heads: int, dim_head: int):
    """The memory cell's prologue (rnn_memory.py:567-653) on the fused kernels:

        xn = RMSNorm(x);  q_in, k_in, v_in = depthwise convs of xn (or xn itself)
        ql, kl, vl = q_in Wq^T, k_in Wk^T, v_in Wv^T;  zl = xn [W_g1; W_g2; ...]^T     (one batched launch)
        q, k = MultiheadRMSNorm of the heads of ql, kl; v = the heads of vl;  gate_i = sigmoid(zl_i + b_i)

    x [B, T, dim]; conv_weights (wq, wk, wv) [dim, 1, K] or None; proj_weights (Wq, Wk, Wv) [H d, dim];
    gate_weights / gate_biases: lists of [H, dim] / [H] (the to_lr, to_decay, [to_momentum],
    [to_omega_gate] heads); q_gamma, k_gamma [H, 1, d] or None (no q/k norm). Every tensor in x's
    dtype (fp32 or bf16; parameters are cast). Returns (xn, q, k, v [(B H), T, d], [gate_i
    [(B H), T]]), all differentiable."""
    _require_gpu(x, norm_weight)
    if x.dim() != 3:
        raise ValueError(f"x must be [B, T, dim], got {tuple(x.shape)}")
    dt = x.dtype
    cast = lambda t: None if t is None else t.to(dt)
    conv_k = 0
    if conv_weights is not None:
        conv_k = conv_weights[0].shape[-1]
        if conv_k > 8:
            raise ValueError("the fused prologue supports depthwise convolutions of up to 8 taps")
    wq, wk, wv = (cast(w) for w in conv_weights) if conv_weights is not None else (None, None, None)
    if conv_k <= 1:
        wq = wk = wv = None
    Wg = torch.cat([cast(w) for w in gate_weights], dim=0) if gate_weights else None
    bias = torch.cat([cast(b) for b in gate_biases]).contiguous() if gate_weights else None
    out = _CellPrologueFn.apply(x, norm_weight.to(dt).contiguous(), wq, wk, wv, cast(proj_weights[0]),
                                cast(proj_weights[1]), cast(proj_weights[2]), Wg, bias, cast(q_gamma), cast(k_gamma),
                                conv_k if conv_k > 1 else 0, eps, heads, dim_head)
    return out[0], out[1], out[2], out[3], list(out[4:])


# ------------------------------------------------------------------------------------------
# Preallocated plan: direct C-ABI calls for a fixed problem shape
# ------------------------------------------------------------------------------------------

class RecurrencePlan:
    """Forward/backward of one problem shape with every buffer allocated up front.

    No autograd and no per-call allocation: `forward` and `backward` only launch the library
    on the current stream. Outputs and gradients live in the plan and are overwritten by the
    next call.
    """

    def __init__(self, bh: int, T: int, d: int, *, window: int = 1, momentum: bool = True,
                 gate_mode: str | None = None, dtype=torch.bfloat16, map_degree: int = 1,
                 has_buffer: bool = False, clamp_every: int | None = None, clamp_final: bool = True,
                 device="cuda"):
        lib = _lib.load()
        self.lib = lib
        self.device = torch.device(device)
        cfg = RecurrenceConfig(window=window, map_mode='elementwise' if map_degree > 1 else 'off',
                               map_degree=map_degree, clamp_every=clamp_every, clamp_final=clamp_final)
        gate_stub = None
        if gate_mode == 'token':
            gate_stub = torch.empty(1, 1)
        elif gate_mode == 'lag':
            gate_stub = torch.empty(1, 1, 1)
        self.prob = _problem(cfg, bh, T, d, d, momentum, gate_stub, has_buffer, dtype)
        _lib.check(lib.atlas_mem_validate(ctypes.byref(self.prob)), "atlas_mem_validate")
        dev, f32 = self.device, torch.float32
        self.shape = (bh, T, d)
        self.momentum, self.window, self.dtype = momentum, window, dtype
        self.y = torch.empty(bh, T, d, device=dev, dtype=dtype)
        self.S_T = torch.empty(bh, d, d, device=dev, dtype=f32)
        self.Z_T = torch.empty(bh, d, d, device=dev, dtype=f32) if momentum else None
        self.buf_out = torch.empty(bh, window - 1, d, d, device=dev, dtype=f32) if window > 1 else None
        self.saved = torch.empty(lib.atlas_mem_saved_bytes(ctypes.byref(self.prob)) // 4, device=dev, dtype=f32)
        self.ws_bytes = lib.atlas_mem_bwd_workspace_bytes(ctypes.byref(self.prob))
        self.ws = torch.empty((self.ws_bytes + 3) // 4, device=dev, dtype=f32)
        self.grads = None
        self._inputs = None

    def _check(self, k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer):
        check_operands(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer, window=self.window,
                       dtype=self.dtype, contiguous=True)
        if tuple(k.shape) != self.shape or tuple(v.shape) != self.shape:
            raise ValueError(f"the plan is for k, v of shape {self.shape}, got {tuple(k.shape)}, {tuple(v.shape)}")
        if k.device != self.device and not (self.device.index is None and k.device.type == self.device.type):
            raise ValueError(f"the plan runs on {self.device}, inputs are on {k.device}")
        if (beta is not None) != self.momentum:
            raise ValueError("beta must be given iff the plan has momentum")
        gmode = _lib.GATE_NONE if gate is None else (_lib.GATE_TOKEN if gate.dim() == 2 else _lib.GATE_LAG)
        if gmode != self.prob.gate_mode:
            raise ValueError(f"gate layout {None if gate is None else tuple(gate.shape)} does not match the plan's gate mode")
        if (buffer is not None) != bool(self.prob.has_buffer):
            raise ValueError("buffer must be given iff the plan was made with has_buffer=True")
        if S_ref is None or S0 is None:
            raise ValueError("S_ref and S0 are required")

    def forward(self, k, q, v, lr, decay, beta=None, gate=None, S_ref=None, S0=None, Z0=None, buffer=None):
        self._check(k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer)
        self._inputs = (k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buffer)
        a = _lib.FwdArgs(k=_ptr(k), q=_ptr(q), v=_ptr(v), lr=_ptr(lr), decay=_ptr(decay), beta=_ptr(beta),
                         gate=_ptr(gate), S_ref=_ptr(S_ref), S0=_ptr(S0), Z0=_ptr(Z0), buffer_in=_ptr(buffer),
                         y=_ptr(self.y), S_T=_ptr(self.S_T), Z_T=_ptr(self.Z_T), buffer_out=_ptr(self.buf_out))
        _lib.check(self.lib.atlas_mem_fwd(ctypes.byref(self.prob), ctypes.byref(a), _ptr(self.saved),
                                          _stream(self.device)), "atlas_mem_fwd")
        return self.y, self.S_T, self.Z_T, self.buf_out

    def backward(self, dy, dS_T=None, dZ_T=None, dbuffer_out=None):
        if self._inputs is None:
            raise RuntimeError("RecurrencePlan.backward before forward")
        k, q, v, lr, decay, beta, gate, S_ref, S0, Z0, buf = self._inputs
        bh, T, d = self.shape
        state = (bh, d, d)
        for name, t, shape, dt in (("dy", dy, self.shape, self.dtype), ("dS_T", dS_T, state, torch.float32),
                                   ("dZ_T", dZ_T, state, torch.float32),
                                   ("dbuffer_out", dbuffer_out, (bh, self.window - 1, d, d), torch.float32)):
            if t is None:
                if name == "dy":
                    raise ValueError("dy is required")
                continue
            if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous() or t.device != k.device:
                raise ValueError(f"{name} must be a contiguous {dt} tensor of shape {shape} on {k.device}, "
                                 f"got {t.dtype} {tuple(t.shape)} on {t.device}")
        if dZ_T is not None and not self.momentum:
            raise ValueError("dZ_T given to a plan without momentum")
        if dbuffer_out is not None and self.window < 2:
            raise ValueError("dbuffer_out given to a plan with window 1")
        if self.grads is None:
            f32 = torch.float32
            bh, T, d = self.shape
            self.grads = dict(
                k=torch.empty_like(k), q=torch.empty_like(q), v=torch.empty_like(v), lr=torch.empty_like(lr),
                decay=torch.empty_like(decay), beta=torch.empty_like(beta) if beta is not None else None,
                gate=torch.empty_like(gate) if gate is not None else None,
                S_ref=torch.empty(bh, d, d, device=self.device, dtype=f32),
                S0=torch.empty(bh, d, d, device=self.device, dtype=f32),
                Z0=torch.empty(bh, d, d, device=self.device, dtype=f32) if self.momentum else None,
                buffer=torch.empty_like(buf) if buf is not None else None)
        gr = self.grads
        a = _lib.BwdArgs(k=_ptr(k), q=_ptr(q), v=_ptr(v), lr=_ptr(lr), decay=_ptr(decay), beta=_ptr(beta),
                         gate=_ptr(gate), S_ref=_ptr(S_ref), S0=_ptr(S0), Z0=_ptr(Z0), buffer_in=_ptr(buf),
                         dy=_ptr(dy), dS_T=_ptr(dS_T), dZ_T=_ptr(dZ_T), dbuffer_out=_ptr(dbuffer_out),
                         dk=_ptr(gr["k"]), dq=_ptr(gr["q"]), dv=_ptr(gr["v"]), dlr=_ptr(gr["lr"]),
                         ddecay=_ptr(gr["decay"]), dbeta=_ptr(gr["beta"]), dgate=_ptr(gr["gate"]),
                         dS_ref=_ptr(gr["S_ref"]), dS0=_ptr(gr["S0"]), dZ0=_ptr(gr["Z0"]),
                         dbuffer_in=_ptr(gr["buffer"]))
        _lib.check(self.lib.atlas_mem_bwd(ctypes.byref(self.prob), ctypes.byref(a), _ptr(self.saved), _ptr(self.ws),
                                          ctypes.c_size_t(self.ws_bytes), _stream(self.device)), "atlas_mem_bwd")
        return gr


def profile_enable(on: bool = True) -> None:
    """Per-kernel HIP-event timing inside the library (see atlas_mem_profile_enable)."""
    _lib.check(_lib.load().atlas_mem_profile_enable(int(on)), "atlas_mem_profile_enable")


def profile_read(reset: bool = True) -> dict:
    """{kernel name: (total ms, launches)} accumulated since the last reset."""
    lib = _lib.load()
    n = _lib.NKERNELS
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_longlong * n)()
    _lib.check(lib.atlas_mem_profile_read(ms, cnt, n, int(reset)), "atlas_mem_profile_read")
    return {lib.atlas_mem_kernel_name(i).decode(): (ms[i], cnt[i]) for i in range(n)}
