"""Module API of the RNN memory cells (atlas_pytorch/rnn_memory.py), on the HIP recurrence.

Same classes, constructor arguments, parameter names, initialisations and state format as the
reference, so checkpoints load with `load_state_dict` and callers switch by changing the import:

* `RNNMemState`, `state_detach`                       (rnn_memory.py:68-83)
* `PolynomialFeatureMap` ('off' / 'elementwise' / 'tensor')  (rnn_memory.py:90-132)
* `MultiheadRMSNorm`                                  (rnn_memory.py:139-147)
* `RNNMemoryCell`                                     (rnn_memory.py:154-408)
* `OmegaRNNMemoryCell`                                (rnn_memory.py:415-814)
* `RNNMemory`, `OmegaRNNMemory`                       (rnn_memory.py:821-885)

The prologue runs in fused kernels around the projection GEMMs (`functional.cell_prologue`:
pre-norm RMSNorm and the depthwise convs in one kernel; the head split, q/k MultiheadRMSNorm and
the gate sigmoids in another; both with hand-written backwards). The memory recurrence itself -
delta, the gated window of outer products, the momentum and decay scans, the clamp, the retrieval
and all their gradients - runs in libatlas_mem.so (`functional.memory_recurrence`) on ROCm
tensors; on CPU tensors the cells raise, there is no CPU implementation in this package. The
elementwise feature map is applied inside the recurrence kernels, the tensor map in its own fused
kernels.

`scan_chunk_len` keeps the reference semantics (S_ref = the call-start state for every chunk,
each chunk's end state clamped to +-100) through the kernels' clamp_every option.
"""

from __future__ import annotations

import math
import warnings
import weakref
from functools import partial
from typing import NamedTuple

import torch
from einops import rearrange
from einops.layers.torch import Rearrange
from torch import Tensor, nn
from torch.nn import Conv1d, Linear, Module, Parameter

from .functional import (AssocScan, AtlasOmegaFunction, cell_prologue, check_cuda_availability, linear,
                         memory_recurrence, tensor_feature_map, window_sum)
from .functional import symmetrized_tables as functional_symmetrized_tables


def exists(v):
    return v is not None


def default(v, d):
    return v if exists(v) else d


LinearNoBias = partial(Linear, bias=False)


def _sliding_sum_along_time(x: Tensor, window: int) -> Tensor:
    """Inclusive sliding window sum along dim 1 (rnn_memory.py:50-61), on the GPU window kernel."""
    return window_sum(x, window)


class RNNMemState(NamedTuple):
    """State carried across calls (rnn_memory.py:68-73)."""
    seq_index: int
    S: Tensor
    Z: Tensor | None
    omega_buffer: Tensor | None


def state_detach(state: RNNMemState) -> RNNMemState:
    """rnn_memory.py:76-83."""
    return RNNMemState(
        seq_index=state.seq_index,
        S=state.S.detach() if exists(state.S) else None,
        Z=state.Z.detach() if exists(state.Z) else None,
        omega_buffer=state.omega_buffer.detach() if exists(state.omega_buffer) else None,
    )


class PolynomialFeatureMap(Module):
    """rnn_memory.py:90-132. 'off': x; 'elementwise': sum_{i=1..g} x^i; 'tensor':
    [x, vec(x x^T)] @ proj with the fixed random projection registered as the buffer `proj`."""

    def __init__(self, dim: int, degree: int = 1, mode: str = 'off'):
        super().__init__()
        self.dim = dim
        self.degree = degree
        self.mode = mode
        # symmetrised tables of proj for the fused map, per (dtype, device):
        # (ps, pst, weak reference to proj, proj version, event recorded after forming them, stream)
        self._tables: dict = {}
        if mode == 'tensor':
            feat_dim = dim + dim * dim
            self.register_buffer('proj', torch.randn(feat_dim, dim) / math.sqrt(feat_dim))

    def refresh_tables(self) -> None:
        """Drops the cached tables of proj. Moves (`.to`, `.cuda`, ...), `load_state_dict` and
        in-place operations that bump proj's version are seen by the cache itself; a write that
        bypasses the version counter (through `proj.data`) must be followed by this call."""
        self._tables.clear()

    def _apply(self, fn, *args, **kwargs):
        self._tables.clear()
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self._tables.clear()
        return super()._load_from_state_dict(*args, **kwargs)

    def _tensor_tables(self, x: Tensor):
        """proj's symmetrised tables in x's dtype, formed once per (dtype, device, proj version) and
        reused by the k and q maps and by later steps. Under HIP graph capture they are formed
        inside the graph on every call (the graph then owns them). Used on another stream than the
        one that formed them, the current stream waits for them and keeps them alive."""
        proj = self.proj
        if torch.cuda.is_current_stream_capturing():
            return functional_symmetrized_tables(proj, self.dim, x.dtype)
        key = (x.dtype, x.device)
        hit = self._tables.get(key)
        cur = torch.cuda.current_stream(x.device)
        if hit is not None and hit[2]() is proj and hit[3] == proj._version:
            ps, pst, _, _, ev, stream = hit
            if stream != cur:
                cur.wait_event(ev)
                ps.record_stream(cur)
                pst.record_stream(cur)
            return ps, pst
        ps, pst = functional_symmetrized_tables(proj, self.dim, x.dtype)
        ev = torch.cuda.Event()
        ev.record(cur)
        self._tables[key] = (ps, pst, weakref.ref(proj), proj._version, ev, cur)
        return ps, pst

    @property
    def fused_elementwise(self) -> bool:
        """True when the map is the elementwise polynomial the recurrence kernels apply themselves."""
        return self.mode == 'elementwise' and self.degree > 1

    def forward(self, x: Tensor) -> Tensor:
        if self.degree <= 1 or self.mode == 'off':
            return x
        if self.mode == 'elementwise':
            out = x.clone()
            power = x
            for _ in range(2, self.degree + 1):
                power = power * x
                out = out + power
            return out
        if self.mode == 'tensor':   # fused kernels (functional.tensor_feature_map), proj cast to x's dtype
            if not x.is_cuda or self.proj.device != x.device:   # the reference moves proj to x's device
                return tensor_feature_map(x, self.proj.to(x.device))    # (raises for CPU tensors)
            return tensor_feature_map(x, self.proj, tables=self._tensor_tables(x))
        return x


class MultiheadRMSNorm(Module):
    """rnn_memory.py:139-147."""

    def __init__(self, dim: int, heads: int):
        super().__init__()
        self.scale = dim ** -0.5
        self.gamma = Parameter(torch.ones(heads, 1, dim))

    def forward(self, x: Tensor) -> Tensor:
        rms = x.norm(dim=-1, keepdim=True) * self.scale
        return (x / rms.clamp(min=1e-8)) * self.gamma


def _gate_head(dim: int, heads: int, bias: float) -> nn.Sequential:
    head = nn.Sequential(Linear(dim, heads), nn.Sigmoid())
    nn.init.zeros_(head[0].weight)
    nn.init.constant_(head[0].bias, bias)
    return head


class _CellBase(Module):
    """Parameters and prologue shared by both cells (rnn_memory.py:193-237, 482-534)."""

    def _build(self, dim, dim_head, heads, use_momentum, poly_degree, poly_mode, qk_norm, qkv_conv_kernel,
               use_accelerated_scan, scan_chunk_len, omega_window, use_omega_gate):
        self.dim = dim
        self.dim_head = dim_head
        self.heads = heads
        self.use_momentum = use_momentum
        self.qkv_conv_kernel = qkv_conv_kernel
        self.scan_chunk_len = scan_chunk_len
        self.omega_window = omega_window
        self.use_omega_gate = use_omega_gate
        self.assoc_scan = AssocScan(use_accelerated=use_accelerated_scan)
        dim_inner = dim_head * heads
        self.activation = nn.Identity()
        self.to_q = LinearNoBias(dim, dim_inner)
        self.to_k = LinearNoBias(dim, dim_inner)
        self.to_v = LinearNoBias(dim, dim_inner)
        self.to_out = LinearNoBias(dim_inner, dim)
        if exists(qkv_conv_kernel) and qkv_conv_kernel > 1:
            padding = qkv_conv_kernel // 2
            self.q_conv = Conv1d(dim, dim, qkv_conv_kernel, padding=padding, groups=dim, bias=False)
            self.k_conv = Conv1d(dim, dim, qkv_conv_kernel, padding=padding, groups=dim, bias=False)
            self.v_conv = Conv1d(dim, dim, qkv_conv_kernel, padding=padding, groups=dim, bias=False)
        else:
            self.q_conv = self.k_conv = self.v_conv = None
        self.to_lr = _gate_head(dim, heads, -4.0)
        self.to_decay = _gate_head(dim, heads, 4.0)
        self.to_momentum = _gate_head(dim, heads, 2.0) if use_momentum else None
        if use_omega_gate is not None:
            self.to_omega_gate = _gate_head(dim, heads, 0.0) if use_omega_gate else None
        self.pre_norm = nn.RMSNorm(dim)
        self.q_norm = MultiheadRMSNorm(dim_head, heads) if qk_norm else nn.Identity()
        self.k_norm = MultiheadRMSNorm(dim_head, heads) if qk_norm else nn.Identity()
        self.phi = PolynomialFeatureMap(dim_head, poly_degree, poly_mode)
        self.split_heads = Rearrange('b n (h d) -> b h n d', h=heads)
        self.merge_heads = Rearrange('b h n d -> b n (h d)')
        self.register_buffer('_dummy', torch.zeros(1))

    def init_state(self, batch: int, device=None, dtype=None) -> RNNMemState:
        """rnn_memory.py:239-248 / 536-554."""
        device = default(device, self._dummy.device)
        dtype = default(dtype, self._dummy.dtype)
        S = torch.zeros(batch * self.heads, self.dim_head, self.dim_head, device=device, dtype=dtype)
        Z = torch.zeros_like(S) if self.use_momentum else None
        buf = None
        if self.omega_window > 1:
            buf = torch.zeros(batch * self.heads, self.omega_window - 1, self.dim_head, self.dim_head,
                              device=device, dtype=dtype)
        return RNNMemState(seq_index=0, S=S, Z=Z, omega_buffer=buf)

    def _gate_heads(self):
        """The sigmoid gate heads in the order the fused prologue computes them."""
        heads = [self.to_lr, self.to_decay]
        if self.use_momentum:
            heads.append(self.to_momentum)
        if getattr(self, 'to_omega_gate', None) is not None:
            heads.append(self.to_omega_gate)
        return heads

    def _inputs(self, x: Tensor):
        """Pre-norm, the depthwise convs, the projections, the q / k norms, the gate heads and the
        feature map (rnn_memory.py:267-337, :572-653) -> the recurrence's operands
        k, q, v [BH, T, d] and lr, decay, beta, omega gate [BH, T]. The norms, convs, head split
        and gate sigmoids run in the fused prologue kernels (functional.cell_prologue); the
        projections are GEMMs."""
        heads = self._gate_heads()
        convs = (self.q_conv.weight, self.k_conv.weight, self.v_conv.weight) if exists(self.q_conv) else None
        qg = self.q_norm.gamma if isinstance(self.q_norm, MultiheadRMSNorm) else None
        kg = self.k_norm.gamma if isinstance(self.k_norm, MultiheadRMSNorm) else None
        eps = self.pre_norm.eps if self.pre_norm.eps is not None else torch.finfo(x.dtype).eps
        _, q, k, v, gates = cell_prologue(
            x, self.pre_norm.weight, eps, convs, (self.to_q.weight, self.to_k.weight, self.to_v.weight),
            [h[0].weight for h in heads], [h[0].bias for h in heads], qg, kg, self.heads, self.dim_head)
        if not self.phi.fused_elementwise:
            k = self.phi(k)
            q = self.phi(q)
        lr, decay = gates[0], gates[1]
        beta = gates[2] if self.use_momentum else None
        gate = gates[-1] if getattr(self, 'to_omega_gate', None) is not None else None
        return k, q, v, lr, decay, beta, gate

    def _memory(self, x, state, window) -> tuple[Tensor, RNNMemState]:
        batch, seq_len, _ = x.shape
        # a state the cell creates itself (init_state) is all zeros: S0 is passed as absent (one fp32
        # zero state, also S_ref) and Z and the omega buffer as absent (the kernels read absent as
        # zeros), which keeps the call on the specialised walks without materialising the zeros
        fresh = not exists(state)
        k, q, v, lr, decay, beta, gate = self._inputs(x)
        S0 = None if fresh else state.S
        Z0 = state.Z if (self.use_momentum and not fresh and exists(state.Z)) else None
        buf = state.omega_buffer if (window > 1 and not fresh) else None
        chunk = self.scan_chunk_len if (exists(self.scan_chunk_len) and seq_len > self.scan_chunk_len) else None
        y, S_T, Z_T, buf_out = memory_recurrence(
            k, q, v, lr, decay, beta, gate, S_ref=S0, S0=S0, Z0=Z0, buffer=buf, window=window,
            map_mode='elementwise' if self.phi.fused_elementwise else 'off', map_degree=self.phi.degree,
            clamp_every=chunk, clamp_final=True)
        y = rearrange(y.to(x.dtype), '(b h) t d -> b h t d', b=batch, h=self.heads)
        out = linear(self.merge_heads(y), self.to_out.weight)   # to_out on the library's bf16 products
        dt = x.dtype if fresh else S0.dtype   # init_state's dtype for a fresh state
        next_state = RNNMemState(
            seq_index=(0 if fresh else state.seq_index) + seq_len,
            S=S_T.to(dt),
            Z=Z_T.to(dt) if (self.use_momentum and exists(Z_T)) else None,
            omega_buffer=buf_out.to(dt) if exists(buf_out) else None,
        )
        return out, next_state


class RNNMemoryCell(_CellBase):
    """Titans-RNN cell (rnn_memory.py:154-408): the Omega recurrence with e = 1 and no gate."""

    def __init__(self, dim: int, dim_head: int = 64, heads: int = 1, use_momentum: bool = True,
                 poly_degree: int = 1, poly_mode: str = 'off', qk_norm: bool = True,
                 qkv_conv_kernel: int | None = 4, use_accelerated_scan: bool = False,
                 scan_chunk_len: int | None = None):
        super().__init__()
        self._build(dim, dim_head, heads, use_momentum, poly_degree, poly_mode, qk_norm, qkv_conv_kernel,
                    use_accelerated_scan, scan_chunk_len, omega_window=1, use_omega_gate=None)

    def forward(self, x: Tensor, state: RNNMemState | None = None) -> tuple[Tensor, RNNMemState]:
        return self._memory(x, state, 1)


class OmegaRNNMemoryCell(_CellBase):
    """OmegaNet-RNN cell (rnn_memory.py:415-814): gated sliding window of the outer products.

    use_cuda=True with omega_window == 16 follows the reference's CUDA-path semantics
    (rnn_memory.py:732-814): bf16 operands, beta = 1 without momentum, gate = 1 without the gate
    head, no clamp, no omega buffer carried; other windows warn and use the standard path
    (rnn_memory.py:456-458). Both paths run on the HIP kernels.
    """

    def __init__(self, dim: int, dim_head: int = 64, heads: int = 1, omega_window: int = 1,
                 use_omega_gate: bool = True, use_momentum: bool = True, poly_degree: int = 1,
                 poly_mode: str = 'off', qk_norm: bool = True, qkv_conv_kernel: int | None = 4,
                 use_accelerated_scan: bool = False, scan_chunk_len: int | None = None, use_cuda: bool = False):
        super().__init__()
        self.use_cuda = use_cuda
        self.cuda_available = False
        if use_cuda:
            if omega_window != 16:
                warnings.warn(f"CUDA backend only supports omega_window=16, got {omega_window}. "
                              "Falling back to PyTorch.")
                self.use_cuda = False
            else:
                available, msg = check_cuda_availability()
                if not available:
                    warnings.warn(f"CUDA not available: {msg}. Falling back to PyTorch.")
                    self.use_cuda = False
                else:
                    self.AtlasOmegaFunction = AtlasOmegaFunction
                    self.cuda_available = True
        self._build(dim, dim_head, heads, use_momentum, poly_degree, poly_mode, qk_norm, qkv_conv_kernel,
                    use_accelerated_scan, scan_chunk_len, omega_window=omega_window,
                    use_omega_gate=use_omega_gate)
        if self.use_cuda and self.cuda_available:
            self.assoc_scan = None

    def forward(self, x: Tensor, state: RNNMemState | None = None) -> tuple[Tensor, RNNMemState]:
        if self.use_cuda and self.cuda_available:
            return self._forward_cuda(x, state)
        return self._memory(x, state, self.omega_window)

    def _forward_cuda(self, x: Tensor, state: RNNMemState | None) -> tuple[Tensor, RNNMemState]:
        """rnn_memory.py:732-814, inside the scan_chunk_len loop of rnn_memory.py:584-601: every
        chunk is one call with S_ref = the call-start state and an empty window. The chunk's Z_T
        becomes the next chunk's Z0 only with momentum: without it the reference's next state has
        Z = None (rnn_memory.py:810), so every chunk starts from Z0 = 0 (:781) with beta = 1."""
        batch, seq_len, _ = x.shape
        if not exists(state):
            state = self.init_state(batch, x.device, x.dtype)
        k, q, v, lr, decay, beta, gate = self._inputs(x)
        if self.phi.fused_elementwise:
            k = self.phi(k)
            q = self.phi(q)
        if beta is None:
            beta = torch.ones_like(lr)
        if gate is None:
            gate = torch.ones_like(lr)
        BH, d = k.shape[0], self.dim_head
        bf = torch.bfloat16
        S_ref = state.S.to(bf).float()
        S = state.S if exists(state.S) else k.new_zeros((BH, d, d))
        zeros = k.new_zeros((BH, d, d))
        Z = state.Z if (self.use_momentum and exists(state.Z)) else zeros
        chunk = self.scan_chunk_len if (exists(self.scan_chunk_len) and seq_len > self.scan_chunk_len) else seq_len
        ys = []
        for start in range(0, seq_len, chunk):
            sl = slice(start, min(seq_len, start + chunk))
            y, S_T, Z_T = self.AtlasOmegaFunction.apply(
                k[:, sl].to(bf), q[:, sl].to(bf), v[:, sl].to(bf), S_ref, lr[:, sl].to(bf), decay[:, sl].to(bf),
                beta[:, sl].to(bf), gate[:, sl].to(bf), S.to(bf).float(), Z.to(bf).float())
            ys.append(y.to(x.dtype))
            S = S_T.to(x.dtype)
            Z = Z_T.to(x.dtype) if self.use_momentum else zeros
        y = torch.cat(ys, dim=1) if len(ys) > 1 else ys[0]
        y = rearrange(y, '(b h) t d -> b h t d', b=batch, h=self.heads)
        out = linear(self.merge_heads(y), self.to_out.weight)   # to_out on the library's bf16 products
        next_state = RNNMemState(seq_index=state.seq_index + seq_len, S=S,
                                 Z=Z if self.use_momentum else None, omega_buffer=None)
        return out, next_state


class RNNMemory(Module):
    """Drop-in replacement for NeuralMemory (rnn_memory.py:821-881)."""

    def __init__(self, dim: int, dim_head: int | None = None, heads: int = 1, use_momentum: bool = True,
                 poly_degree: int = 1, poly_mode: str = 'off', omega_window: int = 1,
                 use_omega_gate: bool = False, chunk_size: int = 1, use_accelerated_scan: bool = False,
                 scan_chunk_len: int | None = None, use_cuda: bool = False, **kwargs):
        super().__init__()
        dim_head = default(dim_head, dim)
        if omega_window > 1 or use_omega_gate:
            self.cell = OmegaRNNMemoryCell(dim=dim, dim_head=dim_head, heads=heads, omega_window=omega_window,
                                           use_omega_gate=use_omega_gate, use_momentum=use_momentum,
                                           poly_degree=poly_degree, poly_mode=poly_mode,
                                           use_accelerated_scan=use_accelerated_scan,
                                           scan_chunk_len=scan_chunk_len, use_cuda=use_cuda, **kwargs)
        else:
            self.cell = RNNMemoryCell(dim=dim, dim_head=dim_head, heads=heads, use_momentum=use_momentum,
                                      poly_degree=poly_degree, poly_mode=poly_mode,
                                      use_accelerated_scan=use_accelerated_scan, scan_chunk_len=scan_chunk_len,
                                      **kwargs)

    def forward(self, seq: Tensor, state: RNNMemState | None = None, **kwargs) -> tuple[Tensor, RNNMemState]:
        return self.cell(seq, state)


OmegaRNNMemory = partial(RNNMemory, omega_window=4, use_omega_gate=True)
