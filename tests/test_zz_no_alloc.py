"""atlas_mem_bwd_noalloc (static device scratch, no allocation) against atlas_mem_bwd (caller workspace),
through the C ABI: two calls in a row on one GPU, the second with a smaller problem, every gradient
compared (fp32 rtol 1e-4, bf16 rtol 2e-2, normwise and elementwise; the two runs differ only in
the order of LDS atomic additions)."""

import ctypes
import sys

import pytest
import torch

from _cases import Case, compare, make_inputs, tol_for
from atlas_rnn_amd import _lib
from atlas_rnn_amd.functional import RecurrencePlan

pytestmark = pytest.mark.gpu

GRADS = ("k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buffer")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _run_pair(case: Case):
    lib = _lib.load()
    p = make_inputs(case)
    dev = torch.device("cuda")
    dt = case.dtype
    x = {}
    for kk in ("k", "q", "v", "lr", "decay", "beta", "gate"):
        x[kk] = p[kk].to(dev, dt).contiguous() if p[kk] is not None else None
    for kk in ("S_ref", "S0", "Z0", "buffer"):
        x[kk] = p[kk].to(dev, torch.float32).contiguous() if p[kk] is not None else None
    plan = RecurrencePlan(case.BH, case.T, case.d, window=case.e, momentum=case.momentum, gate_mode=case.gate,
                          dtype=dt, has_buffer=x["buffer"] is not None, device=dev)
    plan.forward(x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"], x["S_ref"], x["S0"], x["Z0"],
                 x["buffer"])
    dy = p["gy"].to(dev, dt).contiguous()
    dS = p["gS"].to(dev).contiguous()
    ref = {kk: v.clone() for kk, v in plan.backward(dy, dS).items() if v is not None}
    # the same backward through the allocation-free entry point, into fresh gradient tensors
    out = {kk: torch.full_like(v, float("nan")) for kk, v in ref.items()}
    ptr = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)
    a = _lib.BwdArgs(k=ptr(x["k"]), q=ptr(x["q"]), v=ptr(x["v"]), lr=ptr(x["lr"]), decay=ptr(x["decay"]),
                     beta=ptr(x["beta"]), gate=ptr(x["gate"]), S_ref=ptr(x["S_ref"]), S0=ptr(x["S0"]),
                     Z0=ptr(x["Z0"]), buffer_in=ptr(x["buffer"]), dy=ptr(dy), dS_T=ptr(dS), dZ_T=ptr(None),
                     dbuffer_out=ptr(None), dk=ptr(out["k"]), dq=ptr(out["q"]), dv=ptr(out["v"]),
                     dlr=ptr(out["lr"]), ddecay=ptr(out["decay"]), dbeta=ptr(out.get("beta")),
                     dgate=ptr(out.get("gate")), dS_ref=ptr(out["S_ref"]), dS0=ptr(out["S0"]),
                     dZ0=ptr(out.get("Z0")), dbuffer_in=ptr(out.get("buffer")))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.atlas_mem_bwd_noalloc(ctypes.byref(plan.prob), ctypes.byref(a), ptr(plan.saved), stream),
               "atlas_mem_bwd_noalloc")
    torch.cuda.synchronize()
    tol = tol_for(case)
    for kk in ref:
        compare(f"{case.name}.noalloc.d{kk}", out[kk].float().cpu(), ref[kk].float().cpu(), tol)
    return len(ref)


def test_noalloc_backward_matches_workspace_backward_twice():
    lib = _lib.load()
    assert lib.atlas_mem_noalloc_scratch_bytes() == 64 << 20
    # first call: the headline's layout (bf16, d 64, lag gates, specialised walks), 23 MiB of workspace
    big = Case("noalloc_big", BH=16, T=2048, d=64, e=4, gate='lag', momentum=True, dtype=torch.bfloat16, seed=61)
    # second call, smaller: fp32, d 32, token gates, a carried buffer (the general kernels); the
    # array keeps the first call's contents, which the backward overwrites before it reads
    small = Case("noalloc_small", BH=3, T=150, d=32, e=3, gate='token', momentum=True, buffer=True, states=0.1,
                 seed=62)
    for c in (big, small):
        _say(f"noalloc backward {c.name}: BH={c.BH} T={c.T} d={c.d} e={c.e} gate={c.gate} dtype={c.dtype}")
        n = _run_pair(c)
        _say(f"  {n} gradients equal the workspace backward's")
