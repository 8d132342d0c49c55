"""GPU parity of the one-token step (atlas_mem_step; memory_recurrence routes T = 1 calls without
autograd to it): against the fp64 oracle's per-token loop restatement, against the chunked forward
at T = 1, in place through the C ABI, and as decode: T steps carrying (S, Z, buffer) must give what
one call over the T tokens gives (the generation loop of atlas_pytorch/rnn_transformer.py:863-900
against prefill). Tolerances as in the recurrence parity tests: fp32 rtol 1e-4, bf16 rtol 2e-2,
with an atol floor of tol * max|ref| per tensor.
"""

import ctypes
import sys
from dataclasses import replace

import pytest
import torch

from _cases import Case, compare, make_inputs, run_gpu, run_oracle, tol_for

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
OUTS = ("y", "S_T", "Z_T", "buffer_out")

STEP_CASES = [
    Case("step_fp32_nogate", BH=3, T=1, d=64, e=1, gate=None, momentum=True, states=0.3, backward=False, seed=40),
    Case("step_fp32_token_buf_d32", BH=3, T=1, d=32, e=3, gate='token', momentum=True, buffer=True, states=0.3,
         backward=False, seed=41),
    Case("step_fp32_lag_buf", BH=2, T=1, d=64, e=5, gate='lag', momentum=True, buffer=True, states=0.3,
         backward=False, seed=42),
    Case("step_fp32_nomom_map2", BH=2, T=1, d=32, e=2, gate=None, momentum=False, buffer=True, states=0.3,
         map_degree=2, backward=False, seed=43),
    Case("step_fp32_clamp", BH=2, T=1, d=32, e=2, gate='token', momentum=True, states=150.0, decay_shift=7.0,
         backward=False, seed=44),
    Case("step_fp32_no_final_clamp", BH=2, T=1, d=32, e=1, gate=None, momentum=True, states=150.0,
         decay_shift=7.0, clamp_final=False, backward=False, seed=45),
    Case("step_fp32_d16_padded", BH=2, T=1, d=16, e=3, gate='lag', momentum=True, buffer=True, states=0.3,
         backward=False, seed=46),
    Case("step_bf16_c3_shape", BH=32, T=1, d=64, e=4, gate='lag', momentum=True, buffer=True, states=0.1,
         dtype=BF16, backward=False, seed=47),
    Case("step_bf16_max_window", BH=2, T=1, d=64, e=33, gate='lag', momentum=True, buffer=True, states=0.1,
         dtype=BF16, backward=False, seed=48),
    Case("step_bf16_token_nobuf", BH=4, T=1, d=64, e=16, gate='token', momentum=True, states=0.1, dtype=BF16,
         backward=False, seed=49),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(c, got, ref, tol):
    for name, g_, r_ in zip(OUTS, got, ref):
        if r_ is None:
            assert g_ is None, f"{c.name}.{name}: expected no output"
            continue
        compare(f"{c.name}.{name}", g_, r_, tol)


@pytest.mark.parametrize("c", STEP_CASES, ids=lambda c: c.name)
def test_step_parity(c):
    _say(f"step parity {c.name}")
    p = make_inputs(c)
    ref, _ = run_oracle(c, p)
    got, _ = run_gpu(c, p)
    _check(c, got, ref, tol_for(c))


@pytest.mark.parametrize("c", [STEP_CASES[2], STEP_CASES[3], STEP_CASES[7]], ids=lambda c: c.name)
def test_step_matches_chunked_forward(c):
    """The same T = 1 inputs through the step (no autograd) and the chunked forward (inputs that
    require grad take the autograd path)."""
    _say(f"step vs chunked forward {c.name}")
    p = make_inputs(c)
    got_step, _ = run_gpu(c, p)
    got_full, _ = run_gpu(replace(c, backward=True), p)
    _check(c, got_step, got_full, 1e-5 if c.dtype == torch.float32 else 1e-2)


def test_decode_equals_prefill():
    c = Case("decode", BH=4, T=24, d=64, e=4, gate='lag', momentum=True, buffer=True, states=0.3, backward=False,
             seed=50)
    _say("decode vs prefill")
    from atlas_rnn_amd.functional import memory_recurrence
    p = make_inputs(c)
    x = {kk: (v.cuda() if v is not None else None) for kk, v in p.items()}
    with torch.no_grad():
        y_all, S_all, Z_all, B_all = memory_recurrence(
            x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"], x["S_ref"], x["S0"], x["Z0"],
            x["buffer"], window=c.e)
        S, Z, B = x["S0"], x["Z0"], x["buffer"]
        ys = []
        for t in range(c.T):
            sl = slice(t, t + 1)
            y, S, Z, B = memory_recurrence(
                x["k"][:, sl], x["q"][:, sl], x["v"][:, sl], x["lr"][:, sl], x["decay"][:, sl], x["beta"][:, sl],
                x["gate"][:, sl], x["S_ref"], S, Z, B, window=c.e)
            ys.append(y)
    torch.cuda.synchronize()
    assert S_all.abs().max().item() < 100.0   # the per-step clamp is inactive, so the two must agree
    compare("decode.y", torch.cat(ys, 1).cpu(), y_all.cpu(), 1e-4)
    compare("decode.S_T", S.cpu(), S_all.cpu(), 1e-4)
    compare("decode.Z_T", Z.cpu(), Z_all.cpu(), 1e-4)
    compare("decode.buffer", B.cpu(), B_all.cpu(), 1e-4)


def test_step_in_place_through_abi():
    """S_T = S0, Z_T = Z0 and buffer_out = buffer_in in one call give the out-of-place results."""
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import RecurrenceConfig, _problem, _ptr, _stream
    c = STEP_CASES[7]
    _say("step in place")
    p = make_inputs(c)
    dev = torch.device("cuda")
    x = {kk: (v.to(dev, c.dtype if kk in ("k", "q", "v", "lr", "decay", "beta", "gate") else torch.float32)
              .contiguous() if v is not None else None) for kk, v in p.items()}
    lib = _lib.load()
    cfg = RecurrenceConfig(window=c.e)
    prob = _problem(cfg, c.BH, 1, c.d, c.d, True, x["gate"], True, c.dtype)

    def call(S_T, Z_T, B_out, S0, Z0, B_in):
        y = torch.empty(c.BH, 1, c.d, device=dev, dtype=c.dtype)
        a = _lib.FwdArgs(k=_ptr(x["k"]), q=_ptr(x["q"]), v=_ptr(x["v"]), lr=_ptr(x["lr"]), decay=_ptr(x["decay"]),
                         beta=_ptr(x["beta"]), gate=_ptr(x["gate"]), S_ref=_ptr(x["S_ref"]), S0=_ptr(S0),
                         Z0=_ptr(Z0), buffer_in=_ptr(B_in), y=_ptr(y), S_T=_ptr(S_T), Z_T=_ptr(Z_T),
                         buffer_out=_ptr(B_out))
        _lib.check(lib.atlas_mem_step(ctypes.byref(prob), ctypes.byref(a), _stream(dev)), "atlas_mem_step")
        return y

    S_o, Z_o, B_o = (torch.empty_like(x["S0"]), torch.empty_like(x["Z0"]), torch.empty_like(x["buffer"]))
    y_o = call(S_o, Z_o, B_o, x["S0"], x["Z0"], x["buffer"])
    S_i, Z_i, B_i = x["S0"].clone(), x["Z0"].clone(), x["buffer"].clone()
    y_i = call(S_i, Z_i, B_i, S_i, Z_i, B_i)
    torch.cuda.synchronize()
    assert torch.equal(y_i, y_o)
    assert torch.equal(S_i, S_o) and torch.equal(Z_i, Z_o) and torch.equal(B_i, B_o)
