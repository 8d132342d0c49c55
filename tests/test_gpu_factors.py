"""GPU parity of the carried buffer in rank-1 factored form (atlas_mem_step_factored,
atlas_buffer_factors, atlas_buffer_expand; functional.memory_step_factored / buffer_factors /
expand_buffer_factors).

* Factored decode: T tokens stepped one at a time with the buffer carried as factors
  [BH, e-1, 2d] must give the fp64 oracle's outputs over the same T tokens in one call
  (rnn_memory.py:605-730 restated, with the dense buffer the starting factors stand for): every
  y_t, S_T, Z_T and, expanded, buffer_out. The same loop through the dense step (atlas_mem_step)
  must agree with it to fp32 round-off. fp32 rtol 1e-4, bf16 rtol 2e-2 (tests/_cases.compare).
* Prefill: the factors a T-token call leaves, expanded, are the oracle's buffer_out, including
  T < e - 1 (older slots shifted in from the starting factors).
* Expansion: bit-exact against the fp32 outer products formed on the CPU.
"""

import sys

import pytest
import torch

from _cases import Case, compare, make_inputs, run_oracle, tol_for

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16

FAC_CASES = [
    Case("fac_fp32_lag_e5", BH=3, T=12, d=64, e=5, gate='lag', momentum=True, buffer=True, states=0.3,
         backward=False, seed=60),
    Case("fac_fp32_token_e3_d32_map2", BH=2, T=9, d=32, e=3, gate='token', momentum=True, buffer=True, states=0.3,
         map_degree=2, backward=False, seed=61),
    Case("fac_fp32_none_nomom_e2", BH=2, T=7, d=32, e=2, gate=None, momentum=False, buffer=True, states=0.3,
         backward=False, seed=62),
    Case("fac_bf16_c3_shape", BH=32, T=16, d=64, e=4, gate='lag', momentum=True, buffer=True, states=0.1,
         dtype=BF16, backward=False, seed=63),
    Case("fac_bf16_max_window_fresh", BH=2, T=40, d=64, e=33, gate='lag', momentum=True, buffer=False,
         states=0.1, dtype=BF16, backward=False, seed=64),
]

PREFILL_CASES = FAC_CASES + [
    Case("pre_fp32_short_token", BH=2, T=5, d=32, e=9, gate='token', momentum=True, buffer=True, states=0.3,
         backward=False, seed=65),
    Case("pre_bf16_short_none_map3", BH=3, T=2, d=64, e=4, gate=None, momentum=False, buffer=True, states=0.1,
         map_degree=3, dtype=BF16, backward=False, seed=66),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _start_factors(c: Case, p: dict):
    """Random starting factors (or None) and the dense buffer they stand for (fp32 outer products)."""
    if not (c.buffer and c.e > 1):
        p["buffer"] = None
        return None
    g = torch.Generator().manual_seed(2000 + c.seed)
    dl = 0.3 * torch.randn(c.BH, c.e - 1, c.d, generator=g)
    ph = torch.randn(c.BH, c.e - 1, c.d, generator=g)
    ph = ph / ph.norm(dim=-1, keepdim=True)
    f = torch.cat([dl, ph], dim=-1)
    p["buffer"] = torch.einsum('bmi,bmk->bmik', dl, ph)
    return f


def _dev(c: Case, p: dict):
    out = {}
    for kk in ("k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0"):
        if p[kk] is None:
            out[kk] = None
            continue
        dt = c.dtype if kk in ("k", "q", "v", "lr", "decay", "beta", "gate") else torch.float32
        out[kk] = p[kk].to(device="cuda", dtype=dt)
    return out


@pytest.mark.parametrize("c", FAC_CASES, ids=lambda c: c.name)
def test_factored_decode_parity(c):
    from atlas_rnn_amd.functional import expand_buffer_factors, memory_recurrence, memory_step_factored
    _say(f"factored decode {c.name}")
    p = make_inputs(c)
    f0 = _start_factors(c, p)
    ref, _ = run_oracle(c, p)
    x = _dev(c, p)
    mm = dict(map_mode='elementwise' if c.map_degree > 1 else 'off', map_degree=c.map_degree)
    ys, yd = [], []
    with torch.no_grad():
        S, Z, F = x["S0"], x["Z0"], (f0.cuda() if f0 is not None else None)
        Sd, Zd, Bd = x["S0"], x["Z0"], (p["buffer"].cuda() if p["buffer"] is not None else None)
        for t in range(c.T):
            sl = slice(t, t + 1)
            tok = [x[kk][:, sl] if x[kk] is not None else None for kk in ("k", "q", "v", "lr", "decay", "beta", "gate")]
            y, S, Z, F = memory_step_factored(*tok, x["S_ref"], S, Z, F, window=c.e, **mm)
            ys.append(y)
            y2, Sd, Zd, Bd = memory_recurrence(*tok, x["S_ref"], Sd, Zd, Bd, window=c.e, **mm)   # dense step
            yd.append(y2)
        B = expand_buffer_factors(F) if F is not None else None
    torch.cuda.synchronize()
    tol = tol_for(c)
    y_all = torch.cat(ys, 1).float().cpu()
    compare(f"{c.name}.y", y_all, ref[0], tol)
    compare(f"{c.name}.S_T", S.cpu(), ref[1], tol)
    if c.momentum:
        compare(f"{c.name}.Z_T", Z.cpu(), ref[2], tol)
    compare(f"{c.name}.buffer_out", B.cpu(), ref[3], tol)
    # against the dense step: the same arithmetic apart from the order of the window sum's products
    tight = 1e-5 if c.dtype == torch.float32 else 1e-2
    compare(f"{c.name}.y_vs_dense", y_all, torch.cat(yd, 1).float().cpu(), tight)
    compare(f"{c.name}.S_vs_dense", S.cpu(), Sd.cpu(), tight)
    compare(f"{c.name}.B_vs_dense", B.cpu(), Bd.cpu(), tight)


@pytest.mark.parametrize("c", PREFILL_CASES, ids=lambda c: c.name)
def test_prefill_factors(c):
    from atlas_rnn_amd.functional import buffer_factors, expand_buffer_factors
    _say(f"prefill factors {c.name}")
    p = make_inputs(c)
    f0 = _start_factors(c, p)
    ref, _ = run_oracle(c, p)
    x = _dev(c, p)
    with torch.no_grad():
        F = buffer_factors(x["k"], x["v"], x["gate"], x["S_ref"], f0.cuda() if f0 is not None else None,
                           window=c.e, map_mode='elementwise' if c.map_degree > 1 else 'off',
                           map_degree=c.map_degree)
        B = expand_buffer_factors(F)
    torch.cuda.synchronize()
    assert F.shape == (c.BH, c.e - 1, 2 * c.d)
    compare(f"{c.name}.buffer_out", B.cpu(), ref[3], 1e-5 if c.dtype == torch.float32 else 1e-4)


@pytest.mark.parametrize("bh,slots,dv,dk", [(3, 4, 64, 64), (2, 1, 32, 32), (5, 32, 64, 64), (1, 3, 48, 80)])
def test_expand_exact(bh, slots, dv, dk):
    from atlas_rnn_amd.functional import expand_buffer_factors
    _say(f"expand {bh} {slots} {dv} {dk}")
    g = torch.Generator().manual_seed(bh * 100 + slots)
    f = torch.randn(bh, slots, dv + dk, generator=g)
    want = torch.einsum('bmi,bmk->bmik', f[..., :dv], f[..., dv:])
    got = expand_buffer_factors(f.cuda(), d_v=dv)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)
