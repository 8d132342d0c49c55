"""Host-side operand checks (no GPU): every shape, dtype and device mismatch is refused with a
ValueError before any pointer reaches the C ABI (functional.check_operands, called by
memory_recurrence, MemoryRecurrenceFn and RecurrencePlan)."""

import pytest
import torch

from atlas_rnn_amd.functional import check_operands

BH, T, D, E = 4, 10, 8, 4


def _ops(**over):
    z = lambda *s: torch.zeros(*s)
    ops = dict(k=z(BH, T, D), q=z(BH, T, D), v=z(BH, T, D), lr=z(BH, T), decay=z(BH, T), beta=z(BH, T),
               gate=z(BH, T, E), S_ref=z(BH, D, D), S0=z(BH, D, D), Z0=z(BH, D, D), buffer=z(BH, E - 1, D, D))
    ops.update(over)
    return ops


def _check(window=E, **over):
    o = _ops(**over)
    check_operands(o["k"], o["q"], o["v"], o["lr"], o["decay"], o["beta"], o["gate"], o["S_ref"], o["S0"],
                   o["Z0"], o["buffer"], window=window)


def test_consistent_operands_pass():
    _check()
    _check(gate=torch.zeros(BH, T))                           # per-token gate
    _check(gate=None, beta=None, Z0=None, buffer=None)
    _check(v=torch.zeros(BH, T, 2 * D), S_ref=torch.zeros(BH, 2 * D, D), S0=torch.zeros(BH, 2 * D, D),
           Z0=torch.zeros(BH, 2 * D, D), buffer=torch.zeros(BH, E - 1, 2 * D, D))   # d_v != d_k
    _check(window=1, gate=torch.zeros(BH, T, 1), buffer=None)


@pytest.mark.parametrize("name,bad", [
    ("gate", torch.zeros(BH, T, E + 12)),       # a [BH, T, 16] gate with window 4 would be over-read
    ("gate", torch.zeros(BH, T, 2)),
    ("gate", torch.zeros(BH, T, E, 1)),
    ("gate", torch.zeros(BH, T + 1)),
    ("lr", torch.zeros(BH, T + 1)),
    ("decay", torch.zeros(BH - 1, T)),
    ("beta", torch.zeros(BH, T, 1)),
    ("q", torch.zeros(BH, T, D + 1)),
    ("v", torch.zeros(BH, T - 1, D)),
    ("S_ref", torch.zeros(BH, D, D + 1)),
    ("S0", torch.zeros(BH + 1, D, D)),
    ("Z0", torch.zeros(BH, D)),
    ("buffer", torch.zeros(BH, E, D, D)),
    ("buffer", torch.zeros(BH, E - 1, D, D - 1)),
])
def test_mismatched_shapes_are_refused(name, bad):
    with pytest.raises(ValueError, match=name if name != "gate" else "gate"):
        _check(**{name: bad})


def test_k_must_be_three_dimensional():
    with pytest.raises(ValueError, match="k must be"):
        _check(k=torch.zeros(BH * T, D))


def test_dtype_and_contiguity_when_requested():
    o = _ops()
    args = [o[n] for n in ("k", "q", "v", "lr", "decay", "beta", "gate", "S_ref", "S0", "Z0", "buffer")]
    check_operands(*args, window=E, dtype=torch.float32, contiguous=True)
    with pytest.raises(ValueError, match="must be torch.bfloat16"):
        check_operands(*args, window=E, dtype=torch.bfloat16)
    nc = torch.zeros(BH, D, T).transpose(1, 2)
    with pytest.raises(ValueError, match="contiguous"):
        check_operands(nc, *args[1:], window=E, contiguous=True)
    # states stay fp32 whatever the input dtype
    half = [a.to(torch.bfloat16) if i < 7 else a for i, a in enumerate(args)]
    check_operands(*half, window=E, dtype=torch.bfloat16, contiguous=True)
    bad_state = list(half)
    bad_state[7] = bad_state[7].to(torch.bfloat16)
    with pytest.raises(ValueError, match="S_ref must be torch.float32"):
        check_operands(*bad_state, window=E, dtype=torch.bfloat16)
