"""GPU parity of the batched linear-layer products (atlas_linear_batch: C = A B^T or A B, bf16 operands,
fp32 accumulation, bf16 out, up to four problems per launch) against the fp64 product of the same
bf16 values. These are the products autograd forms for the cell's projections (rnn_memory.py:486-489)
and gate heads (:503-520), forward (NT) and input gradient (NN).

Bound, elementwise: |C - ref| <= 1e-5 (|A| |B|) + half a bf16 unit of |ref| (the bf16 output rounding).
Cases: the prologue's four projections in one launch (three 512-wide and the 32-wide gate heads),
their four input gradients (the gate heads' with k = 32), rows not a multiple of the 128-row tile,
widths not multiples of 128, a single problem, and m = 0.
"""

import ctypes
import sys

import pytest
import torch

from atlas_rnn_amd import _lib
from atlas_rnn_amd.functional import _GEMM_NN, _GEMM_NT, _products, _stream

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(c, a, b, layout):
    a64, b64 = a.double().reshape(-1, a.shape[-1]), b.double()
    bm = b64.t() if layout == _GEMM_NT else b64
    ref = a64 @ bm
    scale = a64.abs() @ bm.abs()
    got = c.double().reshape(ref.shape)
    bound = 1e-5 * scale + 2.0 ** -8 * ref.abs() + 1e-30
    worst = ((got - ref).abs() / bound).max().item()
    assert torch.isfinite(got).all()
    assert worst <= 1.0, f"max err / bound = {worst:.3g}"


def _rand(g, *shape):
    return torch.randn(*shape, generator=g).to(DEV, torch.bfloat16)


CASES = [
    # (name, layout, m, [(n, k), ...])
    ("prologue_fwd", _GEMM_NT, 16384, [(512, 512), (512, 512), (512, 512), (32, 512)]),
    ("prologue_dx", _GEMM_NN, 16384, [(512, 512), (512, 512), (512, 512), (512, 32)]),
    ("ragged_nt", _GEMM_NT, 1000, [(200, 72), (64, 24)]),
    ("ragged_nn", _GEMM_NN, 777, [(96, 40), (136, 200), (8, 8)]),
    ("single_nt", _GEMM_NT, 130, [(256, 1024)]),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_linear_batch_matches_fp64(case):
    name, layout, m, dims = case
    _say(f"gemm {name}")
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    acts = [_rand(g, m, k) for n, k in dims]
    ws = [_rand(g, n, k) if layout == _GEMM_NT else _rand(g, k, n) for n, k in dims]
    outs = _products(layout, acts, ws)
    torch.cuda.synchronize()
    for c, a, b in zip(outs, acts, ws):
        _check(c, a, b, layout)


def test_linear_batch_leading_axes_and_empty():
    _say("gemm [B, T, k] activations and m = 0")
    g = torch.Generator().manual_seed(5)
    x = _rand(g, 2, 300, 64)
    w = _rand(g, 48, 64)
    y = _products(_GEMM_NT, [x], [w])[0]
    torch.cuda.synchronize()
    assert y.shape == (2, 300, 48)
    _check(y, x, w, _GEMM_NT)
    lib = _lib.load()
    e = torch.empty(0, 64, device=DEV, dtype=torch.bfloat16)
    I32, VP = ctypes.c_int * 1, ctypes.c_void_p * 1
    assert lib.atlas_linear_batch(_GEMM_NT, 1, 0, I32(48), I32(64), VP(None), VP(w.data_ptr()), VP(None),
                                  _stream(DEV)) == 0
