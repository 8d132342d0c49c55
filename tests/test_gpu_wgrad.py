"""GPU parity of the linear layers' weight gradient (atlas_linear_wgrad: dW = dy^T x over the tokens,
bf16 operands read as stored, fp32 partials over token splits summed in a fixed order) against the
fp64 product of the same bf16 values. This is the weight gradient autograd forms for the cell's
projections (rnn_memory.py:486-489) and gate heads (:503-520).

Bound, elementwise: |dW - ref| <= 1e-5 (|dy|^T |x|) for fp32 dW (fp32 accumulation over at most 16384
terms), plus half a bf16 unit of |ref| for bf16 dW. Shapes: the cell's projections (16384 tokens,
512 x 512), its gate heads (32 rows), partial 128-tiles on both axes, fewer tokens than one K step,
no tokens (dW = 0), and two calls in a row on one workspace, the second smaller.
"""

import sys

import pytest
import torch

from atlas_rnn_amd import _lib
from atlas_rnn_amd.functional import _ptr, _stream, _wgrad

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ref(dy, x):
    """fp64 dy^T x and the scale |dy|^T |x| (on the GPU in fp64 for the large case)."""
    d64, x64 = dy.double(), x.double()
    return d64.t() @ x64, d64.abs().t() @ x64.abs()


def _call(lib, dy, x, out_dtype, ws=None):
    n, o = dy.shape
    i = x.shape[1]
    need = lib.atlas_linear_wgrad_workspace_bytes(n, o, i)
    assert need >= 0
    if ws is None or ws.numel() * 4 < need:
        ws = torch.empty(max(need, 16) // 4, device=DEV, dtype=torch.float32)
    dw = torch.full((o, i), float("nan"), device=DEV, dtype=out_dtype)
    code = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16}[out_dtype]
    _lib.check(lib.atlas_linear_wgrad(code, n, o, i, _ptr(dy), _ptr(x), _ptr(dw), _ptr(ws), ws.numel() * 4,
                                      _stream(DEV)), "atlas_linear_wgrad")
    torch.cuda.synchronize()
    return dw, ws


def _check(dw, dy, x, out_dtype):
    ref, scale = _ref(dy, x)
    err = (dw.double() - ref).abs()
    bound = 1e-5 * scale + 1e-30
    if out_dtype == torch.bfloat16:
        bound = bound + 2.0 ** -8 * ref.abs()
    assert torch.isfinite(dw.double()).all()
    worst = (err / bound).max().item()
    assert worst <= 1.0, f"max err / bound = {worst:.3g}"


CASES = [
    # (n, out_features, in_features, out dtype)
    (16384, 512, 512, torch.float32),
    (16384, 512, 512, torch.bfloat16),
    (1000, 32, 512, torch.bfloat16),
    (777, 200, 72, torch.float32),
    (33, 64, 24, torch.float32),
    (5000, 128, 1024, torch.bfloat16),
]


@pytest.mark.parametrize("n,o,i,odt", CASES)
def test_wgrad_matches_fp64(n, o, i, odt):
    _say(f"wgrad n={n} o={o} i={i} out={odt}")
    lib = _lib.load()
    g = torch.Generator(device="cpu").manual_seed(n + 7 * o + i)
    dy = torch.randn(n, o, generator=g).to(DEV, torch.bfloat16)
    x = torch.randn(n, i, generator=g).to(DEV, torch.bfloat16)
    dw, _ = _call(lib, dy, x, odt)
    _check(dw, dy, x, odt)


def test_wgrad_no_tokens_is_zero():
    _say("wgrad n=0")
    lib = _lib.load()
    dy = torch.empty(0, 64, device=DEV, dtype=torch.bfloat16)
    x = torch.empty(0, 48, device=DEV, dtype=torch.bfloat16)
    dw, _ = _call(lib, dy, x, torch.float32)
    assert (dw == 0).all()


def test_wgrad_reuses_workspace_on_a_smaller_call():
    _say("wgrad two calls, one workspace")
    lib = _lib.load()
    g = torch.Generator(device="cpu").manual_seed(11)
    dy1 = torch.randn(8192, 256, generator=g).to(DEV, torch.bfloat16)
    x1 = torch.randn(8192, 256, generator=g).to(DEV, torch.bfloat16)
    dy2 = torch.randn(300, 256, generator=g).to(DEV, torch.bfloat16)
    x2 = torch.randn(300, 256, generator=g).to(DEV, torch.bfloat16)
    dw1, ws = _call(lib, dy1, x1, torch.float32)
    dw2, _ = _call(lib, dy2, x2, torch.float32, ws)
    _check(dw1, dy1, x1, torch.float32)
    _check(dw2, dy2, x2, torch.float32)


def test_wgrad_through_the_linear_helper():
    """functional._wgrad flattens the leading axes ([B, T, o] activations) and returns dW in the
    weight's dtype."""
    _say("wgrad via functional._wgrad")
    g = torch.Generator(device="cpu").manual_seed(12)
    dy = torch.randn(2, 700, 96, generator=g).to(DEV, torch.bfloat16)
    x = torch.randn(2, 700, 40, generator=g).to(DEV, torch.bfloat16)
    dw = _wgrad(dy, x, torch.bfloat16)
    torch.cuda.synchronize()
    assert dw.dtype == torch.bfloat16 and dw.shape == (96, 40)
    _check(dw, dy.reshape(-1, 96), x.reshape(-1, 40), torch.bfloat16)


def test_wgrad_batch_of_the_prologue_layers():
    """atlas_linear_wgrad_batch through functional._wgrads: the prologue's q / k / v (512 x 512) and
    gate-head (32 x 512) weights over the same 16384 tokens in one launch, each against fp64."""
    from atlas_rnn_amd.functional import _wgrads
    _say("wgrad batch of four layers")
    g = torch.Generator(device="cpu").manual_seed(13)
    n = 16384
    pairs = [(torch.randn(n, o, generator=g).to(DEV, torch.bfloat16), torch.randn(n, 512, generator=g).to(DEV, torch.bfloat16))
             for o in (512, 512, 512, 32)]
    dws = _wgrads(pairs, torch.bfloat16)
    torch.cuda.synchronize()
    for dw, (dy, x) in zip(dws, pairs):
        assert dw.shape == (dy.shape[1], 512)
        _check(dw, dy, x, torch.bfloat16)
