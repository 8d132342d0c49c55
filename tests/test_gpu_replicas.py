"""GPU check of atlas_replicas, the block stacking's scalar copies and their adjoint sums: replicate
must equal torch's repeat along the first axis, and the replica sum must equal the fp32 sum of the
replicas in order 0, 1, ... rounded once to the dtype, bit for bit. Covers bf16 and fp32, 16-byte
vector arrays (n % 8 == 0, aligned) and the element path (odd n, a view one element into its
storage), two to five replicas, up to four arrays per launch, and the autograd pair through
functional._ReplicateFn / _ReplicaSumFn (each the other's adjoint).
"""

import sys

import pytest
import torch

from atlas_rnn_amd.functional import _REPLICA_SUM, _REPLICATE, _ReplicaSumFn, _ReplicateFn, _replicas

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _arrays(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(4 * 8192 + 1, generator=g).to(DEV, dtype)
    return [torch.randn(32, 4096, generator=g).to(DEV, dtype),        # vector path
            torch.randn(7, 333, generator=g).to(DEV, dtype),          # odd size: element path
            base[1:1 + 8192].view(64, 128),                           # one element into its storage
            torch.randn(16, 512, 8, generator=g).to(DEV, dtype)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("nrep", [2, 3, 5])
def test_replicate_and_sum_match_torch(dtype, nrep):
    _say(f"replicas dtype={dtype} nrep={nrep}")
    xs = _arrays(dtype, 100 + nrep)
    reps = _replicas(_REPLICATE, nrep, xs)
    torch.cuda.synchronize()
    for x, r in zip(xs, reps):
        want = x.repeat(nrep, *([1] * (x.dim() - 1)))
        assert torch.equal(r, want)
    stacked = [torch.randn(nrep * x.shape[0], *x.shape[1:], device=DEV).to(dtype) for x in xs]
    sums = _replicas(_REPLICA_SUM, nrep, stacked)
    torch.cuda.synchronize()
    for st, got in zip(stacked, sums):
        parts = st.float().reshape(nrep, -1, *st.shape[1:])
        acc = torch.zeros_like(parts[0])
        for r in range(nrep):
            acc = acc + parts[r]
        assert torch.equal(got, acc.to(dtype))


def test_autograd_pair_is_adjoint():
    _say("replicas through autograd")
    g = torch.Generator().manual_seed(7)
    x = torch.randn(32, 1000, generator=g).to(DEV, torch.bfloat16).requires_grad_(True)
    y = torch.randn(32, 1000, 8, generator=g).to(DEV, torch.bfloat16).requires_grad_(True)
    rx, ry = _ReplicateFn.apply(2, x, y)
    gx = torch.randn(rx.shape, generator=g).to(DEV, torch.bfloat16)
    gy = torch.randn(ry.shape, generator=g).to(DEV, torch.bfloat16)
    dx, dy = torch.autograd.grad((rx, ry), (x, y), grad_outputs=(gx, gy))
    torch.cuda.synchronize()
    assert torch.equal(dx, (gx.float()[:32] + gx.float()[32:]).to(torch.bfloat16))
    assert torch.equal(dy, (gy.float()[:32] + gy.float()[32:]).to(torch.bfloat16))
    z = torch.randn(64, 1000, generator=g).to(DEV, torch.float32).requires_grad_(True)
    (s,) = _ReplicaSumFn.apply(2, z)
    gs = torch.randn(s.shape, generator=g).to(DEV)
    (dz,) = torch.autograd.grad(s, z, grad_outputs=gs)
    torch.cuda.synchronize()
    assert torch.equal(s, z.detach()[:32] + z.detach()[32:])
    assert torch.equal(dz, torch.cat([gs, gs]))
