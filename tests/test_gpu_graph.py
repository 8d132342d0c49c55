"""The memory cell's forward + backward captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

The library makes no host synchronisation, allocation or memset on this path (every buffer comes
from torch's allocator, every launch goes to the current stream), so a caller can capture the whole
training step of OmegaRNNMemoryCell (rnn_memory.py:556-603 and the prologue :567-653) and replay
it. Each replay follows eager work of the same step and a synchronisation, and is checked against
the eager result bit for bit: the output, the final state and every parameter gradient (the bf16
d = 64 kernels this cell runs sum in a fixed order, so the step is reproducible; a stale or
skipped node would be off by O(1)). Fresh and carried states, scan_chunk_len set (the two launch
sequences chosen on the device by the clamp flag).
"""

import sys

import pytest
import torch

import atlas_rnn_amd as am

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _normwise(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("carried", [False, True], ids=["fresh_state", "carried_state"])
def test_cell_step_graph_replays_match_eager(carried):
    _say(f"graph capture of the cell step, carried={carried}")
    torch.cuda.set_device(DEV)
    torch.manual_seed(2024)
    B, T, heads, d = 2, 1024, 4, 64
    dim = heads * d
    cell = am.OmegaRNNMemoryCell(dim=dim, dim_head=d, heads=heads, omega_window=4, use_omega_gate=True,
                                 use_momentum=True, scan_chunk_len=64).to(DEV, torch.bfloat16)
    with torch.no_grad():   # non-constant gates
        for p in cell.parameters():
            if p.ndim == 2 and p.shape[0] == heads:
                p.normal_(0, 0.02)
    g = torch.Generator().manual_seed(2025)
    x = torch.randn(B, T, dim, generator=g).to(DEV, torch.bfloat16)
    gy = torch.randn(B, T, dim, generator=g).to(DEV, torch.bfloat16)
    params = list(cell.parameters())
    state = None
    if carried:
        with torch.no_grad():
            _, st = cell(x)
        state = am.state_detach(st)

    def step():
        out, st = cell(x, state)
        grads = torch.autograd.grad(out, params, grad_outputs=gy)
        return (out.detach(), st.S.detach()) + tuple(grads)

    ref = [t.clone() for t in step()]
    side = torch.cuda.Stream()   # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    torch.cuda.synchronize()
    names = ["out", "S"] + [n for n, _ in cell.named_parameters()]
    for r in range(3):
        step()                     # eager work of the same step between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(names, static, ref):
            assert torch.isfinite(got.double()).all(), f"replay {r}: {name} not finite"
            assert torch.equal(got, want), \
                f"replay {r}: {name} differs from the eager step (normwise {_normwise(got, want):.3e})"
    del graph
