"""GPU parity at the BASELINE configurations' full geometry, against the fp64 oracle on a subset of rows.

The GPU runs the whole problem (every head-batch row, the full sequence, the segment layout the
library plans for that size: C3 is 8 segments of 8 64-token chunks per row); rows are independent,
so the oracle runs only rows 0, middle and last (in 256-token blocks carrying the state,
`_cases.run_oracle_rows`) and those rows of every output and every gradient are compared:
y, S_T, Z_T, buffer_out, dk, dq, dv, dlr, ddecay, dbeta, dgate, dS_ref, dS0, dZ0 (and dbuffer).

Tolerance (bf16 inputs, fp32 state): normwise relative error <= 2e-2 per tensor and elementwise
|err| <= 2e-2 |ref| + 2e-2 max|ref| (`_cases.compare`).
"""

import sys

import pytest
import torch

from _cases import Case, compare, make_inputs, run_gpu, run_oracle_rows, tol_for

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16

CASES = [
    # C3 headline: B=4 H=8 T=4096 d=64, e=4 lag gates, momentum; the benchmark's loss (no buffer_out
    # gradient) and the full loss
    (Case("c3_full_bench_loss", BH=32, T=4096, d=64, e=4, gate='lag', momentum=True, dtype=BF16,
          grad_buffer=False, seed=101), (0, 15, 31)),
    (Case("c3_full", BH=32, T=4096, d=64, e=4, gate='lag', momentum=True, dtype=BF16, seed=102), (0, 15, 31)),
    # C3 as the drop-in cell calls it: a carried (zero) buffer
    (Case("c3_full_zero_buffer", BH=32, T=4096, d=64, e=4, gate='lag', momentum=True, buffer=True,
          buffer_scale=0.0, dtype=BF16, seed=103), (0, 15, 31)),
    # C3 with a carried nonzero buffer (a state from a previous call): the walks with its first-chunk terms
    (Case("c3_full_buffer", BH=32, T=4096, d=64, e=4, gate='lag', momentum=True, buffer=True, states=0.1,
          dtype=BF16, seed=108), (0, 31)),
    # C3 with scan_chunk_len = 64, as the drop-in cell runs it ("chunk 64"): segment-parallel with the
    # clamp points checked on the device
    (Case("c3_full_clamp64", BH=32, T=4096, d=64, e=4, gate='lag', momentum=True, clamp_every=64, dtype=BF16,
          seed=107), (0, 15, 31)),
    # C2: Titans with momentum, B=4 H=8 T=2048
    (Case("c2_full", BH=32, T=2048, d=64, e=1, gate=None, momentum=True, dtype=BF16, seed=104), (0, 15, 31)),
    # C5's memory core: B=8 H=8 T=2048, e=4 per-token gates (the cell's omega gate), momentum;
    # without and with the zero buffer the module passes
    (Case("c5_core_full", BH=64, T=2048, d=64, e=4, gate='token', momentum=True, dtype=BF16, seed=105),
     (0, 31, 63)),
    (Case("c5_core_full_zero_buffer", BH=64, T=2048, d=64, e=4, gate='token', momentum=True, buffer=True,
          buffer_scale=0.0, dtype=BF16, seed=106), (0, 31, 63)),
]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("case,rows", CASES, ids=[c.name for c, _ in CASES])
def test_full_geometry_rows_match_oracle(case, rows):
    _say(f"full geometry {case.name}: BH={case.BH} T={case.T} e={case.e} gate={case.gate} buffer={case.buffer} "
         f"rows={rows}")
    p = make_inputs(case)
    got_out, got_grads = run_gpu(case, p)
    _say(f"  gpu done; oracle on rows {rows}")
    ref_out, ref_grads = run_oracle_rows(case, p, rows)
    idx = torch.tensor(list(rows))
    tol = tol_for(case)
    for name, g, r in zip(("y", "S_T", "Z_T", "buffer_out"), got_out, ref_out):
        if r is None:
            assert g is None, name
            continue
        compare(f"{case.name}.{name}", g[idx], r, tol)
    for name, r in ref_grads.items():
        compare(f"{case.name}.d{name}", got_grads[name][idx], r, tol)
    n_out = sum(r is not None for r in ref_out)
    _say(f"  {case.name}: {n_out} outputs and {len(ref_grads)} gradients match on rows {rows}")
