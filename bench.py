"""Headline benchmark: OmegaNet-RNN memory-layer recurrence, forward + backward, on one MI355X.

Workload (the metric's shape): B=4, H=8 (BH=32), T=4096, d_k=d_v=64,
Omega window e=4 with per-lag softmax gates, momentum, bf16 inputs, fp32 state, chunk 64,
S0 = S_ref = Z0 = 0; dy ~ N(0,1) (loss = sum y * g). Inputs are synthetic, seeded, and resident in
HBM before the timed region. One step = one forward + one backward of the recurrence over the
whole batch (libatlas_mem.so through its C ABI, preallocated buffers).

Prints ONE JSON line (rank 0). `value` and `ms_per_step` come from K plain steps. `roofline`
covers the kernel with the largest share of the step: the same K steps are run again with the
library's HIP events recorded around every launch on the launch stream (the records between
launches lengthen that pass, reported as `profiled_ms_per_step`, so it gives kernel durations only);
`mfma` is the step's matrix-product work against the bf16 peak; `cpu_baseline` times the CPU oracle
(the fp32 torch restatement of the reference op sequence, forward + backward through autograd) on a
bounded sample of the same workload.

`--config c2|c5` runs the other HBM-bound BASELINE configs the same way; `--config c4` the tensor
feature map configuration (MFMA-bound; autograd path); `--config decode` the one-token step.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
B, H, T, D, E = 4, 8, 4096, 64, 4
BH = B * H
TOKENS = B * T               # (b, t) positions through one memory layer, all heads

# The configurations run through the preplanned native path (RecurrencePlan: the C ABI with every
# buffer allocated up front). C3 is the headline (the default run); c2 / c5 are the other HBM-bound
# BASELINE configs. Tokens are (b, t) positions through one memory layer.
PLAN_CONFIGS = {
    "c3": dict(B=4, H=8, T=4096, d=64, e=4, gate="lag", seed=1003, cpu_sample_t=1024,
               workload="C3 OmegaNet-RNN memory layer: B=4 H=8 T=4096 d=64 e=4 lag gates, momentum, "
                        "bf16 inputs, fp32 state, chunk 64"),
    "c2": dict(B=4, H=8, T=2048, d=64, e=1, gate=None, seed=1002, cpu_sample_t=1024,
               workload="C2 Titans-RNN memory layer: B=4 H=8 T=2048 d=64, momentum, bf16 inputs, fp32 state, "
                        "chunk 64"),
    "c5": dict(B=8, H=8, T=2048, d=64, e=4, gate="token", seed=1005, cpu_sample_t=512,
               workload="C5 memory core of one RNN-transformer layer: B=8 H=8 T=2048 d=64 e=4 per-token gates, "
                        "momentum, bf16 inputs, fp32 state"),
}


def n_scalars(e, gate):
    """Per-token-head scalars: eta, alpha, beta, plus e lag gates or one token gate."""
    return 3 + (e if gate == "lag" else 1 if gate == "token" else 0)


def algorithmic_bytes(bh=BH, t=T, d=D, e=E, n_sc=None, s_in=2, s_st=4):
    """Compulsory HBM bytes (each input read once, each output written once) per kernel and per
    step. n_sc: scalars per token-head (default: eta, alpha, beta and e lag gates)."""
    n = bh * t
    n_sc = 3 + e if n_sc is None else n_sc
    st = bh * d * d * s_st
    buf = 2 * bh * (e - 1) * d * d * s_st
    fwd = n * 3 * d * s_in + n * n_sc * s_in + n * d * s_in + 5 * st + buf
    bwd = n * 4 * d * s_in + 2 * n * n_sc * s_in + n * 3 * d * s_in + 8 * st + buf
    per_kernel = {
        # segment aggregates (zero state): read k, v, scalars, S_ref
        "k_fwd_seg_agg": n * 2 * d * s_in + n * n_sc * s_in + st,
        # forward walk: read k, q, v, scalars, S_ref/S0/Z0; write y, S_T, Z_T
        "k_fwd_seg": n * 3 * d * s_in + n * n_sc * s_in + n * d * s_in + 5 * st,
        "k_buffer_out": bh * (e - 1) * (2 * d * s_in + d * d * s_st),
        # adjoint aggregates: read q, dy, alpha/eta/beta
        "k_bwd_seg_agg": n * 2 * d * s_in + n * 3 * s_in,
        # backward walk: read k, q, v, dy, S_ref, dS_T, dZ_T; write dk, dq, dv, dS0, dZ0
        "k_bwd_seg": n * 4 * d * s_in + n * 3 * d * s_in + 5 * st,
        # scalar gradients: read the per-token scalars, write their gradients
        "k_bwd_scalar": 2 * n * n_sc * s_in,
        "k_bwd_seg_fixup": 0,
        "k_seg_reduce_dsref": st,
        # segment scans and chunk-coefficient passes: intermediate data only; the coefficient
        # passes read the per-token scalars once
        "k_fwd_seg_scan": 0,
        "k_bwd_seg_scan": 0,
        # forward and backward chunk records in one launch (reads the per-token scalars once)
        "k_chunk_coef_pair": n * n_sc * s_in,
        # forward chunk records only, on the matrix cores (plans whose backward forms its own)
        "k_chunk_coef_fwd": n * n_sc * s_in,
    }
    # launches that carry a second, independent stage as extra workgroups
    per_kernel["k_fwd_seg_scan+buffer_out"] = per_kernel["k_fwd_seg_scan"] + per_kernel["k_buffer_out"]
    per_kernel["k_scalar_chain+fixup"] = per_kernel["k_bwd_scalar"] + per_kernel["k_bwd_seg_fixup"] + st
    # the specialised bf16 d = 64 path launches these kernels for the same stages
    for spec, gen in (("k_walk_agg", "k_fwd_seg_agg"), ("k_walk_full", "k_fwd_seg"), ("k_walk_bwd", "k_bwd_seg"),
                      ("k_scalar_chain", "k_bwd_scalar")):
        per_kernel[spec] = per_kernel[gen]
    # the backward walk with in-kernel coefficients (chunk_bwd.hip): the walk's reads and writes plus
    # the per-token scalars read and their gradients written; its fixup writes dS_ref once
    per_kernel["k_cp_bwd"] = per_kernel["k_bwd_seg"] + per_kernel["k_bwd_scalar"]
    per_kernel["k_cp_fixup"] = st
    return fwd, bwd, per_kernel


def flops_per_step(bh, t, d=D, momentum=True, bwd_factor=2.0, chunk=64):
    """Matrix-core work of one step (the chunked form's products, per token-head): delta = S_ref phi
    (2 d^2), the intra-chunk psi phi^T and its product with delta (2 * 2 C d), the chunk-start
    state's contribution psi S (and psi Z) (2 d^2 each) and the end-state update delta^T W phi per
    chunk (2 d^2 per token for S, and for Z); the backward does about twice the forward's. At d = 64,
    C = 64 with momentum: 57,344 flop per token-head forward."""
    ns = 2 if momentum else 1
    fwd = 2 * d * d + 2 * 2 * chunk * d + ns * 2 * d * d + ns * 2 * d * d
    return bh * t * fwd * (1.0 + bwd_factor)


def cpu_threads():
    """Host threads for the CPU baseline: every core of this process's affinity mask, limited to
    the box's CPU share where the environment states one (OMP_NUM_THREADS)."""
    aff = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    n = min(aff, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else aff
    return max(1, n), aff


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def make_inputs(device, cfg=None):
    """Seeded synthetic inputs of a PLAN_CONFIGS entry (default C3) on `device` (bf16 operands, fp32
    zero states) and their fp32 CPU originals."""
    import torch
    cfg = PLAN_CONFIGS["c3"] if cfg is None else cfg
    bh, t, d, e = cfg["B"] * cfg["H"], cfg["T"], cfg["d"], cfg["e"]
    g = torch.Generator().manual_seed(cfg["seed"])       # seed = 1000 + config number
    r = lambda *s: torch.randn(*s, generator=g)
    k = r(bh, t, d)
    k = k / k.norm(dim=-1, keepdim=True)
    x = dict(k=k, q=r(bh, t, d), v=r(bh, t, d),
             lr=0.1 * torch.sigmoid(r(bh, t)), decay=torch.sigmoid(r(bh, t) * 0.5 + 2.0),
             beta=torch.sigmoid(r(bh, t) * 0.5 + 1.0))
    if cfg["gate"] == "lag":
        x["gate"] = torch.softmax(r(bh, t, e), dim=-1)
    elif cfg["gate"] == "token":
        x["gate"] = torch.sigmoid(r(bh, t))
    x["dy"] = r(bh, t, d)
    out = {kk: v.to(device=device, dtype=torch.bfloat16).contiguous() for kk, v in x.items()}
    out.setdefault("gate", None)
    x.setdefault("gate", None)
    zeros = torch.zeros(bh, d, d, device=device, dtype=torch.float32)
    out.update(S_ref=zeros, S0=zeros, Z0=zeros)
    return out, x


def cpu_baseline(x_cpu, cfg=None, sample_t=256, reps=3, proj=None, map_degree=1):
    """The CPU oracle (fp32 torch restatement of the reference op sequence, forward + backward
    through autograd) on the first `sample_t` tokens of every (b, h) row: 1 warmup, median of
    `reps`. The oracle's work per token does not grow with T (its scans are linear-work), so the
    sample's tokens/s stands for the full sequence. With `proj`, k and q first go through the tensor
    feature map (and the elementwise map of `map_degree`). Returns (tokens/s, threads, affinity
    cores, median seconds)."""
    import torch
    from oracle import memory_recurrence_vectorised, poly_feature_map
    cfg = PLAN_CONFIGS["c3"] if cfg is None else cfg
    threads, aff = cpu_threads()
    torch.set_num_threads(threads)
    bh, e = cfg["B"] * cfg["H"], cfg["e"]
    sl = slice(0, sample_t)
    f32 = torch.float32
    names = ("k", "q", "v", "lr", "decay", "beta") + (("gate",) if x_cpu.get("gate") is not None else ())
    leaves = {kk: x_cpu[kk][:, sl].to(torch.bfloat16).to(f32).clone().requires_grad_(True) for kk in names}
    dy = x_cpu["dy"][:, sl].to(torch.bfloat16).to(f32)
    dk = proj.shape[1] if proj is not None else leaves["k"].shape[-1]
    dv = leaves["v"].shape[-1]
    S0 = torch.zeros(bh, dv, dk, requires_grad=True)
    Z0 = torch.zeros(bh, dv, dk, requires_grad=True)
    P = proj.to(f32) if proj is not None else None

    def feat(x):
        if P is None:
            return x
        return poly_feature_map(poly_feature_map(x, 2, 'tensor', P), map_degree, 'elementwise')

    times = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        y, S_T, Z_T, buf = memory_recurrence_vectorised(
            feat(leaves["k"]), feat(leaves["q"]), leaves["v"], leaves["lr"], leaves["decay"], leaves["beta"],
            leaves.get("gate"), S0, S0, Z0, None, window=e)
        (y * dy).sum().backward()
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        for t in list(leaves.values()) + [S0, Z0]:
            t.grad = None
    med = statistics.median(times)
    return cfg["B"] * sample_t / med, threads, aff, med


def cpu_baseline_record(x_cpu, cfg, sample_t, **kw):
    tps, threads, aff, med = cpu_baseline(x_cpu, cfg, sample_t=sample_t, **kw)
    bh = cfg["B"] * cfg["H"]
    return {"value": round(tps, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle fp32 fwd+bwd (autograd) on tokens 0..{sample_t - 1} of all {bh} (b,h) rows, "
                       f"median of 3 = {med:.2f} s; linear-work scans, so the rate stands for T = {cfg['T']}"),
            "cpu_model": cpu_model(), "affinity_cores": aff,
            "threads_note": "threads = affinity cores, capped at the box's CPU share (OMP_NUM_THREADS)"}


def traffic_file(name):
    return os.path.join(ROOT, "profiles", f"hbm_traffic_{name}.md")


def measured_traffic(kernel, name="c3"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary of config
    `name` (lines `traffic: <kernel> <bytes>`, FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel
    factor), or None when there is no summary or no figure for it."""
    try:
        with open(traffic_file(name)) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic:" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        return None
    return None


def calibrate_copy(nbytes=256 << 20, reps=5):
    """A plain device-to-device copy of known size, for scaling the HBM counters
    (FETCH_SIZE / WRITE_SIZE of this launch against nbytes read and nbytes written)."""
    import torch
    src = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "launches": reps}), flush=True)


# C4 (`--config c4`): OmegaNet-RNN with the tensor feature map phi = elementwise_g3([k; vec(k k^T)] P),
# P: 4160 -> 128 (Xavier-uniform), d_k = 128, d_v = 64, e = 8, lag gates. The map is a GEMM with
# K = 4160 (MFMA-bound); the step runs through the autograd API (the map's fused kernels, then the
# recurrence on 64 x 64 state blocks).
C4 = dict(B=2, H=8, T=8192, dk=128, dv=64, e=8, gate="lag", seed=1004, d_in=64, degree=3,
          workload="C4 OmegaNet-RNN memory layer with the tensor feature map (64+4096 -> 128, then the "
                   "elementwise map of degree 3): B=2 H=8 T=8192 d_k=128 d_v=64 e=8 lag gates, momentum, "
                   "bf16 inputs, fp32 state")


def run_c4(steps, warmup, cpu=True, cpu_sample_t=128):
    """C4 fwd+bwd through the autograd API (torch.autograd.grad of y against a fixed random output
    gradient, i.e. the gradient of sum(y * g)). The roofline is the matrix-core one of the dominant
    kernel, the fused tensor map's backward or forward, timed with HIP events on the stream it is
    launched on (direct C-ABI calls on preallocated buffers, the same launches the step makes)."""
    import ctypes
    import torch
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import memory_recurrence, tensor_feature_map, symmetrized_tables, _ptr, _stream
    c = C4
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bh, t, dk, dv, e, kin, deg = c["B"] * c["H"], c["T"], c["dk"], c["dv"], c["e"], c["d_in"], c["degree"]
    g = torch.Generator().manual_seed(c["seed"])
    r = lambda *sh: torch.randn(*sh, generator=g)
    bf = lambda x: x.to(device=dev, dtype=torch.bfloat16).contiguous()
    k = r(bh, t, kin)
    k = k / k.norm(dim=-1, keepdim=True)
    q = r(bh, t, kin)
    q = q / q.norm(dim=-1, keepdim=True)
    x_cpu = dict(k=k, q=q, v=r(bh, t, dv), lr=0.1 * torch.sigmoid(r(bh, t)),
                 decay=torch.sigmoid(r(bh, t) * 0.5 + 2.0), beta=torch.sigmoid(r(bh, t) * 0.5 + 1.0),
                 gate=torch.softmax(r(bh, t, e), dim=-1))
    leaves = {kk: bf(v).requires_grad_(True) for kk, v in x_cpu.items()}
    bound = (6.0 / (kin + kin * kin + dk)) ** 0.5
    P_cpu = (torch.rand(kin + kin * kin, dk, generator=g) * 2 - 1) * bound
    P = bf(P_cpu)
    dy_cpu = r(bh, t, dv)
    x_cpu["dy"] = dy_cpu
    gy = bf(dy_cpu)
    zeros = torch.zeros(bh, dv, dk, device=dev)

    # P is a constant projection: its symmetrised tables are formed once and kept, as
    # PolynomialFeatureMap keeps them for its buffer (one launch per dtype and device)
    tables = symmetrized_tables(P, kin, torch.bfloat16)

    def feat(x):   # fused tensor-map kernels, elementwise map of degree 3 in their epilogue
        return tensor_feature_map(x, P, degree=deg, tables=tables)

    def step():
        y, S_T, Z_T, B_out = memory_recurrence(
            feat(leaves["k"]), feat(leaves["q"]), leaves["v"], leaves["lr"], leaves["decay"], leaves["beta"],
            leaves["gate"], zeros, zeros, zeros, None, window=e)
        torch.autograd.grad(y, list(leaves.values()), grad_outputs=gy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0

    # the map's kernels alone, on preallocated buffers: n = BH * T tokens per call (k or q)
    lib = _lib.load()
    n = bh * t
    xk = leaves["k"].detach().reshape(n, kin).contiguous()
    stream = _stream(dev)
    ps = torch.empty_like(P)                          # the symmetrised table the step uses
    pst = torch.empty(dk, P.shape[0], device=dev, dtype=P.dtype)
    _lib.check(lib.atlas_tensor_map_symmetrize(_lib.DT_BF16, kin, dk, _ptr(P), _ptr(ps), _ptr(pst), stream),
               "atlas_tensor_map_symmetrize")
    out = torch.empty(n, dk, device=dev, dtype=torch.bfloat16)
    pre = torch.empty_like(out)
    dout = bf(r(n, dk))
    dx = torch.empty_like(xk)
    fwd_call = lambda: _lib.check(lib.atlas_tensor_map_fwd_sym(_lib.DT_BF16, n, kin, dk, deg, _ptr(xk), _ptr(pst),
                                                               _ptr(out), _ptr(pre), stream), "atlas_tensor_map_fwd_sym")
    bwd_call = lambda: _lib.check(lib.atlas_tensor_map_bwd_sym(_lib.DT_BF16, n, kin, dk, deg, _ptr(xk), _ptr(ps),
                                                               _ptr(pre), _ptr(dout), _ptr(dx), stream),
                                  "atlas_tensor_map_bwd_sym")
    kern = {}
    for name, call in (("k_tmap_fwd", fwd_call), ("k_tmap_bwd", bwd_call)):
        for _ in range(3):
            call()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(torch.cuda.current_stream(dev))
        for _ in range(steps):
            call()
        ev1.record(torch.cuda.current_stream(dev))
        torch.cuda.synchronize()
        kern[name] = 1e3 * ev0.elapsed_time(ev1) / steps   # microseconds per launch
    map_flops = 2.0 * (kin + kin * kin) * dk * n          # one call: [n, 4160] x [4160, 128]
    # per step: 2 forward and 2 backward map calls + the recurrence on 2 state blocks (d = 64)
    step_flops = 4 * map_flops + 2 * flops_per_step(bh, t, 64)
    dom = max(kern, key=kern.get)
    ach = map_flops / (kern[dom] * 1e-6) / 1e12
    tokens = c["B"] * t
    ms = 1e3 * el / steps
    line = {"metric": "memory-layer tokens/s fwd+bwd", "value": round(tokens * steps / el, 1), "unit": "tokens/s",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded)",
            "config": {"workload": c["workload"], "global_batch": c["B"], "seq_len": t, "heads": c["H"], "d_k": dk,
                       "d_v": dv, "window": e, "parallelism": "single GPU"},
            "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": None,
                         "algorithmic_flops_per_launch": map_flops, "avg_launch_us": round(kern[dom], 2)},
            "kernels": {kk: {"avg_us": round(v, 2)} for kk, v in kern.items()},
            "mfma": {"flops_per_step": step_flops, "achieved_tflops": round(step_flops / (ms * 1e-3) / 1e12, 1),
                     "peak_tflops": BF16_PEAK_TFLOPS,
                     "frac": round(step_flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}}
    if cpu:
        line["cpu_baseline"] = cpu_baseline_record(x_cpu, dict(B=c["B"], H=c["H"], T=t, e=e), cpu_sample_t,
                                                   proj=P_cpu.to(torch.bfloat16).float(), map_degree=deg)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def run_affine(steps, warmup, n=32, t=1024, d=64, r=64, cpu=True):
    """The right-affine scan (affine_scan.py:36-158) at D = R = 64, T = 1024, N = 32, forward + backward
    on the chunked fp32 matrix-core kernels, each pass timed with HIP events on its stream. HBM
    roofline: A and B read once, H written once (forward); A, H, dout read once, dA, dB written once
    (backward). `mfma` counts the sequential scan's products (2 N T R D^2 per pass, twice that for dA
    and the adjoint) against the fp32 matrix peak."""
    import ctypes
    import torch
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import _ptr, _stream
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(1007)
    A_cpu = 0.95 * torch.eye(d) + 0.3 * torch.randn(n, t, d, d, generator=g) / d ** 0.5
    B_cpu = torch.randn(n, t, r, d, generator=g)
    A, B = A_cpu.to(dev), B_cpu.to(dev)
    prev = torch.randn(n, r, d, generator=g).to(dev)
    H = torch.empty_like(B)
    dout = torch.randn(n, t, r, d, generator=g).to(dev)
    dA, dB, dprev = torch.empty_like(A), torch.empty_like(B), torch.empty_like(prev)
    lib = _lib.load()
    nb = lib.atlas_affine_scan_workspace_bytes(n, t, r, d)
    ws = torch.empty((nb + 3) // 4, device=dev)
    st = _stream(dev)
    fwd = lambda: _lib.check(lib.atlas_affine_scan_fwd(n, t, r, d, _ptr(A), _ptr(B), _ptr(prev), _ptr(H), _ptr(ws),
                                                       nb, st), "atlas_affine_scan_fwd")
    bwd = lambda: _lib.check(lib.atlas_affine_scan_bwd(n, t, r, d, _ptr(A), _ptr(H), _ptr(prev), _ptr(dout), _ptr(dA),
                                                       _ptr(dB), _ptr(dprev), _ptr(ws), nb, st), "atlas_affine_scan_bwd")
    us = {}
    for name, call in (("fwd", fwd), ("bwd", bwd)):
        for _ in range(warmup):
            call()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(torch.cuda.current_stream(dev))
        for _ in range(steps):
            call()
        ev1.record(torch.cuda.current_stream(dev))
        torch.cuda.synchronize()
        us[name] = 1e3 * ev0.elapsed_time(ev1) / steps
    a_b, bh_b = n * t * d * d * 4, n * t * r * d * 4
    alg = {"fwd": a_b + 2 * bh_b, "bwd": 2 * a_b + 3 * bh_b}
    flops = 2.0 * n * t * r * d * d * 3          # forward scan, adjoint scan, dA
    step_us = us["fwd"] + us["bwd"]
    dom = max(us, key=us.get)
    ach = alg[dom] / (us[dom] * 1e-6) / 1e9
    line = {"metric": "affine-scan steps/s fwd+bwd (H_t = H_{t-1} A_t + B_t)", "value": round(n * t / (step_us * 1e-6), 1),
            "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(step_us / 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded)",
            "config": {"workload": f"affine_associative_scan N={n} T={t} R={r} D={d}, fp32, with prev",
                       "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "kernel": f"affine scan {dom} pass", "achieved": round(ach, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes_per_launch": alg[dom], "avg_launch_us": round(us[dom], 2)},
            "passes_us": {kk: round(v, 2) for kk, v in us.items()},
            "mfma": {"flops_per_step": flops, "achieved_tflops": round(flops / (step_us * 1e-6) / 1e12, 2),
                     "peak_tflops": 157.3, "frac": round(flops / (step_us * 1e-6) / 1e12 / 157.3, 4)}}
    if cpu:
        from oracle import affine_scan_sequential
        threads, aff = cpu_threads()
        torch.set_num_threads(threads)
        ts = 64
        Ac = A_cpu[:, :ts].clone().requires_grad_()
        Bc = B_cpu[:, :ts].clone().requires_grad_()
        pc = prev.cpu().clone().requires_grad_()
        times = []
        for i in range(4):
            t0 = time.perf_counter()
            out = affine_scan_sequential(Ac, Bc, pc, remove_prev=True)
            (out * dout[:, :ts].cpu()).sum().backward()
            if i:
                times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        line["cpu_baseline"] = {"value": round(n * ts / med, 1), "unit": "steps/s", "cores": threads, "kind": "port",
                                "sample": f"oracle sequential matmul loop fwd+bwd (autograd, fp32) on steps 0..{ts - 1} "
                                          f"of all {n} scans, median of 3 = {med:.2f} s; linear in T",
                                "cpu_model": cpu_model(), "affinity_cores": aff}
    print(json.dumps(line), flush=True)


def run_prologue(steps, warmup, B=8, T=2048, dim=512, heads=8, d=64, conv_k=4, n_gates=4):
    """The cell prologue at C5's layer shape (B=8 T=2048 dim=512, 8 heads of 64, conv 4, four gate
    heads), bf16: forward + backward of functional.cell_prologue (fused kernels + the projection
    GEMMs), timed with HIP events on the stream; the same composition of unfused torch ops (the
    reference's sequence) timed beside it. HBM roofline of the fused kernels alone: the prologue
    kernel reads x and writes xn, q_in, k_in, v_in; the heads kernel reads ql, kl, vl and the gate
    logits and writes q, k, v and the gates (forward), the backward moves twice as much."""
    import torch
    from atlas_rnn_amd.functional import cell_prologue
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(1008)
    bf = lambda t: t.to(dev, torch.bfloat16).requires_grad_()
    r = lambda *sh: torch.randn(*sh, generator=g)
    x = bf(r(B, T, dim))
    p = dict(nw=bf(1 + 0.1 * r(dim)), wq=bf(0.5 * r(dim, 1, conv_k)), wk=bf(0.5 * r(dim, 1, conv_k)),
             wv=bf(0.5 * r(dim, 1, conv_k)), Wq=bf(r(heads * d, dim) / dim ** 0.5), Wk=bf(r(heads * d, dim) / dim ** 0.5),
             Wv=bf(r(heads * d, dim) / dim ** 0.5), qg=bf(torch.ones(heads, 1, d)), kg=bf(torch.ones(heads, 1, d)))
    G = [bf(0.1 * r(heads, dim) / dim ** 0.5) for _ in range(n_gates)]
    bias = [bf(r(heads)) for _ in range(n_gates)]
    eps = torch.finfo(torch.bfloat16).eps
    F = torch.nn.functional

    def fused():
        xn, q, k, v, gates = cell_prologue(x, p["nw"], eps, (p["wq"], p["wk"], p["wv"]), (p["Wq"], p["Wk"], p["Wv"]),
                                           G, bias, p["qg"], p["kg"], heads, d)
        return [q, k, v, *gates]

    def unfused():   # rnn_memory.py:567-653 as torch ops
        xn = F.rms_norm(x, (dim,), p["nw"], eps)
        outs = []
        for w, W, gam in (("wq", "Wq", "qg"), ("wk", "Wk", "kg"), ("wv", "Wv", None)):
            xi = F.conv1d(xn.transpose(1, 2), p[w], padding=conv_k // 2, groups=dim).transpose(1, 2)
            y = F.linear(xi, p[W]).reshape(B, T + 1, heads, d).permute(0, 2, 1, 3)[:, :, :T]
            if gam:
                y = y / (y.norm(dim=-1, keepdim=True) * d ** -0.5).clamp(min=1e-8) * p[gam]
            outs.append(y.reshape(B * heads, T, d))
        outs += [torch.sigmoid(F.linear(xn, G[i], bias[i])).permute(0, 2, 1).reshape(B * heads, T)
                 for i in range(n_gates)]
        return outs

    leaves = [x, *p.values(), *G, *bias]
    grads_out = None
    us = {}
    for name, fn in (("fused", fused), ("torch", unfused)):
        def step():
            outs = fn()
            torch.autograd.grad(outs, leaves, grad_outputs=[torch.ones_like(o) for o in outs])
        for _ in range(warmup):
            step()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
        us[name] = 1e3 * ev0.elapsed_time(ev1) / steps
    # the two forward kernels alone, on preallocated buffers (direct C-ABI calls)
    import ctypes
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import _ptr, _stream
    lib = _lib.load()
    st = _stream(dev)
    xd = x.detach()
    taps = [p[w].detach().reshape(dim, conv_k).contiguous() for w in ("wq", "wk", "wv")]
    xn_, qi_, ki_, vi_ = (torch.empty_like(xd) for _ in range(4))
    inv_ = torch.empty(B, T, device=dev)
    ql_ = torch.empty(B, T, heads * d, device=dev, dtype=torch.bfloat16)
    zl_ = torch.empty(B, T, n_gates * heads, device=dev, dtype=torch.bfloat16)
    q_, k_, v_ = (torch.empty(B * heads, T, d, device=dev, dtype=torch.bfloat16) for _ in range(3))
    gt_ = torch.empty(n_gates, B * heads, T, device=dev, dtype=torch.bfloat16)
    bcat = torch.cat([b.detach() for b in bias])
    calls = {
        "k_pro_fwd": lambda: _lib.check(lib.atlas_prologue_fwd(
            _lib.DT_BF16, B, T, dim, conv_k, eps, _ptr(xd), _ptr(p["nw"].detach()), _ptr(taps[0]), _ptr(taps[1]),
            _ptr(taps[2]), _ptr(xn_), _ptr(qi_), _ptr(ki_), _ptr(vi_), _ptr(inv_), st), "atlas_prologue_fwd"),
        "k_heads_fwd": lambda: _lib.check(lib.atlas_heads_fwd(
            _lib.DT_BF16, B, T, heads, d, n_gates, _ptr(ql_), _ptr(ql_), _ptr(ql_), _ptr(zl_),
            _ptr(p["qg"].detach()), _ptr(p["kg"].detach()), _ptr(bcat), _ptr(q_), _ptr(k_), _ptr(v_), _ptr(gt_), st),
            "atlas_heads_fwd")}
    kus = {}
    for name, call in calls.items():
        for _ in range(3):
            call()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            call()
        ev1.record()
        torch.cuda.synchronize()
        kus[name] = 1e3 * ev0.elapsed_time(ev1) / steps
    n_tok = B * T
    e = 2
    kbytes = {"k_pro_fwd": n_tok * dim * e * 5 + n_tok * 4,
              "k_heads_fwd": n_tok * heads * d * e * 6 + n_tok * heads * n_gates * e * 2}
    kern_bytes_fwd = sum(kbytes.values())
    line = {"metric": "cell-prologue tokens/s fwd+bwd (norms, convs, projections, head split, gates)",
            "value": round(n_tok / (us["fused"] * 1e-6), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(us["fused"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded)",
            "config": {"workload": f"memory-cell prologue at C5's layer shape: B={B} T={T} dim={dim} heads={heads} d={d} "
                                   f"conv {conv_k} gate heads {n_gates}, bf16", "parallelism": "single GPU"},
            "torch_unfused_ms_per_step": round(us["torch"] / 1e3, 4),
            "speedup_vs_torch": round(us["torch"] / us["fused"], 2),
            "kernels": {kk: {"avg_us": round(v, 2), "gbs": round(kbytes[kk] / (v * 1e-6) / 1e9, 1)} for kk, v in kus.items()}}
    dom = max(kus, key=kus.get)
    ach = kbytes[dom] / (kus[dom] * 1e-6) / 1e9
    line["roofline"] = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                        "algorithmic_bytes_per_launch": kbytes[dom], "avg_launch_us": round(kus[dom], 2)}
    print(json.dumps(line), flush=True)


def run_module(steps, warmup, B=4, T=4096, heads=8, d=64, e=4, chunk=64):
    """The drop-in cell at the C3 shape: OmegaRNNMemoryCell(dim=512, 8 heads of 64, omega_window=4,
    per-token omega gate, momentum, scan_chunk_len=64) in bf16, forward + backward of every parameter
    (loss = sum out * g), called with a fresh state (state=None: a new sequence) and with a carried
    state (the previous call's S, Z and omega buffer). The library's recurrence kernels inside the
    cell step are timed with its HIP events and set against the same recurrence through the
    preplanned path (RecurrencePlan, token gates, clamp_every=64). The same step captured in a HIP
    graph (torch.cuda.CUDAGraph) is timed too: `value` stays the eager call a drop-in user makes."""
    import torch
    import atlas_rnn_amd as am
    from atlas_rnn_amd.functional import RecurrencePlan, profile_enable, profile_read
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    torch.manual_seed(1009)
    dim = heads * d
    cell = am.OmegaRNNMemoryCell(dim=dim, dim_head=d, heads=heads, omega_window=e, use_omega_gate=True,
                                 use_momentum=True, scan_chunk_len=chunk).to(dev, torch.bfloat16)
    with torch.no_grad():   # non-trivial gate heads (zero-initialised weights give constant gates)
        for pp in cell.parameters():
            if pp.ndim == 2 and pp.shape[0] == heads:
                pp.normal_(0, 0.02)
    g = torch.Generator().manual_seed(1010)
    x = torch.randn(B, T, dim, generator=g).to(dev, torch.bfloat16)
    gy = torch.randn(B, T, dim, generator=g).to(dev, torch.bfloat16)
    params = list(cell.parameters())
    with torch.no_grad():
        _, st0 = cell(x)
    st0 = am.state_detach(st0)

    def step(state):
        out, _ = cell(x, state)
        torch.autograd.grad(out, params, grad_outputs=gy)

    res = {}
    for name, state in (("fresh_state", None), ("carried_state", st0)):
        for _ in range(warmup):
            step(state)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(state)
        torch.cuda.synchronize()
        ms = 1e3 * (time.perf_counter() - t0) / steps
        profile_enable(True)
        profile_read(reset=True)
        for _ in range(steps):
            step(state)
        torch.cuda.synchronize()
        prof = profile_read(reset=True)
        profile_enable(False)
        rec_ms = sum(v for v, n in prof.values()) / steps
        # the same step captured in a HIP graph and replayed (no Python, autograd or launch cost)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step(state)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(state)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        graph_ms = 1e3 * (time.perf_counter() - t0) / steps
        del graph
        res[name] = {"ms_per_step": round(ms, 4), "graph_replay_ms_per_step": round(graph_ms, 4),
                     "recurrence_kernels_ms": round(rec_ms, 4),
                     "kernels": {kk: round(1e3 * v / steps, 2) for kk, (v, n) in prof.items() if n}}
    # the same recurrence through the preplanned path
    bh = B * heads
    xin, _ = make_inputs(dev, dict(B=B, H=heads, T=T, d=d, e=e, gate="token", seed=1003))
    plan = RecurrencePlan(bh, T, d, window=e, momentum=True, gate_mode='token', dtype=torch.bfloat16, device=dev,
                          clamp_every=chunk)

    def pstep():
        plan.forward(xin["k"], xin["q"], xin["v"], xin["lr"], xin["decay"], xin["beta"], xin["gate"], xin["S_ref"],
                     xin["S0"], None)
        plan.backward(xin["dy"])

    for _ in range(warmup):
        pstep()
    profile_enable(True)
    profile_read(reset=True)
    for _ in range(steps):
        pstep()
    torch.cuda.synchronize()
    prof = profile_read(reset=True)
    profile_enable(False)
    plan_ms = sum(v for v, n in prof.values()) / steps
    ms = res["fresh_state"]["ms_per_step"]
    line = {"metric": "memory-cell tokens/s fwd+bwd (prologue, recurrence, output projection, every parameter gradient)",
            "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded), random-init cell",
            "config": {"workload": f"OmegaRNNMemoryCell(dim={dim}, dim_head={d}, heads={heads}, omega_window={e}, "
                                   f"use_omega_gate=True, use_momentum=True, scan_chunk_len={chunk}), x [{B}, {T}, {dim}]",
                       "parallelism": "single GPU"},
            "module": res, "plan_recurrence_kernels_ms": round(plan_ms, 4),
            "module_vs_plan_recurrence": round(res["fresh_state"]["recurrence_kernels_ms"] / plan_ms, 3)}
    print(json.dumps(line), flush=True)


def run_decode(steps, warmup, factored=False):
    """Generation steps at the C3 head shape (B=4 H=8 d=64 e=4 lag gates, momentum, bf16 inputs,
    fp32 state): atlas_mem_step through the C ABI with the state updated in place, the way a decode
    loop carries it. One step = one token for every sequence of the batch; `value` counts those
    (b) tokens per second, timed on a HIP graph of the steps (the eager per-call rate, host-bound,
    is reported beside it). The kernel is timed with events on the stream it runs on; its
    algorithmic bytes are the state read and written once (S_ref, S0, Z0, buffer in; S_T, Z_T,
    buffer out) plus the token's vectors. factored: the buffer carried as rank-1 factors
    [bh, e-1, 2d] (atlas_mem_step_factored, two factor buffers used in turn)."""
    import ctypes
    import torch
    from atlas_rnn_amd import _lib
    from atlas_rnn_amd.functional import RecurrenceConfig, _problem, _ptr, _stream
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, d, e = 4, 8, 64, 4
    bh = B * H
    g = torch.Generator().manual_seed(1006)
    r = lambda *sh: torch.randn(*sh, generator=g)
    bf = lambda x: x.to(device=dev, dtype=torch.bfloat16).contiguous()
    k = r(bh, 1, d)
    x = dict(k=bf(k / k.norm(dim=-1, keepdim=True)), q=bf(r(bh, 1, d)), v=bf(r(bh, 1, d)),
             lr=bf(0.1 * torch.sigmoid(r(bh, 1))), decay=bf(torch.sigmoid(r(bh, 1) * 0.5 + 2.0)),
             beta=bf(torch.sigmoid(r(bh, 1) * 0.5 + 1.0)), gate=bf(torch.softmax(r(bh, 1, e), dim=-1)))
    S_ref = (0.1 * r(bh, d, d)).to(dev)
    S, Z, Bf = S_ref.clone(), (0.1 * r(bh, d, d)).to(dev), (0.1 * r(bh, e - 1, d, d)).to(dev)
    y = torch.empty(bh, 1, d, device=dev, dtype=torch.bfloat16)
    lib = _lib.load()
    prob = _problem(RecurrenceConfig(window=e), bh, 1, d, d, True, x["gate"], True, torch.bfloat16)
    a = _lib.FwdArgs(k=_ptr(x["k"]), q=_ptr(x["q"]), v=_ptr(x["v"]), lr=_ptr(x["lr"]), decay=_ptr(x["decay"]),
                     beta=_ptr(x["beta"]), gate=_ptr(x["gate"]), S_ref=_ptr(S_ref), S0=_ptr(S), Z0=_ptr(Z),
                     buffer_in=_ptr(Bf), y=_ptr(y), S_T=_ptr(S), Z_T=_ptr(Z), buffer_out=_ptr(Bf))
    fac = [(0.1 * r(bh, e - 1, 2 * d)).to(dev), torch.empty(bh, e - 1, 2 * d, device=dev)]
    fp = [_ptr(f) for f in fac]
    af = _lib.FwdArgs(k=_ptr(x["k"]), q=_ptr(x["q"]), v=_ptr(x["v"]), lr=_ptr(x["lr"]), decay=_ptr(x["decay"]),
                      beta=_ptr(x["beta"]), gate=_ptr(x["gate"]), S_ref=_ptr(S_ref), S0=_ptr(S), Z0=_ptr(Z),
                      y=_ptr(y), S_T=_ptr(S), Z_T=_ptr(Z))

    def step(i, st):   # token i (the factor buffers alternate with its parity)
        if factored:
            _lib.check(lib.atlas_mem_step_factored(ctypes.byref(prob), ctypes.byref(af), fp[i & 1], fp[(i & 1) ^ 1],
                                                   st), "atlas_mem_step_factored")
        else:
            _lib.check(lib.atlas_mem_step(ctypes.byref(prob), ctypes.byref(a), st), "atlas_mem_step")

    stream = _stream(dev)
    for i in range(warmup):
        step(i, stream)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        step(i, stream)
    ev1.record()
    torch.cuda.synchronize()
    eager_us = 1e3 * ev0.elapsed_time(ev1) / steps
    # the same steps replayed from a HIP graph of G launches (no host work between tokens): the
    # kernel-bound rate a captured generation loop sees; this is `value`
    G = 64
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = _stream(dev)   # the capturing stream
        for i in range(G):
            step(i, cap)
    torch.cuda.synchronize()
    reps = max(1, steps // G)
    graph.replay()
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(reps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    us = 1e3 * ev0.elapsed_time(ev1) / (reps * G)
    state_bytes = bh * d * d * 4 * (3 + 2)                  # S_ref, S0, S_T; Z0, Z_T
    state_bytes += bh * (e - 1) * 4 * (2 * 2 * d if factored else 2 * d * d)   # buffer in / out
    vec_bytes = bh * (3 * d + 3 + e) * 2 + bh * d * 2       # k, q, v, scalars, gates; y
    alg = state_bytes + vec_bytes
    out = {"metric": "decode tokens/s (one memory-layer step per token)", "value": round(B / (us * 1e-6), 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(us / 1e3, 6),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded)", "timing": f"HIP graph of {G} steps replayed {reps} times",
           "eager_us_per_step": round(eager_us, 3),
           "config": {"workload": "decode step at the C3 head shape: B=4 H=8 d=64 e=4 lag gates, momentum, "
                                  "state in place" + (", buffer as rank-1 factors" if factored else ""),
                      "global_batch": B, "seq_len": 1, "parallelism": "single GPU"},
           "roofline": {"bound": "hbm", "achieved": round(alg / (us * 1e-6) / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                        "frac": round(alg / (us * 1e-6) / 8e12, 4), "traffic": None}}
    print(json.dumps(out), flush=True)


def bench_plan(name, steps, warmup, cpu=True, cpu_sample_t=256, with_buffer=False, clamp_every=None):
    """fwd+bwd of PLAN_CONFIGS[name] through the preplanned native path: K plain steps timed
    (value, ms_per_step); the same K steps again with the library's HIP events around every launch
    on its stream (per-kernel durations for the roofline); then the CPU oracle on a sample."""
    import torch
    from atlas_rnn_amd.functional import RecurrencePlan, profile_enable, profile_read
    cfg = PLAN_CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bh, t, d, e = cfg["B"] * cfg["H"], cfg["T"], cfg["d"], cfg["e"]
    x, x_cpu = make_inputs(dev, cfg)
    buf = torch.zeros(bh, e - 1, d, d, device=dev) if (with_buffer and e > 1) else None
    plan = RecurrencePlan(bh, t, d, window=e, momentum=True, gate_mode=cfg["gate"], dtype=torch.bfloat16, device=dev,
                          has_buffer=buf is not None, clamp_every=clamp_every)

    def step():
        plan.forward(x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"], x["S_ref"], x["S0"], x["Z0"],
                     buf)
        plan.backward(x["dy"])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # timed region: K steps, nothing else on the stream
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # the same K steps again with the library's per-kernel HIP events on the launch stream; the
    # event records between launches lengthen the step, so only kernel durations come from here
    profile_enable(True)
    profile_read(reset=True)
    torch.cuda.synchronize()
    tp0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    tp1 = time.perf_counter()
    prof = profile_read(reset=True)
    profile_enable(False)

    elapsed = t1 - t0
    ms_per_step = 1e3 * elapsed / steps
    tokens = cfg["B"] * t
    value = tokens * steps / elapsed
    fwd_b, bwd_b, per_kernel = algorithmic_bytes(bh, t, d, e, n_scalars(e, cfg["gate"]))
    step_bytes = fwd_b + bwd_b
    kernels = {kk: {"avg_us": 1e3 * ms / max(n, 1), "launches": n} for kk, (ms, n) in prof.items() if n}
    dom = max(kernels, key=lambda kk: kernels[kk]["avg_us"] * kernels[kk]["launches"])
    # the stage's time per step: under scan_chunk_len clamps both flag-selected sequences are
    # launched every step and the unselected one returns at once, so launches != steps there
    dom_s = kernels[dom]["avg_us"] * kernels[dom]["launches"] / steps * 1e-6
    achieved = per_kernel[dom] / dom_s / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": measured_traffic(dom, name),
                "algorithmic_bytes_per_launch": per_kernel[dom], "avg_launch_us": round(dom_s * 1e6, 2)}
    step_gbs = step_bytes / (elapsed / steps) / 1e9
    flops = flops_per_step(bh, t, d)
    tflops = flops / (elapsed / steps) / 1e12
    out = {
        "metric": "memory-layer tokens/s fwd+bwd at H=8,d=64,T=4096; % HBM/MFMA roofline" if name == "c3"
        else "memory-layer tokens/s fwd+bwd",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v with L2-normalised keys, sigmoid gates"
                + (", softmax lag gates)" if cfg["gate"] == "lag" else ")"),
        "config": {"workload": cfg["workload"] + (", carried (zero) buffer" if buf is not None else "")
                   + (f", S clamped every {clamp_every} tokens (scan_chunk_len)" if clamp_every else ""),
                   "global_batch": cfg["B"], "seq_len": t, "heads": cfg["H"], "d": d, "window": e,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "step_roofline": {"bytes_per_step": step_bytes, "achieved_gbs": round(step_gbs, 2),
                          "frac": round(step_gbs / HBM_PEAK_GBS, 5)},
        "mfma": {"flops_per_step": flops, "achieved_tflops": round(tflops, 2), "peak_tflops": BF16_PEAK_TFLOPS,
                 "frac": round(tflops / BF16_PEAK_TFLOPS, 5),
                 "note": "the chunked form's matrix products (bf16 in, fp32 accumulate) per step"},
        "kernels": {kk: {"avg_us": round(v["avg_us"], 2), "launches": v["launches"]} for kk, v in kernels.items()},
        "profiled_ms_per_step": round(1e3 * (tp1 - tp0) / steps, 4),
    }
    if name == "c3" and clamp_every is None and buf is None:
        out["scan_chunk_len_64"] = time_clamp_variant(x, cfg, steps, warmup, 64)
    out["cpu_baseline"] = cpu_baseline_record(x_cpu, cfg, cpu_sample_t) if cpu else None
    print(json.dumps(out), flush=True)


def time_clamp_variant(x, cfg, steps, warmup, clamp_every):
    """The same fwd+bwd step as the drop-in cell runs it for scan_chunk_len = clamp_every (S clamped
    to +-100 at every clamp_every-token boundary, rnn_memory.py:584-601): the library's dual plan
    (the segment-parallel sequence with the clamp points checked on the device, the exact sequence
    launched behind it and skipped unless a clamp fires). Same inputs, K steps timed after W warmup."""
    import torch
    from atlas_rnn_amd.functional import RecurrencePlan
    dev = x["k"].device
    bh, t, d, e = cfg["B"] * cfg["H"], cfg["T"], cfg["d"], cfg["e"]
    plan = RecurrencePlan(bh, t, d, window=e, momentum=True, gate_mode=cfg["gate"], dtype=torch.bfloat16, device=dev,
                          has_buffer=False, clamp_every=clamp_every)

    def step():
        plan.forward(x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"], x["S_ref"], x["S0"], x["Z0"],
                     None)
        plan.backward(x["dy"])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    return {"clamp_every": clamp_every, "ms_per_step": round(1e3 * elapsed / steps, 4),
            "value": round(cfg["B"] * t * steps / elapsed, 1), "unit": "tokens/s",
            "note": "the same step with S clamped every 64 tokens (OmegaRNNMemoryCell(scan_chunk_len=64)); "
                    "value stays on the unclamped plan"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-tokens", type=int, default=None,
                    help="tokens per row of the CPU baseline sample (default: 1024 c2/c3, 512 c5, 128 c4)")
    ap.add_argument("--with-buffer", action="store_true",
                    help="c2/c3/c5: pass a carried (zero) omega buffer, as the drop-in cells do")
    ap.add_argument("--clamp-every", type=int, default=None,
                    help="c2/c3/c5: clamp S every N tokens (the cells' scan_chunk_len)")
    ap.add_argument("--factored", action="store_true",
                    help="--config decode: carry the buffer as rank-1 factors (atlas_mem_step_factored)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain copy kernel of known size (HBM counter calibration)")
    ap.add_argument("--config", choices=sorted(PLAN_CONFIGS) + ["c4", "decode", "affine", "prologue", "module"],
                    default="c3",
                    help="c3 (default): the headline; c2 / c4 / c5: the other BASELINE configs; decode: the "
                         "one-token step")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the memory-layer recurrence shards over (batch, head) rows "
              "with no exchange, so there is no multi-GPU figure to report (use --gpus 1).", file=sys.stderr)
        sys.exit(2)
    cpu = not args.no_cpu_baseline
    if args.config == "decode":
        run_decode(args.steps, args.warmup, factored=args.factored)
    elif args.config == "module":
        run_module(args.steps, args.warmup)
    elif args.config == "prologue":
        run_prologue(args.steps, args.warmup)
    elif args.config == "affine":
        run_affine(args.steps, args.warmup, cpu=cpu)
    elif args.config == "c4":
        run_c4(args.steps, args.warmup, cpu=cpu, cpu_sample_t=args.cpu_sample_tokens or 128)
    else:
        bench_plan(args.config, args.steps, args.warmup, cpu=cpu,
                   cpu_sample_t=args.cpu_sample_tokens or PLAN_CONFIGS[args.config]["cpu_sample_t"],
                   with_buffer=args.with_buffer, clamp_every=args.clamp_every)


if __name__ == "__main__":
    main()
