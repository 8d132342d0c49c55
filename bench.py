"""Headline benchmark: OmegaNet-RNN memory-layer recurrence, forward + backward, on one MI355X.

Workload (the metric's shape): B=4, H=8 (BH=32), T=4096, d_k=d_v=64,
Omega window e=4 with per-lag softmax gates, momentum, bf16 inputs, fp32 state, chunk 64,
S0 = S_ref = Z0 = 0, zero buffer; dy ~ N(0,1) (loss = sum y * g). Inputs are synthetic, seeded,
and resident in HBM before the timed region. One step = one forward + one backward of the
recurrence over the whole batch (libatlas_mem.so through its C ABI, preallocated buffers).

Prints ONE JSON line (rank 0). `value` and `ms_per_step` come from K plain steps. `roofline`
covers the kernel with the largest share of the step: the same K steps are run again with the
library's HIP events recorded around every launch on the launch stream (the records between
launches lengthen that pass, reported as `profiled_ms_per_step`, so it gives kernel durations only);
`cpu_baseline` times the CPU oracle (the fp32 torch restatement of the reference op sequence,
forward + backward through autograd) on a bounded sample of the same workload.
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
B, H, T, D, E = 4, 8, 4096, 64, 4
BH = B * H
TOKENS = B * T               # (b, t) positions through one memory layer, all heads


def algorithmic_bytes(bh=BH, t=T, d=D, e=E, s_in=2, s_st=4):
    """Compulsory HBM bytes (each input read once, each output written once) per kernel and per
    step. Scalars per token-head: eta, alpha, beta and e lag gates."""
    n = bh * t
    n_sc = 3 + e
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
    }
    # launches that carry a second, independent stage as extra workgroups
    per_kernel["k_fwd_seg_scan+buffer_out"] = per_kernel["k_fwd_seg_scan"] + per_kernel["k_buffer_out"]
    per_kernel["k_scalar_chain+fixup"] = per_kernel["k_bwd_scalar"] + per_kernel["k_bwd_seg_fixup"] + st
    # the specialised bf16 d = 64 path launches these kernels for the same stages
    for spec, gen in (("k_walk_agg", "k_fwd_seg_agg"), ("k_walk_full", "k_fwd_seg"), ("k_walk_bwd", "k_bwd_seg"),
                      ("k_scalar_chain", "k_bwd_scalar")):
        per_kernel[spec] = per_kernel[gen]
    return fwd, bwd, per_kernel


def make_inputs(device):
    import torch
    g = torch.Generator().manual_seed(1003)       # seed = 1000 + config number
    r = lambda *s: torch.randn(*s, generator=g)
    k = r(BH, T, D)
    k = k / k.norm(dim=-1, keepdim=True)
    x = dict(k=k, q=r(BH, T, D), v=r(BH, T, D),
             lr=0.1 * torch.sigmoid(r(BH, T)), decay=torch.sigmoid(r(BH, T) * 0.5 + 2.0),
             beta=torch.sigmoid(r(BH, T) * 0.5 + 1.0), gate=torch.softmax(r(BH, T, E), dim=-1),
             dy=r(BH, T, D))
    out = {kk: v.to(device=device, dtype=torch.bfloat16).contiguous() for kk, v in x.items()}
    zeros = torch.zeros(BH, D, D, device=device, dtype=torch.float32)
    out.update(S_ref=zeros, S0=zeros, Z0=zeros)
    return out, x


def cpu_baseline(x_cpu, sample_t=256, reps=3):
    """Oracle (fp32, autograd) on the first `sample_t` tokens of every (b, h): 1 warmup, median
    of `reps`. Returns tokens/s of the sample and the thread count."""
    import torch
    from oracle import memory_recurrence_vectorised
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(cores)
    sl = slice(0, sample_t)
    f32 = torch.float32
    leaves = {kk: x_cpu[kk][:, sl].to(torch.bfloat16).to(f32).clone().requires_grad_(True)
              for kk in ("k", "q", "v", "lr", "decay", "beta", "gate")}
    dy = x_cpu["dy"][:, sl].to(torch.bfloat16).to(f32)
    S0 = torch.zeros(BH, D, D, requires_grad=True)
    Z0 = torch.zeros(BH, D, D, requires_grad=True)
    times = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        y, S_T, Z_T, buf = memory_recurrence_vectorised(
            leaves["k"], leaves["q"], leaves["v"], leaves["lr"], leaves["decay"], leaves["beta"], leaves["gate"],
            S0, S0, Z0, None, window=E)
        (y * dy).sum().backward()
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        for t in list(leaves.values()) + [S0, Z0]:
            t.grad = None
    med = statistics.median(times)
    return B * sample_t / med, cores, med


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_c3.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary (lines
    `traffic: <kernel> <bytes>`, FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel factor), or
    None when the summary has no figure for it."""
    try:
        with open(TRAFFIC_FILE) as f:
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


# The other BASELINE configs (`--config c2|c4|c5`): one JSON line each, same keys; the default
# run (no flag) is the C3 headline above. Tokens are (b, t) positions through one memory layer.
OTHER_CONFIGS = {
    # Titans-RNN with momentum, no window, no gate, bf16, B=4 H=8 T=2048 d=64
    "c2": dict(B=4, H=8, T=2048, dk=64, dv=64, e=1, gate=None, seed=1002,
               workload="C2 Titans-RNN memory layer: B=4 H=8 T=2048 d=64, momentum, bf16 inputs, fp32 state, "
                        "chunk 64"),
    # OmegaNet-RNN with the tensor feature map phi = elementwise_g3([k; vec(k k^T)] P), P: 4160 -> 128
    # (Xavier-uniform), d_k = 128, d_v = 64, e = 8, lag gates; the map's GEMM is part of the step
    "c4": dict(B=2, H=8, T=8192, dk=128, dv=64, e=8, gate="lag", seed=1004, tensor_map=True,
               workload="C4 OmegaNet-RNN memory layer with the tensor feature map (64+4096 -> 128, then the "
                        "elementwise map of degree 3): B=2 H=8 T=8192 d_k=128 d_v=64 e=8 lag gates, momentum, "
                        "bf16 inputs, fp32 state"),
    # the memory core of one layer of the byte-level RNN transformer: B=8 H=8 T=2048, e=4, per-token gates
    "c5": dict(B=8, H=8, T=2048, dk=64, dv=64, e=4, gate="token", seed=1005,
               workload="C5 memory core of one RNN-transformer layer: B=8 H=8 T=2048 d=64 e=4 per-token gates, "
                        "momentum, bf16 inputs, fp32 state"),
}


def run_other_config(name, steps, warmup):
    """fwd+bwd of config `name` through the autograd API (torch.autograd.grad of y against a fixed
    random output gradient, i.e. the gradient of sum(y * g))."""
    import torch
    from atlas_rnn_amd.functional import memory_recurrence, tensor_feature_map
    c = OTHER_CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bh, t, dk, dv, e = c["B"] * c["H"], c["T"], c["dk"], c["dv"], c["e"]
    g = torch.Generator().manual_seed(c["seed"])
    r = lambda *sh: torch.randn(*sh, generator=g)
    bf = lambda x: x.to(device=dev, dtype=torch.bfloat16).contiguous()
    tensor_map = c.get("tensor_map", False)
    kin = 64 if tensor_map else dk
    k = r(bh, t, kin)
    k = k / k.norm(dim=-1, keepdim=True)
    q = r(bh, t, kin)
    q = q / q.norm(dim=-1, keepdim=True) if tensor_map else q
    gate = None
    if c["gate"] == "lag":
        gate = torch.softmax(r(bh, t, e), dim=-1)
    elif c["gate"] == "token":
        gate = torch.sigmoid(r(bh, t))
    leaves = dict(k=bf(k), q=bf(q), v=bf(r(bh, t, dv)), lr=bf(0.1 * torch.sigmoid(r(bh, t))),
                  decay=bf(torch.sigmoid(r(bh, t) * 0.5 + 2.0)), beta=bf(torch.sigmoid(r(bh, t) * 0.5 + 1.0)),
                  gate=bf(gate) if gate is not None else None)
    for v in leaves.values():
        if v is not None:
            v.requires_grad_(True)
    P = None
    if tensor_map:   # Xavier-uniform (64 + 4096) -> 128, seeded
        bound = (6.0 / (kin + kin * kin + dk)) ** 0.5
        P = bf((torch.rand(kin + kin * kin, dk, generator=g) * 2 - 1) * bound)
    gy = bf(r(bh, t, dv))
    zeros = torch.zeros(bh, dv, dk, device=dev)

    def feat(x):   # fused tensor-map kernels, elementwise map of degree 3 in their epilogue
        return tensor_feature_map(x, P, degree=3) if tensor_map else x

    def step():
        y, S_T, Z_T, B_out = memory_recurrence(
            feat(leaves["k"]), feat(leaves["q"]), leaves["v"], leaves["lr"], leaves["decay"], leaves["beta"],
            leaves["gate"], zeros, zeros, zeros, None, window=e)
        ins = [v for v in leaves.values() if v is not None]
        torch.autograd.grad(y, ins, grad_outputs=gy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    tokens = c["B"] * t
    out = {"metric": "memory-layer tokens/s fwd+bwd", "value": round(tokens * steps / el, 1), "unit": "tokens/s",
           "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(1e3 * el / steps, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded)", "config": {"workload": c["workload"], "global_batch": c["B"],
                                                     "seq_len": t, "heads": c["H"], "d_k": dk, "d_v": dv,
                                                     "window": e, "parallelism": "single GPU"}}
    print(json.dumps(out), flush=True)


def run_decode(steps, warmup):
    """Generation steps at the C3 head shape (B=4 H=8 d=64 e=4 lag gates, momentum, bf16 inputs,
    fp32 state): atlas_mem_step through the C ABI with the state updated in place, the way a decode
    loop carries it. One step = one token for every sequence of the batch; `value` counts those
    (b) tokens per second. The kernel is timed with events on the stream it runs on; its
    algorithmic bytes are the state read and written once (S_ref, S0, Z0, buffer in; S_T, Z_T,
    buffer out) plus the token's vectors."""
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
    stream = _stream(dev)

    def step():
        _lib.check(lib.atlas_mem_step(ctypes.byref(prob), ctypes.byref(a), stream), "atlas_mem_step")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    us = 1e3 * ev0.elapsed_time(ev1) / steps
    state_bytes = bh * d * d * 4 * (3 + 2 + 2 * (e - 1))   # S_ref, S0, S_T; Z0, Z_T; buffer in / out
    vec_bytes = bh * (3 * d + 3 + e) * 2 + bh * d * 2       # k, q, v, scalars, gates; y
    alg = state_bytes + vec_bytes
    out = {"metric": "decode tokens/s (one memory-layer step per token)", "value": round(B / (us * 1e-6), 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(us / 1e3, 6),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded)",
           "config": {"workload": "decode step at the C3 head shape: B=4 H=8 d=64 e=4 lag gates, momentum, "
                                  "state in place", "global_batch": B, "seq_len": 1, "parallelism": "single GPU"},
           "roofline": {"bound": "hbm", "achieved": round(alg / (us * 1e-6) / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                        "frac": round(alg / (us * 1e-6) / 8e12, 4), "traffic": None}}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-tokens", type=int, default=256)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain copy kernel of known size (HBM counter calibration)")
    ap.add_argument("--config", choices=["c3"] + sorted(OTHER_CONFIGS) + ["decode"], default="c3",
                    help="c3 (default): the headline; c2 / c4 / c5: the other BASELINE configs; decode: the "
                         "one-token step")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.config != "c3":
        if args.gpus != 1:
            print("bench.py measures one GPU (use --gpus 1).", file=sys.stderr)
            sys.exit(2)
        if args.config == "decode":
            run_decode(args.steps, args.warmup)
        else:
            run_other_config(args.config, args.steps, args.warmup)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the memory-layer recurrence shards over (batch, head) rows "
              "with no exchange, so there is no multi-GPU figure to report (use --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch
    from atlas_rnn_amd.functional import RecurrencePlan, profile_enable, profile_read

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, x_cpu = make_inputs(dev)
    plan = RecurrencePlan(BH, T, D, window=E, momentum=True, gate_mode='lag', dtype=torch.bfloat16, device=dev)

    def step():
        plan.forward(x["k"], x["q"], x["v"], x["lr"], x["decay"], x["beta"], x["gate"], x["S_ref"], x["S0"], x["Z0"])
        plan.backward(x["dy"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: K steps, nothing else on the stream
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # the same K steps again with the library's per-kernel HIP events on the launch stream; the
    # event records between launches lengthen the step, so only kernel durations come from here
    profile_enable(True)
    profile_read(reset=True)
    torch.cuda.synchronize()
    tp0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    tp1 = time.perf_counter()
    prof = profile_read(reset=True)
    profile_enable(False)

    elapsed = t1 - t0
    ms_per_step = 1e3 * elapsed / args.steps
    value = TOKENS * args.steps / elapsed
    fwd_b, bwd_b, per_kernel = algorithmic_bytes()
    step_bytes = fwd_b + bwd_b
    kernels = {name: {"avg_us": 1e3 * ms / max(n, 1), "launches": n} for name, (ms, n) in prof.items() if n}
    dom = max(kernels, key=lambda kk: kernels[kk]["avg_us"] * kernels[kk]["launches"])
    dom_s = kernels[dom]["avg_us"] * 1e-6
    achieved = per_kernel[dom] / dom_s / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": measured_traffic(dom),
                "algorithmic_bytes_per_launch": per_kernel[dom], "avg_launch_us": round(kernels[dom]["avg_us"], 2)}
    step_gbs = step_bytes / (elapsed / args.steps) / 1e9
    out = {
        "metric": "memory-layer tokens/s fwd+bwd at H=8,d=64,T=4096; % HBM/MFMA roofline",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v with L2-normalised keys, sigmoid gates, softmax lag gates)",
        "config": {"workload": "C3 OmegaNet-RNN memory layer: B=4 H=8 T=4096 d=64 e=4 lag gates, momentum, "
                               "bf16 inputs, fp32 state, chunk 64", "global_batch": B, "seq_len": T,
                   "heads": H, "d": D, "window": E, "parallelism": "single GPU"},
        "roofline": roofline,
        "step_roofline": {"bytes_per_step": step_bytes, "achieved_gbs": round(step_gbs, 2),
                          "frac": round(step_gbs / HBM_PEAK_GBS, 5)},
        "kernels": {kk: {"avg_us": round(v["avg_us"], 2), "launches": v["launches"]} for kk, v in kernels.items()},
        "profiled_ms_per_step": round(1e3 * (tp1 - tp0) / args.steps, 4),
    }
    if not args.no_cpu_baseline:
        cpu_tps, cores, med = cpu_baseline(x_cpu, sample_t=args.cpu_sample_tokens)
        out["cpu_baseline"] = {"value": round(cpu_tps, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
                               "sample": f"oracle fp32 fwd+bwd (autograd) on tokens 0..{args.cpu_sample_tokens - 1} "
                                         f"of all {BH} (b,h) rows, median of 3 = {med:.2f} s"}
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
