"""Benchmark of the window hot path on one MI355X: window positions/s, fwd+bwd, at the ref shape.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config ref] [--no-cpu]

A step is one window of the configuration, inputs resident in HBM: the router and the forward
sweep (``hsn_win_route`` then ``hsn_win_forward``, the library's choice; ``--route-forward one``
times ``hsn_win_route_forward`` as one launch, its forward's workgroups routing the window
themselves) and the backward with the carried-state gradient (``hsn_win_backward``). ``value`` is positions/s over K timed steps
launched eagerly as a PyTorch loop calls them (B*T positions per step, bracketed by
synchronisations); ``--graph`` times K replays of the step captured as a HIP graph instead
(``ms_per_step_graph`` is reported either way unless ``--no-graph``). Each kernel's average
duration is measured with HIP events recorded on the stream the kernels run on (torch's current
stream), over K eager steps queued behind device copies so that the kernels run back to back;
``roofline`` reports the dominant part's algorithmic bytes per launch (the byte model of
``hsn_amd.workload.byte_model``) over its average duration against the 8 TB/s HBM peak.
``cpu_baseline`` times the repository's CPU oracle (the reference's profile:cpu algorithm) on a
bounded sample of the same workload on the host cores. One GPU only: ``--gpus`` above 1 exits.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def _args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="ref")
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--path", choices=["auto", "slice", "chain", "evmap"], default="auto",
                   help="the sweeps' design (auto: the library's choice by shape)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-h-max", action="store_true", help="do not produce the row maxima")
    p.add_argument("--route-forward", choices=["auto", "one", "two"], default="auto",
                   help="route and forward sweep as the library chooses, as one launch "
                        "(hsn_win_route_forward where the routed forward takes the shape) or as "
                        "two (hsn_win_route, hsn_win_forward)")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="after the timed steps, copy a buffer of MIB MiB three times (outside "
                        "the timed region): the reference kernel for scaling rocprofv3's "
                        "FETCH_SIZE / WRITE_SIZE counters")
    p.add_argument("--graph", action="store_true",
                   help="value from replays of the step captured as a HIP graph")
    p.add_argument("--no-graph", action="store_true",
                   help="skip the graph capture and its replays")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="repeat the CPU baseline's sample until this much time has passed")
    p.add_argument("--sweep", choices=["ref", "tiny"], default=None,
                   help="measure the state-gradient reverse sweep (hsn_amd.state_sweep) at this "
                        "workload instead of the window (not the headline line)")
    p.add_argument("--products", choices=["bf16", "f32"], default="bf16",
                   help="the reverse sweep's product dtype (bf16: autocast's)")
    p.add_argument("--three-steps", action="store_true",
                   help="the reverse sweep's three glue steps around all-units GEMMs instead of "
                        "the fused step")
    p.add_argument("--round", choices=["ref", "tiny"], default=None,
                   help="measure the fused cell round (hsn::window_cell_round) over a window of "
                        "positions at this workload instead of the window (not the headline line)")
    p.add_argument("--ops", choices=["ref", "model"], default=None,
                   help="measure the P2.9 ops (include/hsn_ops.h) one call at a time at the "
                        "golden vectors' ref size or the reference model's per-position size "
                        "(not the headline line)")
    p.add_argument("--round-positions", type=int, default=64,
                   help="positions a --round step runs (the state carried from one to the next)")
    p.add_argument("--trainer", choices=sorted(TRAINER_LISTS), default=None,
                   help="measure the trainer's AdamW pass (hsn_tr_adamw) over a synthetic "
                        "parameter list instead of the window (not the headline line)")
    return p.parse_args()


#: Synthetic parameter lists for ``--trainer``: (tensor sizes, what they stand for). "model" is
#: the size of the reference's trained models (about 2 M parameters: weights, biases, gains);
#: "large" 256 M parameters in 64 tensors, where the pass is HBM-bound.
TRAINER_LISTS = {
    "model": ([64 * 64] * 48 + [256 * 64] * 96 + [64] * 48 + [256 * 128] * 6, "1.97 M in 198"),
    "large": ([1 << 22] * 64, "256 M in 64"),
}
#: Algorithmic HBM bytes per element of the AdamW pass: reads param, grad, exp_avg, exp_avg_sq
#: and writes param, exp_avg, exp_avg_sq, 4 bytes each.
TRAINER_BYTES_PER_ELEMENT = 28


def _traffic(workload: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter summary
    (profiles/traffic_<workload>.json), or None."""
    path = ROOT / "profiles" / f"traffic_{workload}.json"
    if not path.is_file():
        return None
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


def _cpu_model() -> str:
    """The host CPU's model name (``/proc/cpuinfo``), as ``lscpu`` reports it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _copy_gbs(dev, mib: int = 512, reps: int = 5) -> float:
    """A plain device copy's bandwidth (bytes read plus written per second, in GB/s), of a
    buffer larger than the 256 MB Infinity Cache so that it streams from HBM: the bandwidth a
    kernel of perfect access pattern reaches on this card, beside the 8 TB/s peak."""
    import torch

    src = torch.ones(mib * (1 << 20) // 4, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    secs = t0.elapsed_time(t1) * 1e-3
    del src, dst
    return 2.0 * mib * (1 << 20) * reps / secs / 1e9


def _cpu_baseline(cfg, seed, min_seconds):
    """The CPU oracle on one full window of the configuration (or a prefix of its positions for
    the large configurations), on all host cores, repeated until ``min_seconds`` have passed."""
    import torch

    from hsn_amd.workload import make_cotangents, make_window
    from oracle import hsn_oracle as O

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    T = cfg.T if cfg.B * cfg.T <= 8192 else max(8, 8192 // cfg.B)
    sample = cfg.scaled(T=T)
    w = make_window(sample, seed)
    c = make_cotangents(sample, seed)
    kw = dict(k=sample.K)
    # warm-up on two positions
    short = {k: (v[:, :2] if k in ("logits", "y", "gate_pre", "reset") else v) for k, v in w.items()}
    O.window_forward(short["logits"], short["y"], short["gate_pre"], short["reset"], w["h0"], w["q0"],
                     w["age0"], w["pos0"], w["cost"], **kw)
    reps = 0
    t0 = time.perf_counter()
    while True:
        f = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                             w["age0"], w["pos0"], w["cost"], **kw)
        O.window_backward(w["y"], w["gate_pre"], f["h_old"], f["cells"], f["valid"], w["reset"],
                          sample.N, c["d_q_pre"], c["d_q_post"],
                          torch.where(f["valid"][..., None], c["d_h_sel"].float(),
                                      0.0).to(c["d_h_sel"].dtype),
                          c["d_h_T"], c["d_q_T"])
        reps += 1
        secs = time.perf_counter() - t0
        if secs >= min_seconds:
            break
    positions = sample.B * sample.T * reps
    return {
        "value": positions / secs,
        "unit": "positions/s",
        "cores": torch.get_num_threads(),
        "cpu": _cpu_model(),
        "kind": "port",
        "sample": f"{reps} x ({sample.B} rows x {sample.T} positions of the {cfg.name} window), "
                  f"fwd+bwd, the repository's PyTorch-CPU oracle ({secs:.1f} s)",
    }


def _trainer_main(args) -> int:
    """The AdamW pass (``hsn_tr_adamw``) against the PyTorch multi-tensor sequence it replaces
    (the reference's ``LazyAdamW._dense_steps``) over one synthetic parameter list, on the same
    device. A step is one optimiser step over the whole list; ``value`` is elements/s of the
    pass (eager launches, host work included); the roofline is the pass's kernel time from HIP
    events on its stream (the launches queued behind device copies so they run back to back)."""
    import torch

    from hsn_amd import trainer

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    sizes, what = TRAINER_LISTS[args.trainer]
    gen = torch.Generator(device=dev).manual_seed(args.seed)

    def make():
        return [torch.randn(n, device=dev, generator=gen) for n in sizes]

    params, grads, exp_avgs = make(), make(), make()
    exp_avg_sqs = [g.square() for g in make()]
    hyper = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)
    elements = sum(sizes)

    def pass_step(step):
        assert trainer.adamw(params, grads, exp_avgs, exp_avg_sqs, step=step, **hyper)

    def torch_step(step):
        lr, b1, b2 = hyper["lr"], hyper["beta1"], hyper["beta2"]
        torch._foreach_mul_(params, 1 - lr * hyper["weight_decay"])
        torch._foreach_lerp_(exp_avgs, grads, 1 - b1)
        torch._foreach_mul_(exp_avg_sqs, b2)
        torch._foreach_addcmul_(exp_avg_sqs, grads, grads, value=1 - b2)
        denoms = torch._foreach_sqrt(exp_avg_sqs)
        torch._foreach_div_(denoms, (1 - b2**step) ** 0.5)
        torch._foreach_add_(denoms, hyper["eps"])
        torch._foreach_addcdiv_(params, exp_avgs, denoms, value=-lr / (1 - b1**step))

    def timed(fn):
        for i in range(args.warmup):
            fn(i + 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            fn(args.warmup + i + 1)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / args.steps

    pass_secs = timed(pass_step)
    torch_secs = timed(torch_step)
    busy = torch.empty(64 << 20, device=dev)
    busy_dst = torch.empty_like(busy)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    torch.cuda.synchronize()
    for _ in range(args.steps + 8):
        busy_dst.copy_(busy)
    for i, (a, b) in enumerate(events):
        a.record()
        pass_step(i + 1)
        b.record()
    torch.cuda.synchronize()
    kernel_ms = sum(a.elapsed_time(b) for a, b in events) / args.steps
    achieved = elements * TRAINER_BYTES_PER_ELEMENT / (kernel_ms * 1e-3) / 1e9
    launches = -(-len([n for n in sizes if n]) // 88)  # tensors a launch of the AdamW pass
    result = {
        "metric": f"trainer AdamW pass elements/sec ({args.trainer} parameter list, 1 GPU)",
        "value": elements / pass_secs,
        "unit": "elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pass_secs * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded normal parameters, gradients and moments)",
        "config": {"workload": f"trainer_adamw_{args.trainer}", "tensors": len(sizes),
                   "elements": elements, "list": what, "launches_per_step": launches,
                   "parallelism": "single GPU"},
        "roofline": {
            "bound": "hbm",
            "kernel": "tr_pass<kAdamW>",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
        },
        "kernel_ms": kernel_ms,
        "torch_foreach_ms_per_step": torch_secs * 1e3,
        "speedup_vs_torch_foreach": torch_secs / pass_secs,
    }
    if not args.no_cpu:  # the oracle's restatement on a bounded sample, one host thread
        from oracle import hsn_oracle as O

        rng = np.random.default_rng(args.seed)
        n = 1 << 20
        p, g, m = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
        v = np.square(rng.standard_normal(n)).astype(np.float32)
        coefs = [1 - 1e-5, 0.1, 0.999, 0.001, 1 / 0.001**0.5, 1e-8, -1e-2]
        reps, t0 = 0, time.perf_counter()
        while True:
            p, m, v = O.tr_adamw(p, g, m, v, coefs, True)
            reps += 1
            secs = time.perf_counter() - t0
            if secs >= args.cpu_seconds:
                break
        result["cpu_baseline"] = {
            "value": n * reps / secs, "unit": "elements/s", "cores": 1, "kind": "port",
            "sample": f"{reps} x AdamW over {n} elements, the repository's numpy oracle "
                      f"({secs:.1f} s)",
        }
    print(json.dumps(result), flush=True)
    return 0


def _sweep_main(args) -> int:
    """The state-gradient reverse sweep over one synthetic window of the workload: a step is the
    runner's call for one window (the window's values loaded into the sweep's buffers, the T
    positions replayed from the captured HIP graph, the results copied out), inputs resident in
    HBM; ``value`` is positions/s (B x T per window; the replay alone is reported beside). Each part's
    duration comes from HIP events between the parts of eager windows queued behind device
    copies; the roofline is the dominant part's against its bound (the products: the all-units
    GEMMs' FLOPs against the MFMA peak of the product dtype; the glue: its bytes against HBM)."""
    import torch

    from hsn_amd.state_sweep import ReverseSweep, SweepRunner, sweep_shape
    from hsn_amd.workload import SWEEP_CONFIGS, make_sweep_window

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    shape_kw = SWEEP_CONFIGS[args.sweep]
    product = torch.bfloat16 if args.products == "bf16" else torch.float32
    wargs, wkw = make_sweep_window(**shape_kw, seed=args.seed, device=dev, product_dtype=product)
    runner = SweepRunner(graph=True, fused=False if args.three_steps else None)
    assert runner(*wargs, **wkw) is not None, "the runner declined the workload"
    (sweep,) = runner.sweeps.values()
    torch.cuda.synchronize()
    # a step is the runner's whole call for a window, as the reference's autograd node makes it:
    # the window's values into the static buffers, the graph's replay, the results' copies
    for _ in range(args.warmup):
        runner(*wargs, **wkw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        runner(*wargs, **wkw)
    torch.cuda.synchronize()
    step_secs = (time.perf_counter() - t0) / args.steps
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sweep.run()
    torch.cuda.synchronize()
    graph_secs = (time.perf_counter() - t0) / args.steps
    s = sweep.shape
    # per part: eager windows with events between the parts, behind a queue of device copies
    windows = max(1, min(args.steps, 3))
    busy = torch.empty(64 << 20, device=dev)
    busy_dst = torch.empty_like(busy)
    import ctypes

    from hsn_amd import _lib

    parts = (("cell step", "tail") if sweep.fused else
             ("head", "act product", "middle", "dv product", "tail"))
    events = []
    torch.cuda.synchronize()
    for _ in range(windows * s.T // 4 + 8):
        busy_dst.copy_(busy)
    stream = _lib.stream_of(dev)
    ref = ctypes.byref(sweep._struct)
    for _ in range(windows):
        for t in range(s.T - 1, -1, -1):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)]
            if sweep.fused:
                ev[0].record()
                _lib.call("hsn_win_back_cell", ref, t, stream)
                ev[1].record()
                _lib.call("hsn_win_back_cell_tail", ref, t, stream)
                ev[2].record()
                events.append(ev)
                continue
            ev[0].record()
            _lib.call("hsn_win_back_head", ref, t, stream)
            ev[1].record()
            torch.mm(sweep.op1, sweep.w2_t, out=sweep.act)
            ev[2].record()
            _lib.call("hsn_win_back_mid", ref, t, stream)
            ev[3].record()
            torch.mm(sweep.op2, sweep.w1_state_t, out=sweep.dv)
            ev[4].record()
            _lib.call("hsn_win_back_tail", ref, t, stream)
            ev[5].record()
            events.append(ev)
    torch.cuda.synchronize()
    del busy, busy_dst
    per_part = {p: sum(ev[i].elapsed_time(ev[i + 1]) for ev in events) / (windows * s.T)
                for i, p in enumerate(parts)}  # ms per position
    rows = s.B * s.K
    esize = 2 if product == torch.bfloat16 else 4
    flops = {"act product": 2.0 * rows * s.M * s.d * s.H,  # the all-units GEMMs
             "dv product": 2.0 * rows * (s.M * s.H + s.d) * 2 * s.d,
             # the fused step multiplies each slot's own unit blocks only
             "cell step": 2.0 * rows * (s.d * s.H + (s.H + s.d) * 2 * s.d)}
    peak_tf = 2500.0 if product == torch.bfloat16 else 157.3
    touched = min(s.N, s.K * (int(shape_kw["D"]) + 1))  # cells a row's tail reads and writes
    glue_bytes = {  # algorithmic bytes per position
        # c, b, h_old, d_h_sel, y, gate_pre read, A read and written, dc, db written (fp32);
        # op1's block cleared and written, op2's gate columns written
        "head": rows * s.d * (11 * 4 + 3 * esize),
        # hidden and act read, op2's block cleared and written
        "middle": rows * s.H * 4 * esize,
        # dv read, h_old and m V read (fp32), the touched cells' rows of A read and written
        "tail": rows * s.d * (2 * esize + 2 * 4) + s.B * touched * s.d * 8,
    }
    dominant = max(per_part, key=per_part.get)
    if dominant in flops:
        achieved = flops[dominant] / (per_part[dominant] * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": dominant, "achieved": achieved, "peak": peak_tf,
                "unit": "TFLOP/s", "frac": achieved / peak_tf, "traffic": None}
    else:
        achieved = glue_bytes[dominant] / (per_part[dominant] * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": dominant, "achieved": achieved, "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None}
    positions = s.B * s.T
    result = {
        "metric": f"state-gradient reverse sweep positions/sec ({args.sweep} model, 1 GPU)",
        "value": positions / step_secs,
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_secs * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if product == torch.bfloat16 else "f32",
        "data": "synthetic (hsn_amd/workload.py make_sweep_window)",
        "config": {"workload": f"sweep_{args.sweep}", **shape_kw, "products": args.products,
                   "timing": "the runner's call per window: load, HIP graph replay, result copies",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "parts_us_per_position": {k: v * 1e3 for k, v in per_part.items()},
        "fused_step": sweep.fused,
        "position_us_graph": graph_secs / s.T * 1e6,
        "ms_per_window_replay_only": graph_secs * 1e3,
    }
    if not args.no_cpu:  # the oracle on a bounded sample: 2 rows x 8 positions, one thread
        from oracle import state_gradient as O

        torch.set_num_threads(1)
        sample = dict(shape_kw, B=2, T=8)
        cargs, _ = make_sweep_window(**sample, seed=args.seed)
        record = dict(cargs[12], hidden=cargs[12]["hidden"].float())
        consts = O.CellConstants(*cargs[13])
        reps, t0 = 0, time.perf_counter()
        while True:
            O.state_gradient_backward(*cargs[:12], record, consts)
            reps += 1
            secs = time.perf_counter() - t0
            if secs >= args.cpu_seconds:
                break
        result["cpu_baseline"] = {
            "value": 2 * 8 * reps / secs, "unit": "positions/s", "cores": 1, "kind": "port",
            "sample": f"{reps} x (2 rows x 8 positions of the {args.sweep} model), the "
                      f"repository's PyTorch-CPU oracle ({secs:.1f} s)",
        }
    print(json.dumps(result), flush=True)
    return 0


#: Sizes of ``--ops``: the golden vectors' "ref" dimensions (tests/golden MANIFEST) and the
#: reference model's per-position round (B 32 rows, K 8 slots of N 256 cells, d 64, H 512, M 8,
#: 8 in-edges a cell).
OPS_SIZES = {
    "ref": dict(B=4, K=4, N=32, d=64, E=128, P=16, M=8, H=512),
    "model": dict(B=32, K=8, N=256, d=64, E=2048, P=256, M=8, H=512),
}


def _ops_main(args) -> int:
    """The P2.9 ops (``include/hsn_ops.h``), forward and backward, one call at a time: device
    time per call from HIP events around ``--steps`` calls queued behind device copies (so host
    dispatch is not counted), synthetic fp32 inputs of the size's shapes. ``value`` is the
    grouped unit MLP's forward calls/s; its roofline is against the fp32 MFMA peak (useful
    FLOPs: 2 P (4d H + H d)). The reference's own comparison is per op against its PyTorch path
    (``scripts/bench_kernels.py``); here the CPU oracle of the unit MLP stands beside it."""
    import torch

    from hsn_amd.kernels import ops

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    z = OPS_SIZES[args.ops]
    B, K, N, d, E, P, M, H = (z[k] for k in ("B", "K", "N", "d", "E", "P", "M", "H"))
    g = torch.Generator().manual_seed(args.seed)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dev)

    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)]).to(dev)
    valid = torch.ones(B, K, dtype=torch.int32, device=dev)
    h, q = rnd(B, N, d, scale=0.5), rnd(B, d)
    age = torch.zeros(B, N, dtype=torch.int32, device=dev)
    c, b = rnd(B, K, d).tanh(), torch.sigmoid(rnd(B, K, d))
    u, eps, m = rnd(B, d), rnd(B, d), rnd(B, K, d)
    unit = torch.randint(0, M, (P,), generator=g).to(dev)
    v = rnd(P, 4 * d)
    w1, b1 = rnd(M, 4 * d, H, scale=(4 * d) ** -0.5), rnd(M, H, scale=0.1)
    w2, b2 = rnd(M, H, d, scale=H ** -0.5), rnd(M, d, scale=0.1)
    deg = torch.full((N,), E // N, dtype=torch.int64)
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), deg.cumsum(0)]).to(dev)
    indices = torch.randint(0, N, (E,), generator=g).to(dev)
    a = torch.rand(E, generator=g).to(dev)
    V = rnd(d, d, scale=d ** -0.5)
    out, hidden = ops.mlp_op(v, unit, w1, b1, w2, b2)
    calls = {
        "gated_delta_update_functional": lambda: ops.update_op(
            h, q, age.long(), idx, valid, c, b),
        "gated_delta_update_backward": lambda: ops.update_backward(
            idx, valid, c, b, c, h, q),
        "gather_concat": lambda: ops.gather_op(u, eps, h, m, idx),
        "gather_concat_backward": lambda: ops.gather_backward(
            rnd_dv, idx, N),
        "grouped_unit_mlp": lambda: ops.mlp_op(v, unit, w1, b1, w2, b2),
        "grouped_unit_mlp_backward": lambda: ops.mlp_backward(
            v, unit, w1, w2, hidden, out),
        "csr_messages": lambda: ops.messages_op(h, indptr, indices, a, V, idx),
        "csr_messages_backward": lambda: ops.messages_backward(
            h, indptr, indices, a, V, idx, m),
    }
    # the same calls as the adapters make them outside grad mode: the ops' bodies without the
    # custom op's dispatch
    direct = {
        "gated_delta_update_functional": lambda: ops._functional(
            h, q, age.long(), idx, valid, c, b),
        "gated_delta_update_backward": lambda: ops._update_bwd_body(
            idx, valid, c, b, c, h, q),
        "gather_concat": lambda: ops._gather_body(u, eps, h, m, idx),
        "gather_concat_backward": lambda: ops._gather_bwd_body(rnd_dv, idx, N),
        "grouped_unit_mlp": lambda: ops._mlp_body(v, unit, w1, b1, w2, b2),
        "grouped_unit_mlp_backward": lambda: ops._mlp_bwd_body(v, unit, w1, w2, hidden, out),
        "csr_messages": lambda: ops._messages_body(h, indptr, indices, a, V, idx),
        "csr_messages_backward": lambda: ops._messages_bwd_body(
            h, indptr, indices, a, V, idx, m),
    }
    rnd_dv = rnd(B, K, 4 * d)
    busy = torch.empty(64 << 20, device=dev)
    busy_dst = torch.empty_like(busy)
    per_call, end_to_end, end_to_end_direct = {}, {}, {}
    with torch.no_grad():
        for name, fn in calls.items():
            for _ in range(max(1, args.warmup)):
                fn()
            torch.cuda.synchronize()
            # one 256 MiB copy (about 100 us) a call queued ahead, so the host's dispatch of the
            # calls (Python and the op wrappers, tens of us a call) ends before the device's work
            for _ in range(args.steps + 8):
                busy_dst.copy_(busy)
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
            for _ in range(args.steps):
                fn()
            ev[1].record()
            torch.cuda.synchronize()
            per_call[name] = ev[0].elapsed_time(ev[1]) / args.steps * 1e3  # us
            # end to end: the same calls from an idle queue, host dispatch included
            t0 = time.perf_counter()
            for _ in range(args.steps):
                fn()
            torch.cuda.synchronize()
            end_to_end[name] = (time.perf_counter() - t0) / args.steps * 1e6
            t0 = time.perf_counter()
            for _ in range(args.steps):
                direct[name]()
            torch.cuda.synchronize()
            end_to_end_direct[name] = (time.perf_counter() - t0) / args.steps * 1e6
    del busy, busy_dst
    mlp_us = per_call["grouped_unit_mlp"]
    flops = 2.0 * P * (4 * d * H + H * d)
    achieved = flops / (mlp_us * 1e-6) / 1e12
    result = {
        "metric": f"grouped unit MLP forward calls/sec of device time ({args.ops} size, 1 GPU)",
        "value": 1e6 / mlp_us,
        "unit": "calls/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": mlp_us * 1e-3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, bench.py OPS_SIZES shapes)",
        "config": {"workload": f"ops_{args.ops}", **z,
                   "timing": "HIP events around the calls, queued behind device copies",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "grouped_unit_mlp forward",
                     "achieved": achieved, "peak": 157.3, "unit": "TFLOP/s",
                     "frac": achieved / 157.3, "traffic": None, "flops_per_call": flops},
        "us_per_call": per_call,
        # the rate a Python caller reaches: host dispatch (the op wrappers and ctypes) included
        "us_per_call_end_to_end": end_to_end,
        "us_per_call_end_to_end_direct": end_to_end_direct,
    }
    if not args.no_cpu:  # the oracle's unit MLP on the same size, one thread
        from oracle import hsn_oracle as O

        torch.set_num_threads(1)
        cpu = [t.cpu() for t in (v, unit, w1, b1, w2, b2)]
        reps, t0 = 0, time.perf_counter()
        while True:
            O.grouped_unit_mlp(*cpu)
            reps += 1
            secs = time.perf_counter() - t0
            if secs >= args.cpu_seconds:
                break
        result["cpu_baseline"] = {
            "value": reps / secs, "unit": "calls/s", "cores": 1, "kind": "port",
            "sample": f"{reps} calls of the repository's PyTorch-CPU oracle grouped_unit_mlp at "
                      f"the same size ({secs:.1f} s)",
        }
    print(json.dumps(result), flush=True)
    return 0


def _round_main(args) -> int:
    """The fused cell round over a window of T synthetic positions (the state carried from one
    position to the next, as the forward sweep runs it): a step is the T positions' rounds, inputs
    and decisions resident in HBM; ``value`` is positions/s (B x T per step) from replays of the
    step captured as a HIP graph (the op allocates nothing the graph cannot hold), the eager rate
    beside it. The roofline treats the round's two launches as one unit: the algorithmic bytes
    of a position (``hsn_amd.workload.round_bytes``) over its device time, from HIP events on the
    replay stream around the timed replays (the two kernels' rocprofv3 averages add up to it)."""
    import torch

    from hsn_amd.kernels.window import _cell_round_run, cell_round_op
    from hsn_amd.workload import (ROUND_CONFIGS, make_round_cell, make_round_positions,
                                  round_bytes)

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    cfg = ROUND_CONFIGS[args.round]
    T = args.round_positions
    cell, edge_w = make_round_cell(N=cfg["N"], d=cfg["d"], M=cfg["M"], H=cfg["H"], D=cfg["D"],
                                   seed=args.seed, device=dev)
    pos = make_round_positions(B=cfg["B"], K=cfg["K"], N=cfg["N"], d=cfg["d"], M=cfg["M"], T=T,
                               seed=args.seed, device=dev)
    weights = [t.detach() for t in (cell.V.weight, edge_w, cell.graph._pad_src, cell.norm.weight,
                                    cell.gate.weight, cell.gate.bias, cell.units.W1,
                                    cell.units.b1, cell.units.W2, cell.units.b2,
                                    cell.W_out.weight, cell.cand_norm.weight)]
    alpha = pos["valid"].float()
    start = pos["state"]

    def one(t, h, q, age, fn=cell_round_op):
        return fn(pos["u"][t], pos["eps"][t], h, q, age, pos["cells"][t], pos["units"][t],
                  pos["valid"][t], alpha[t], *weights, True, 1e-6, 1e-6)[:3]

    def step(fn=cell_round_op):
        h, q, age = start.h, start.q, start.age
        for t in range(T):
            h, q, age = one(t, h, q, age, fn)
        return h

    with torch.no_grad():
        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        eager_secs = (time.perf_counter() - t0) / args.steps
        # the same rounds as hsn_amd.kernels.window.cell_round runs them eagerly: the op's body
        # without the custom op's dispatch
        step(_cell_round_run)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step(_cell_round_run)
        torch.cuda.synchronize()
        call_secs = (time.perf_counter() - t0) / args.steps
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize()
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        t0 = time.perf_counter()
        ev[0].record()
        for _ in range(args.steps):
            graph.replay()
        ev[1].record()
        torch.cuda.synchronize()
        step_secs = (time.perf_counter() - t0) / args.steps
    device_us = ev[0].elapsed_time(ev[1]) / (args.steps * T) * 1e3
    # units a position reads: all M at the bench's shape (B K = 256 slots over 8 units)
    present = int(torch.unique(pos["units"][0][pos["valid"][0]]).numel())
    nbytes = round_bytes(cfg, present)
    achieved = nbytes / (device_us * 1e-6) / 1e9
    positions = cfg["B"] * T
    result = {
        "metric": f"fused cell round positions/sec ({args.round} model, 1 GPU)",
        "value": positions / step_secs,
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_secs * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (hsn_amd/workload.py make_round_cell, make_round_positions)",
        "config": {"workload": f"cell_round_{args.round}", **cfg, "positions": T,
                   "timing": "HIP graph replay of the T positions' rounds",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "round_units + round_back (one position)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "bytes_per_position": nbytes},
        "position_us_device": device_us,
        "position_us_wall": step_secs / T * 1e6,
        "position_us_eager": eager_secs / T * 1e6,
        "position_us_eager_call": call_secs / T * 1e6,
    }
    if not args.no_cpu:  # the oracle on a bounded sample: 2 rows x 4 positions, one thread
        from oracle import hsn_oracle as O

        torch.set_num_threads(1)
        ccell, cedge = make_round_cell(N=cfg["N"], d=cfg["d"], M=cfg["M"], H=cfg["H"],
                                       D=cfg["D"], seed=args.seed)
        cpos = make_round_positions(B=2, K=cfg["K"], N=cfg["N"], d=cfg["d"], M=cfg["M"], T=4,
                                    seed=args.seed)
        w = dict(V=ccell.V.weight.detach(), edge_w=cedge, pad_src=ccell.graph._pad_src,
                 norm_w=ccell.norm.weight.detach(), norm_eps=1e-6,
                 gate_w=ccell.gate.weight.detach(), gate_b=ccell.gate.bias.detach(),
                 W1=ccell.units.W1, b1=ccell.units.b1, W2=ccell.units.W2, b2=ccell.units.b2,
                 W_out=ccell.W_out.weight.detach(), cand_w=ccell.cand_norm.weight.detach(),
                 cand_norm=True, cand_eps=1e-6)
        reps, t0 = 0, time.perf_counter()
        while True:
            st = cpos["state"]
            h, q, age, p_ = st.h, st.q, st.age, st.pos
            for t in range(4):
                h, q, age, p_, _ = O.window_cell_round(
                    cpos["u"][t], cpos["eps"][t], h, q, age, p_, cpos["cells"][t],
                    cpos["units"][t], cpos["valid"][t], cpos["valid"][t].float(), **w)
            reps += 1
            secs = time.perf_counter() - t0
            if secs >= args.cpu_seconds:
                break
        result["cpu_baseline"] = {
            "value": 2 * 4 * reps / secs, "unit": "positions/s", "cores": 1, "kind": "port",
            "sample": f"{reps} x (2 rows x 4 positions of the {args.round} model), the "
                      f"repository's PyTorch-CPU oracle in fp32 ({secs:.1f} s)",
        }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the window path "
              "shards over rows (each GPU owns whole rows, no exchange), so one GPU's rate "
              "times N is the job's", file=sys.stderr)
        return 2
    if args.trainer:
        return _trainer_main(args)
    if args.sweep:
        return _sweep_main(args)
    if args.round:
        return _round_main(args)
    if args.ops:
        return _ops_main(args)
    import torch

    from hsn_amd import window
    from hsn_amd.workload import CONFIGS, byte_model, describe, make_cotangents, make_window

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    from hsn_amd import _lib

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    _lib.set_path(args.path)
    io_code = _lib.DTYPE_BF16 if cfg.io == "bf16" else _lib.DTYPE_F32
    paths = {op: _lib.path_for(code, cfg.B, cfg.T, cfg.N, cfg.d, cfg.K, io_code)
             for op, code in (("forward", _lib.OP_FORWARD), ("backward", _lib.OP_BACKWARD))}
    w = {k: v.to(dev) for k, v in make_window(cfg, args.seed).items()}
    cot = make_cotangents(cfg, args.seed, carried=True)
    cot = {k: (None if v is None else v.to(dev)) for k, v in cot.items()}
    rcfg = window.RouteConfig(k=cfg.K)
    B, T, N, d, K = cfg.B, cfg.T, cfg.N, cfg.d, cfg.K
    # the parts of a step, each bracketed by HIP events: route and forward as one launch (the
    # forward's workgroups route the window themselves) or as the two
    _lib.set_route_forward(args.route_forward)
    fuses, fuse_why = window.route_forward_fuses(B, T, N, d, K, M=cfg.M,
                                                 logits_dtype=w["logits"].dtype,
                                                 io=w["y"].dtype, device=dev)
    parts = ["route_forward", "backward"] if fuses else ["route", "forward", "backward"]

    def step(ev=None):
        if ev:
            ev[0].record()
        if not fuses:
            h_max = None if args.no_h_max else torch.empty(B, T, device=dev)
            cells, units, valid, theta, refreshed, slots = window.route(
                w["logits"], w["cost"], rcfg, h_max_zero=h_max, with_slots=True)
            if ev:
                ev[1].record()
            out = window.forward(w["y"], w["gate_pre"], w["reset"], slots, w["h0"], w["q0"],
                                 w["age0"], w["pos0"], N, h_max=h_max, h_max_zeroed=True)
        else:
            out = window.route_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"],
                                       w["q0"], w["age0"], w["pos0"], w["cost"], rcfg,
                                       with_h_max=not args.no_h_max)
            slots = out["slots"]
        if ev:
            ev[len(parts) - 1].record()
        grads = window.backward(w["y"], w["gate_pre"], out["h_old"], slots, w["reset"], N,
                                cot["d_q_pre"], cot["d_q_post"], cot["d_h_sel"], cot["d_h_T"],
                                cot["d_q_T"])
        if ev:
            ev[len(parts)].record()
        return out, grads

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # eager steps as the host issues them (host work per launch included)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_secs = time.perf_counter() - t0
    # per-kernel durations: eager steps with events between the launches, queued behind a few
    # milliseconds of plain device copies so the host has issued every launch before the GPU
    # reaches them (the kernels then run back to back and an event pair brackets one kernel's
    # execution, not the host's launch latency)
    busy = torch.empty(64 << 20, device=dev)
    busy_dst = torch.empty_like(busy)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)]
              for _ in range(args.steps)]
    torch.cuda.synchronize()
    for _ in range(2 * args.steps + 8):  # about 0.1 ms each, ahead of the host's issue rate
        busy_dst.copy_(busy)
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    del busy, busy_dst
    # the step captured once as a HIP graph (its outputs in the graph's pool) and replayed K
    # times: the host's per-launch work is out of the loop, the graph launch's is in it
    secs = eager_secs
    graph_secs = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        capture = torch.cuda.Stream()
        capture.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(capture):
            step()  # warm the capture stream's allocator
        torch.cuda.current_stream().wait_stream(capture)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        graph_secs = time.perf_counter() - t0
    graphed = args.graph and graph_secs is not None
    if graphed:
        secs = graph_secs
    per_kernel = {name: sum(ev[i].elapsed_time(ev[i + 1]) for ev in events) / args.steps
                  for i, name in enumerate(parts)}  # ms per part

    bm = byte_model(cfg)
    positions = B * T
    algo = {  # algorithmic bytes per part
        "route": bm["route"] * positions,
        "forward": bm["forward_update"] * positions,
        "route_forward": bm["forward"] * positions,
        "backward": bm["backward"] * positions,
    }
    dominant = max(per_kernel, key=per_kernel.get)
    achieved = algo[dominant] / (per_kernel[dominant] * 1e-3) / 1e9
    ms_per_step = secs / args.steps * 1e3
    window_gbs = bm["window_bytes"] / (ms_per_step * 1e-3) / 1e9
    traffic = _traffic(cfg.name)
    result = {
        "metric": "window positions/sec fwd+bwd at ref shape (1 GPU); achieved HBM GB/s vs peak",
        "value": positions / (ms_per_step * 1e-3),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.io == "bf16" else "f32",
        "data": "synthetic (seeded workload generator, hsn_amd/workload.py)",
        "config": {"workload": cfg.name, "shape": describe(cfg), "B": B, "T": T, "N": N, "d": d,
                   "K": K, "M": cfg.M, "storage": cfg.io, "h_max": not args.no_h_max,
                   "sweep_path": paths, "parallelism": "single GPU",
                   "route_forward": "one launch" if fuses else f"two launches: {fuse_why}"},
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None if traffic is None else traffic.get(dominant),
        },
        "timing": "HIP graph replays of the captured step" if graphed else "eager launches",
        "ms_per_step_eager": eager_secs / args.steps * 1e3,
        "ms_per_step_graph": None if graph_secs is None else graph_secs / args.steps * 1e3,
        "kernels_ms": per_kernel,
        "kernels_gbs": {k: algo[k] / (per_kernel[k] * 1e-3) / 1e9 for k in per_kernel},
        "parts": parts,
        "window_gbs": window_gbs,
        "window_frac": window_gbs / HBM_PEAK_GBS,
    }
    copy_gbs = _copy_gbs(dev)  # after the timed region
    result["copy_gbs"] = copy_gbs
    result["roofline"]["frac_of_copy"] = achieved / copy_gbs
    result["window_frac_of_copy"] = window_gbs / copy_gbs
    if args.calibrate_copy > 0:  # outside the timed region: a plain copy of known size
        src = torch.ones(args.calibrate_copy * (1 << 20) // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = args.calibrate_copy * (1 << 20)
    if not args.no_cpu:
        result["cpu_baseline"] = _cpu_baseline(cfg, args.seed, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
