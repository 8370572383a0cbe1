"""Benchmark of the MI355X causal FLARE forward (one JSON line on stdout).

Workload: the headline is long-context prefill, config 3
(B=1, N=65536, H=16, M=256, D=128, bf16, q ~ N(0,1)/sqrt(D), k,v ~ N(0,1),
seed 2).  One step = one full forward (flare_autoregressive_triton) over the
65536 tokens with inputs already resident in HBM.  The same run also measures
config 4 (B=64 decode after a 2048-token prefill, 256 steps) and reports it
under "decode".

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]

Roofline figures (algorithmic work per launch / measured average launch time):
  prefill: 6*M*D flop per token-head (scores, encoder numerator, readout),
           peak = 2500 TFLOP/s dense bf16 MFMA;
  decode:  fp32 state read+write 2*(8M + 4*M*Dv) bytes per (b,h), plus k, v, y
           and Q, peak = 8000 GB/s HBM.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "causal-flare_amd"))

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def _cfg3_inputs(torch, device):
    torch.manual_seed(2)
    B, N, H, M, D = 1, 65536, 16, 256, 128
    q = (torch.randn(H, M, D) / math.sqrt(D)).to(torch.bfloat16)
    k = torch.randn(B, N, H, D).to(torch.bfloat16)
    v = torch.randn(B, N, H, D).to(torch.bfloat16)
    return (B, N, H, M, D), q.to(device), k.to(device), v.to(device)


def bench_prefill(torch, flare, steps, warmup):
    dev = torch.device("cuda:0")
    (B, N, H, M, D), q, k, v = _cfg3_inputs(torch, dev)
    for _ in range(warmup):
        flare.flare_autoregressive_triton(q, k, v)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        y = flare.flare_autoregressive_triton(q, k, v)
    torch.cuda.synchronize()
    dt_eager = time.perf_counter() - t0
    # The same `steps` forwards captured once in a HIP graph and replayed, as for
    # decode: the kernels are identical, the launches back to back.  Every step's
    # output of the replay must equal the eager one bit for bit, else the eager time
    # is reported.
    dt_graph, graph_ok = None, False
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                flare.flare_autoregressive_triton(q, k, v)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        ygs = []   # every step's output is kept, so no step's buffers are reused within the graph
        with torch.cuda.graph(graph):
            for _ in range(steps):
                ygs.append(flare.flare_autoregressive_triton(q, k, v))
        graph.replay()
        torch.cuda.synchronize()
        graph_ok = all(bool(torch.equal(yg, y)) for yg in ygs)
        if graph_ok:
            times = []
            for _ in range(2):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                graph.replay()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
            dt_graph = min(times)
        del graph, ygs
    except Exception as exc:   # capture unavailable: the eager loop is the measurement
        print(f"prefill graph replay unavailable: {exc}", file=sys.stderr)
    dt = dt_graph if graph_ok else dt_eager
    ms = dt * 1e3 / steps
    tok_s = B * N * steps / dt
    # Per-kernel durations: the same `steps` forwards launched back to back (the
    # library's three phase entry points, the kernels of the API call), with start /
    # end events recorded on the launch stream around each phase and no
    # synchronisation until the loop has finished.
    from causal_flare._common import EventLog
    from causal_flare.autoregressive.training import run_chunked_forward
    chunk = int(flare._lib.lib().flare_ar_default_chunk(B, N, H, M, D))
    log = EventLog()
    torch.cuda.synchronize()
    for _ in range(steps):
        run_chunked_forward(q, k, v, None, None, scale=D ** -0.5, chunk=chunk, out_dtype=v.dtype, timings=log)
    torch.cuda.synchronize()
    phases = log.mean_ms()
    flops = 6.0 * M * D * B * N * H
    dom = "flare_chunk_fwd"
    dom_ms = phases.get(dom, ms)
    achieved = flops / (dom_ms * 1e-3) / 1e12
    whole = flops / (ms * 1e-3) / 1e12
    return {
        "B": B, "N": N, "H": H, "M": M, "D": D, "ms_per_step": ms, "tok_s": tok_s,
        "timing": "graph replay of the step loop (bit-identical to eager)" if graph_ok else "eager API loop",
        "ms_per_step_eager": dt_eager * 1e3 / steps, "tok_s_eager_api_loop": B * N * steps / dt_eager,
        "phase_ms": phases, "alg_tflop_per_step": flops / 1e12,
        "roofline": {
            "bound": "mfma", "kernel": "chunk_output_tr", "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": measured_traffic("traffic_cfg3_prefill.txt", "chunk_output_tr"),
            "kernel_ms": dom_ms, "alg_flop_per_launch": flops,
            "timing": f"mean of {steps} back-to-back launches, HIP events on the launch stream",
            "whole_pass_tflops": whole, "whole_pass_frac": whole / PEAK_BF16_TFLOPS,
        },
    }


def bench_decode(torch, flare, steps=256):
    """Config 4: 64 sequences, 2048-token prefill, then `steps` decode steps with fresh k, v.

    Two loops over the same steps: the eager Python API loop (one
    flare_autoregressive_decode_triton call per step) and the same calls
    captured once in a HIP graph and replayed (back-to-back kernels, no Python
    between steps).  The state is reset from the prefill result before each
    timed run, outside the timed region.
    """
    dev = torch.device("cuda:0")
    torch.manual_seed(3)
    B, T, H, M, D = 64, 2048, 16, 128, 64
    q = (torch.randn(H, M, D) / math.sqrt(D)).to(torch.bfloat16).to(dev)
    k = torch.randn(B, T, H, D).to(torch.bfloat16).to(dev)
    v = torch.randn(B, T, H, D).to(torch.bfloat16).to(dev)
    kd = torch.randn(steps, B, H, D).to(torch.bfloat16).to(dev)
    vd = torch.randn(steps, B, H, D).to(torch.bfloat16).to(dev)
    _, base = flare.flare_autoregressive_prefill_triton(q, k, v)
    st = {kk: vv.clone() for kk, vv in base.items()}

    def reset():
        for kk in st:
            st[kk].copy_(base[kk])
        torch.cuda.synchronize()

    def eager():
        reset()
        t0 = time.perf_counter()
        for s in range(steps):
            flare.flare_autoregressive_decode_triton(q, kd[s], vd[s], state=st)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    eager()
    dt_eager = min(eager() for _ in range(3))
    eager_state = {kk: vv.clone() for kk, vv in st.items()}
    # graph capture of the same step loop
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for s in range(3):
            flare.flare_autoregressive_decode_triton(q, kd[s], vd[s], state=st)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s in range(steps):
            flare.flare_autoregressive_decode_triton(q, kd[s], vd[s], state=st)
    times = []
    for _ in range(5):
        reset()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3)
    dt_graph = min(times)
    # the replayed loop must leave the state the eager loop left, bit for bit
    replay_ok = all(bool(torch.equal(st[kk], eager_state[kk])) for kk in st)
    if not replay_ok:
        dt_graph = dt_eager
    k_ms = dt_graph * 1e3 / steps
    state_bytes = 2 * (8 * M + 4 * M * D) * B * H
    io_bytes = B * H * D * 2 * 3 + H * M * D * 2
    bytes_step = state_bytes + io_bytes
    achieved = bytes_step / (k_ms * 1e-3) / 1e9
    return {
        "B": B, "H": H, "M": M, "D": D, "prefill_T": T, "steps": steps,
        "tok_s": B * steps / dt_graph, "ms_per_step": k_ms,
        "timing": "graph replay of the step loop (final state bit-identical to eager)" if replay_ok
                  else "eager API loop (graph replay differed)",
        "tok_s_eager_api_loop": B * steps / dt_eager, "ms_per_step_eager": dt_eager * 1e3 / steps,
        "roofline": {
            "bound": "hbm", "kernel": "decode_step_fast", "achieved": achieved,
            "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
            "traffic": measured_traffic("traffic_cfg4_decode.txt", "decode_step_fast"),
            "alg_bytes_per_step": bytes_step,
            "note": "graph replay of 256 back-to-back steps; per-step time includes launch gaps",
            "basis": ("algorithmic bytes per step over the step time: the 34.6 MB fp32 state fits in the 256 MB "
                      "last-level cache between steps, and FETCH_SIZE / WRITE_SIZE cannot tell its hits from HBM, "
                      "so this is not a measured HBM rate"),
        },
        # the prefill state (before any decode step): the CPU baseline's decode starts from it
        "prefill_state": {kk: vv.cpu() for kk, vv in base.items()},
    }


def _inputs(torch, seed, B, N, H, M, D):
    torch.manual_seed(seed)
    q = (torch.randn(H, M, D) / math.sqrt(D)).to(torch.bfloat16).cuda()
    return q, torch.randn(B, N, H, D).to(torch.bfloat16).cuda(), torch.randn(B, N, H, D).to(torch.bfloat16).cuda()


def _timed(torch, fn, reps=20, warm=1):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps


def _replayed(torch, fn, reps=20):
    """`reps` calls captured once in a HIP graph and replayed back to back (as the
    prefill line): the kernels of the eager calls without the host's enqueue time.
    Every replayed output must equal the eager one bit for bit, else None."""
    first = lambda r: r[0] if isinstance(r, tuple) else r
    try:
        ref = first(fn()).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        outs = []
        with torch.cuda.graph(graph):
            for _ in range(reps):
                outs.append(first(fn()))
        graph.replay()
        torch.cuda.synchronize()
        if not all(bool(torch.equal(o, ref)) for o in outs):
            return None
        best = None
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            graph.replay()
            torch.cuda.synchronize()
            dt = (time.perf_counter() - t0) / reps
            best = dt if best is None else min(best, dt)
        del graph, outs
        return best
    except Exception as exc:   # capture unavailable: the eager loop stands
        print(f"graph replay unavailable: {exc}", file=sys.stderr)
        return None


def _hbm_roofline(B, N, H, D, dt):
    # algorithmic bytes: K and V read, Y written, bf16: 6 D bytes per token-head
    alg = 6.0 * D * B * N * H
    gbs = alg / dt / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": gbs / PEAK_HBM_GBS, "alg_bytes": alg, "scope": "whole forward (all kernels)"}


# configs 2 and 5: (seed, B, N) and the forward call
FWD_CONFIGS = {
    "config2_prefill": (1, 4, 4096, lambda flare, q, k, v: lambda: flare.flare_autoregressive_triton(q, k, v)),
    "config5_semi_ar": (4, 2, 8192, lambda flare, q, k, v: lambda: flare.flare_semi_autoregressive_trition(
        q, k, v, block_size=64, chunk_size=64)),
}


def bench_forward_config(torch, flare, name):
    """One of configs 2 / 5 (H=16, M=128, D=64, bf16): graph replay (the kernels back to
    back) where its outputs are bit-identical to the eager calls', with the eager API
    loop's host-clock time beside it."""
    seed, B, N, fn_of = FWD_CONFIGS[name]
    q, k, v = _inputs(torch, seed, B, N, 16, 128, 64)
    fn = fn_of(flare, q, k, v)
    dt_eager = _timed(torch, fn)
    dt_graph = _replayed(torch, fn)
    dt = dt_graph if dt_graph is not None else dt_eager
    return {"ms": dt * 1e3, "tok_s": B * N / dt,
            "tflops_alg": 6 * 128 * 64 * B * N * 16 / dt / 1e12,
            "roofline": _hbm_roofline(B, N, 16, 64, dt),
            "timing": "graph replay (bit-identical to eager)" if dt_graph is not None else "eager API loop",
            "ms_eager_api_loop": dt_eager * 1e3}


def bench_others(torch, flare):
    """Informational timings of configs 2 and 5 (their parity is tested, they are not the headline),
    config 3 with score jumps, and the backward of configs 2, 3 and 5."""
    inputs = lambda *a: _inputs(torch, *a)
    timed = lambda fn, reps=20, warm=1: _timed(torch, fn, reps, warm)
    replayed = lambda fn, reps=20: _replayed(torch, fn, reps)
    out = {name: bench_forward_config(torch, flare, name) for name in FWD_CONFIGS}
    out["config3_score_jump"] = bench_score_jump(torch, flare, replayed, timed)
    # the stablemax variant at the config-2 shape (forward and backward on the softmax path's kernels)
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    q, k, v = inputs(1, 4, 4096, 16, 128, 64)
    fn = lambda: flare_autoregressive_stablemax_triton(q, k, v, power=2.0)
    dt = replayed(fn)
    how = "graph replay (bit-identical to eager)"
    if dt is None:
        dt, how = timed(fn), "eager API loop"
    sm = {"forward_ms": dt * 1e3, "timing": how, "power": 2.0,
          "vs_softmax_forward": dt * 1e3 / out["config2_prefill"]["ms"]}
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    y = flare_autoregressive_stablemax_triton(q, k, v, power=2.0)
    dy = torch.randn_like(y)
    sm["backward_ms"] = timed(lambda: y.backward(dy, retain_graph=True), 5, warm=1) * 1e3
    out["config2_stablemax"] = sm
    del q, k, v, y, dy
    # backward (autograd through flare_autoregressive_triton) on configs 2 and 3
    for name, shape, reps in (("config2_backward", (4, 4096, 16, 128, 64), 5),
                              ("config3_backward", (1, 65536, 16, 256, 128), 3)):
        q, k, v = (t.requires_grad_(True) for t in inputs(7, *shape))
        y = flare.flare_autoregressive_triton(q, k, v)
        dy = torch.randn_like(y)
        dt = timed(lambda: y.backward(dy, retain_graph=True), reps, warm=2)
        B, N = shape[0], shape[1]
        out[name] = {"ms": dt * 1e3, "tok_s": B * N / dt}
        del q, k, v, y, dy
    q, k, v = (t.requires_grad_(True) for t in inputs(4, 2, 8192, 16, 128, 64))
    y, _ = flare.flare_semi_autoregressive_trition(q, k, v, block_size=64, chunk_size=64)
    dy = torch.randn_like(y)
    dt = timed(lambda: y.backward(dy, retain_graph=True), 5, warm=2)
    out["config5_semi_ar_backward"] = {"ms": dt * 1e3, "tok_s": 2 * 8192 / dt}
    return out


def _jump_keys(torch, q, k, tokens, lat, nats, scale):
    """Key outliers (as the GPU parity tests build them): at tokens[i] the key of every
    head points along the sum of the latent directions `lat`, scaled so that the
    smallest of those latents' scores is nats[i] -- a reference jump far past the fp32
    range within one 32-token subtile."""
    qf = q.float()
    for h in range(q.shape[0]):
        u = sum(qf[h, m] / qf[h, m].norm() for m in lat)
        s = torch.stack([qf[h, m] @ u for m in lat]).min() * scale
        for t, n in zip(tokens, nats):
            k[:, t, h] = (u * (n / float(s))).to(k.dtype)
    return k


def bench_score_jump(torch, flare, replayed, timed):
    """Config 3 with score jumps: one outlier key in one chunk, and one in every chunk
    (rising, so each one jumps).  The output kernel flags the jumping subtile and the
    tokenwise fp32 kernel replays that subtile only; the cost is the clean forward's
    plus the replay."""
    dev = torch.device("cuda:0")
    (B, N, H, M, D), q, k, v = _cfg3_inputs(torch, dev)
    chunk = int(flare._lib.lib().flare_ar_default_chunk(B, N, H, M, D))
    lat = list(range(0, M, M // 8))
    res = {"chunk": chunk}
    cases = (("clean", [], []),
             ("one_chunk", [5 * chunk + 1000 + 17], [150.0]),
             ("every_chunk", [c * chunk + 1000 + 17 for c in range(N // chunk)],
              [150.0 * (c + 1) for c in range(N // chunk)]))
    for name, toks, nats in cases:
        kj = _jump_keys(torch, q, k.clone(), toks, lat, nats, D ** -0.5) if toks else k
        fn = lambda: flare.flare_autoregressive_triton(q, kj, v)
        dt = replayed(fn)
        how = "graph replay (bit-identical to eager)"
        if dt is None:
            dt, how = timed(fn), "eager API loop"
        res[name] = {"ms": dt * 1e3, "outliers": len(toks), "timing": how}
    for name in ("one_chunk", "every_chunk"):
        res[name]["vs_clean"] = res[name]["ms"] / res["clean"]["ms"]
    return res


def measured_traffic(fname, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprof PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", fname)
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0] == kernel + ":":
            return float(parts[1])
    return None


def _cpu_threads():
    """Threads for the CPU baseline: the process's OpenMP share (OMP_NUM_THREADS, which
    the GPU boxes set to the CPU share of one GPU), else every core it may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env), "OMP_NUM_THREADS"
    try:
        return len(os.sched_getaffinity(0)), "sched_getaffinity"
    except AttributeError:
        return os.cpu_count() or 1, "os.cpu_count"


def cpu_baseline(decode_state=None):
    """The fp32 C oracle on bounded samples of config 3 (prefill) and config 4 (decode)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import flare_oracle as O
    cores, how = _cpu_threads()
    B, N, H, M, D = 1, int(os.environ.get("FLARE_BENCH_CPU_TOKENS", "65536")), 16, 256, 128
    rng = np.random.default_rng(2)
    q = (rng.standard_normal((H, M, D)) / math.sqrt(D)).astype(np.float32)
    k = rng.standard_normal((B, N, H, D)).astype(np.float32)
    v = rng.standard_normal((B, N, H, D)).astype(np.float32)
    t0 = time.perf_counter()
    O.ar_chunked(q, k, v, nthreads=cores)
    dt = time.perf_counter() - t0
    out = {"value": B * N / dt, "unit": "tok/s", "cores": cores, "kind": "port",
           "host_cores": os.cpu_count(), "threads_from": how,
           "sample": f"config 3 (B=1, N={N}, H=16, M=256, D=128) in fp32 through the C oracle "
                     f"(chunked 3-phase restatement of reference.py:203-512), one pass, {dt:.1f}s wall"}
    # config 4 decode: 256 single-token steps of the oracle's recurrent step (the
    # restatement of flare_decode_pytorch, inference.py:318-351) from the 2048-token
    # prefill state, one call per step as a caller drives decode
    Bd, Hd, Md, Dd, steps = 64, 16, 128, 64, int(os.environ.get("FLARE_BENCH_CPU_DECODE_STEPS", "256"))
    rng = np.random.default_rng(3)
    qd = (rng.standard_normal((Hd, Md, Dd)) / math.sqrt(Dd)).astype(np.float32)
    if decode_state is not None:
        st = {kk: vv.numpy().astype(np.float32) for kk, vv in decode_state.items()}
    else:
        st = {"m": np.zeros((Bd, Hd, Md), np.float32), "d": np.ones((Bd, Hd, Md), np.float32),
              "u": rng.standard_normal((Bd, Hd, Md, Dd)).astype(np.float32)}
    kd = rng.standard_normal((Bd, steps, Hd, Dd)).astype(np.float32)
    vd = rng.standard_normal((Bd, steps, Hd, Dd)).astype(np.float32)
    t0 = time.perf_counter()
    for s in range(steps):
        _, st = O.ar_recurrent(qd, kd[:, s:s + 1], vd[:, s:s + 1], state=st, nthreads=cores)
    dtd = time.perf_counter() - t0
    out["decode"] = {"value": Bd * steps / dtd, "unit": "tok/s", "cores": cores, "kind": "port",
                     "sample": f"config 4 decode: {steps} steps x B=64 (H=16, M=128, D=64) in fp32, one oracle "
                               f"call per step from the GPU prefill's state, {dtd:.1f}s wall"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--only", choices=("prefill", "decode", "config2", "config5", "jump"), default=None,
                    help="run one workload alone (profiler passes); the JSON line then holds that part only")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="finish with a plain 1 GiB device-to-device copy (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the causal FLARE hot path here is a single-GPU kernel "
              "set (multi-GPU sharding is design-only); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import causal_flare as flare

    if args.only is not None:
        if args.only == "prefill":
            part = bench_prefill(torch, flare, args.steps, args.warmup)
        elif args.only == "decode":
            part = bench_decode(torch, flare)
        elif args.only == "jump":
            part = bench_score_jump(torch, flare, lambda fn, reps=20: _replayed(torch, fn, reps),
                                    lambda fn: _timed(torch, fn))
        else:
            part = bench_forward_config(torch, flare, {"config2": "config2_prefill", "config5": "config5_semi_ar"}[args.only])
        part.pop("prefill_state", None)
        print(json.dumps({"only": args.only, **part}))
        if args.calibration_copy:
            calibration_copy(torch)
        return
    pre = bench_prefill(torch, flare, args.steps, args.warmup)
    dec = None if args.no_decode else bench_decode(torch, flare)
    others = None if args.no_decode else bench_others(torch, flare)
    dstate = dec.pop("prefill_state", None) if dec else None
    cpu = None if args.no_cpu else cpu_baseline(dstate)
    out = {
        "metric": "prefill tok/s (N=64k) & decode tok/s (B=64) on 1 MI355X; % of roofline",
        "value": pre["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs of the config-3 shape, generated on host, resident in HBM)",
        "config": {"workload": "config 3: long-context prefill B=1 N=65536 H=16 M=256 D=128 bf16",
                   "global_batch": pre["B"], "seq_len": pre["N"], "heads": pre["H"], "latents": pre["M"],
                   "head_dim": pre["D"], "parallelism": "single GPU"},
        "roofline": pre["roofline"],
        "phase_ms": pre["phase_ms"],
        "prefill_timing": pre["timing"],
        "prefill_eager": {"ms_per_step": pre["ms_per_step_eager"], "tok_s": pre["tok_s_eager_api_loop"]},
        "decode": dec,
        "other_configs": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    if args.calibration_copy:
        calibration_copy(torch)


def calibration_copy(torch):
    """A plain 1 GiB device-to-device copy: the known-size kernel that scales the HBM byte counters."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()


if __name__ == "__main__":
    main()
