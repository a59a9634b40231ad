"""Benchmark of the integer Mamba inference hot path on one MI355X.

Workload (one "step"): the d768 x 24-layer integer Mamba (d_inner 1536,
d_state 16, dt_rank 48, vocab 32000, random ternary weights) runs a batch
8 x 2048-token prefill of uniform synthetic token ids, then 256 greedy decode
steps (HIP-graph decode step).  value = (8*2048 + 8*256) tokens / step time.

Also reported: prefill and decode tok/s separately; the roofline of the
dominant kernel (the fused block scan), timed with HIP events on its launch
stream inside the timed steps; and the CPU oracle (C, OpenMP on every host
core) on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mamba-integer_amd"))

HBM_PEAK_GBS = 8000.0
VALU_PEAK_GOPS = 256 * 64 * 2.4  # int32 lane-ops per ns (= G ops/s / 1000): 39321.6 G/s


def scan_bytes(B, L, D, N):
    """Algorithmic HBM bytes of one fused block-scan launch: per (token, channel)
    xs, dm, z in and yo out (4 B); per token B and C (2N B); base decays
    (D*N*4 B) and the final scan state (B*D*N*4 B)."""
    T = B * L
    return T * D * 4 + T * 2 * N + D * N * 4 + B * D * N * 4


def cpu_baseline(params, threads):
    """Oracle (C, OpenMP) on a bounded sample: batch 8 x 32-token prefill and 4
    decode steps of the same model, extrapolated to the 8 x 2048 + 256-step
    workload by per-token prefill time and per-step decode time."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import oracle as O
    O.set_threads(threads)
    om = O.OracleModel(params)
    ids = np.random.default_rng(3).integers(0, params.dims.vocab_size, size=(8, 32))
    t0 = time.perf_counter()
    logits, st = om.prefill(ids)
    t1 = time.perf_counter()
    tok = np.argmax(logits, axis=-1)
    steps = 4
    for _ in range(steps):
        logits, st = om.decode_step(tok, st)
        tok = np.argmax(logits, axis=-1)
    t2 = time.perf_counter()
    t_tok_prefill = (t1 - t0) / ids.size
    t_decode_step = (t2 - t1) / steps
    t_work = 8 * 2048 * t_tok_prefill + 256 * t_decode_step
    return {
        "value": (8 * 2048 + 8 * 256) / t_work, "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": "oracle C/OpenMP: batch 8 x 32-token prefill + 4 decode steps of the d768x24 model "
                  f"({t2 - t0:.1f} s), extrapolated to 8x2048 prefill + 256 decode steps",
        "prefill_tok_s": 1.0 / t_tok_prefill, "decode_tok_s": 8.0 / t_decode_step,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=256)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the integer inference path has no "
              "multi-GPU code; sharding is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from mamba_int import ModelDims, init_random_params, _lib
    from mamba_int.model import IntegerMambaRunner

    _lib.load()
    dims = ModelDims(d_model=768, n_layer=24, vocab_size=32000, d_state=16, dt_rank=48)
    B, L, NDEC = 8, 2048, args.decode_steps
    params = init_random_params(dims, 3)
    dev = torch.device("cuda:0")
    run = IntegerMambaRunner(params, device="cuda:0")
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, dims.vocab_size, size=(B, L))).to(dev)

    scan_events = []
    timing = {"on": False}

    def before():
        if timing["on"]:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            scan_events.append([e, None])

    def after():
        if timing["on"]:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            scan_events[-1][1] = e

    run.scan_timer = (before, after)

    def step(ev):
        ev[0].record()
        logits, st = run.prefill(ids)
        ev[1].record()
        run.decode_loop(logits, st, NDEC + 1, use_graph=True)
        ev[2].record()

    for _ in range(args.warmup):
        step([torch.cuda.Event(enable_timing=True) for _ in range(3)])
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    timing["on"] = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
        print(f"bench: step {i + 1}/{args.steps} enqueued", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    timing["on"] = False

    wall = (t1 - t0) / args.steps
    ms_prefill = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    ms_decode = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    ms_step = wall * 1e3
    tokens = B * L + B * NDEC
    scan_ms = [a.elapsed_time(b) for a, b in scan_events if b is not None]
    scan_avg_ms = sum(scan_ms) / len(scan_ms)
    sbytes = scan_bytes(B, L, dims.d_inner, dims.d_state)
    achieved = sbytes / (scan_avg_ms * 1e-3) / 1e9
    updates = B * L * dims.d_inner * dims.d_state

    line = {
        "metric": "prefill + decode tok/s, 1 GPU, int-Mamba d768x24; scan/GEMV % HBM roofline",
        "value": tokens / wall,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8/int32",
        "data": "synthetic (uniform token ids, random ternary weights, seed 3)",
        "config": {"workload": "int-Mamba d768x24 (d_inner 1536, d_state 16, dt_rank 48, vocab 32000): "
                               f"batch {B} x {L}-token prefill + {NDEC} greedy decode steps",
                   "global_batch": B, "seq_len": L, "decode_steps": NDEC, "parallelism": "none (1 GPU)"},
        "prefill_tok_s": B * L / (ms_prefill * 1e-3),
        "decode_tok_s": B * NDEC / (ms_decode * 1e-3),
        "ms_prefill": ms_prefill,
        "ms_decode_step": ms_decode / NDEC,
        "roofline": {
            "kernel": "fused block scan (scan_kernel<16,G,model>), one launch per layer in prefill",
            "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": None,
            "bytes_per_launch": sbytes, "avg_launch_ms": scan_avg_ms, "launches_timed": len(scan_ms),
            "valu_updates_per_s": updates / (scan_avg_ms * 1e-3),
        },
    }
    if not args.no_cpu:
        threads = len(os.sched_getaffinity(0))
        line["cpu_baseline"] = cpu_baseline(params, threads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
