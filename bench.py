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


def _time_kernel(fn, iters=20, warmup=2, reps=3):
    """Milliseconds per launch of fn(): `iters` launches captured in one HIP graph,
    the graph replayed `reps` times between HIP events (median), so host launch
    overhead is not part of the figure."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for _ in range(iters):
                fn()
    cur.wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) / iters)
    times.sort()
    return times[len(times) // 2]


def kernel_table():
    """Per-config kernel timings: config-1 scan, config-2 GEMM and GEMV (weights
    rotated over 512 copies so the GEMV reads HBM, not the 256 MB MALL), the
    config-3 decode GEMVs, config-4 chunked scan."""
    import numpy as np
    import torch
    from mamba_int import ops, pack_ternary
    dev = "cuda:0"
    rng = np.random.default_rng(1)
    out = {}

    def t8(*shape):
        return torch.from_numpy(rng.integers(-127, 128, size=shape, dtype=np.int8)).to(dev)

    # config 1: B1 L256 D512 N16
    x, b, c = t8(1, 256, 512), t8(1, 256, 16), t8(1, 256, 16)
    n = torch.from_numpy(rng.integers(16384, 32768, size=(512, 16), dtype=np.int32)).to(dev)
    ms = _time_kernel(lambda: ops.dyadic_scan(x, b, c, n, 15))
    byt = 696320
    out["config1_scan"] = {"ms": ms, "GB_s": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                           "G_updates_s": 256 * 512 * 16 / ms / 1e6}
    # config 2: GEMM M4096 K768 N3072 -> int8, and GEMV M1
    M, K, N = 4096, 768, 3072
    a = t8(M, K)
    wp = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(N, K), dtype=np.int8))).to(dev)
    o8 = torch.empty((M, N), dtype=torch.int8, device=dev)
    ms = _time_kernel(lambda: ops.bitlinear(a, wp, ops.OUT_INT8, N, shift=5, out=o8, path="gemm"))
    tops = 2 * M * N * K / ms / 1e9
    out["config2_gemm"] = {"ms": ms, "TOPS": tops, "mfma_frac": tops / 5000.0,
                           "GB_s": 16318464 / ms / 1e6}
    copies = 512
    wrot = wp.repeat(copies, 1).view(copies, N, K // 4)
    a1 = a[:1].contiguous()
    o1 = torch.empty((1, N), dtype=torch.int8, device=dev)
    idx = {"i": 0}

    def gemv():
        ops.bitlinear(a1, wrot[idx["i"] % copies], ops.OUT_INT8, N, shift=5, out=o1, path="gemv")
        idx["i"] += 1
    ms = _time_kernel(gemv, iters=copies)
    byt = 593664
    out["config2_gemv_m1"] = {"ms": ms, "GB_s": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                              "note": "weights rotated over 512 copies (302 MB > MALL)"}
    # config-3 decode GEMVs at batch 8
    for name, (NN, KK) in {"in_proj": (3072, 768), "out_proj": (768, 1536), "lm_head": (32000, 768)}.items():
        w = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(NN, KK), dtype=np.int8))).to(dev)
        a8 = t8(8, KK)
        o = torch.empty((8, NN), dtype=torch.int32, device=dev)
        ms = _time_kernel(lambda: ops.bitlinear(a8, w, ops.OUT_INT32, NN, out=o, path="gemv"))
        byt = NN * KK // 4 + 8 * KK + 8 * NN * 4
        out[f"config3_decode_{name}_gemv"] = {"ms": ms, "GB_s": byt / ms / 1e6, "bytes": byt}
    # config 4: B4 L8192 H24 P64 N128, chunk 256
    B, L, H, P, NS = 4, 8192, 24, 64, 128
    x4, b4, c4 = t8(B, L, H, P), t8(B, L, H, NS), t8(B, L, H, NS)
    n4 = torch.from_numpy(rng.integers(24576, 32768, size=(H,), dtype=np.int32)).to(dev)
    ms = _time_kernel(lambda: ops.ssd_chunked_scan(x4, b4, c4, n4, 15, 256), iters=3, warmup=1)
    byt = 452984928
    upd = B * L * H * P * NS
    out["config4_ssd"] = {"ms": ms, "GB_s": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                          "G_updates_s": upd / ms / 1e6}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--kernels", action="store_true", help="also time each config's kernel")
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
    if args.kernels:
        line["kernels"] = kernel_table()
    if not args.no_cpu:
        threads = len(os.sched_getaffinity(0))
        line["cpu_baseline"] = cpu_baseline(params, threads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
