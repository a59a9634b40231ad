"""Benchmark of the integer Mamba inference hot path on one MI355X.

Workload (one "step"): the d768 x 24-layer integer Mamba (d_inner 1536,
d_state 16, dt_rank 48, vocab 32000, random ternary weights) runs a batch
8 x 2048-token prefill of uniform synthetic token ids, then 256 greedy decode
steps (HIP-graph decode step).  value = (8*2048 + 8*256) tokens / step time.

Also reported: prefill and decode tok/s separately; the roofline of the
dominant kernel (the decode step's fused norm + in_proj + conv + x_proj-partial
kernel, 24 launches per decode step); the decode step against its algorithmic
bytes; the prefill block scan (timed with HIP events around each launch inside
the timed steps) against HBM and the int32 VALU rate; and the CPU oracle (C,
OpenMP on every host core) on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-kernels]
    python bench.py --pmc-probe     # only the dominant kernel + a copy of known size, for rocprofv3 --pmc
    python bench.py --gemm-probe [--gemm-shape M,K,N]   # only a prefill GEMM (20 launches; default config 2), for rocprofv3 counters
    python bench.py --scan-probe    # only the scan kernels at their benchmark shapes, for rocprofv3 counters
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mamba-integer_amd"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the decode in_proj stage kernel at batch 8, measured
# with rocprofv3 FETCH_SIZE and WRITE_SIZE (one run each) and scaled by the
# same counters on a 256 MiB device copy (FETCH x 2.000, WRITE x 1.000)
IN_PROJ_STAGE_TRAFFIC_B8 = 1456128   # 561.0 KiB x 2 + 300.0 KiB
VALU_PEAK_GOPS = 256 * 64 * 2.4  # int32 lane-ops per ns (= G ops/s / 1000): 39321.6 G/s
# VALU lane-ops the prefill block scan (the mixed 48-channel block) issues per
# state update at the bench shape, measured with rocprofv3 --pmc SQ_INSTS_VALU
# (wave64 instructions x 64 / updates; profiles/scan_kernels_valu_pmc.md)
SCAN_LANE_OPS_PER_UPDATE = 13.61
# the same for the config-4 chunked multi-head scan (B4 L8192, 24 heads x 64, N128; the mixed
# 24-channel block)
C4_LANE_OPS_PER_UPDATE = 10.21
MFMA_I8_PEAK_TOPS = 5000.0


def scan_bytes(B, L, D, N):
    """Algorithmic HBM bytes of one fused block-scan launch: per (token, channel)
    xs, dm, z in and yo out (4 B); per token B and C (2N B); base decays
    (D*N*4 B) and the final scan state (B*D*N*4 B)."""
    T = B * L
    return T * D * 4 + T * 2 * N + D * N * 4 + B * D * N * 4


def decode_step_bytes(dims, B):
    """Algorithmic HBM bytes of one decode step at batch B: every packed ternary
    matrix once (in_proj, x_proj, dt_proj, out_proj per layer, lm_head), the
    per-layer int8 conv taps, int32 conv bias and decays, gamma, the int8
    embedding rows, and the recurrent state read and written once (int32 scan
    state B*D*N, int8 conv ring B*3*D)."""
    d, D, N, R, V = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank, dims.vocab_size
    w_layer = (2 * D * d + (R + 2 * N) * D + D * R + d * D) // 4
    p_layer = D * 4 + D * 4 + D * N * 4 + d * 2
    s_layer = 2 * (B * D * N * 4 + B * 3 * D)
    return dims.n_layer * (w_layer + p_layer + s_layer) + V * d // 4 + d * 2 + B * d


def in_proj_step_bytes(dims, B):
    """Algorithmic bytes of one launch of the decode in_proj stage kernel
    (mi_norm_in_proj_conv_xpart) at batch B, as layers 1.. run it: reads packed
    in_proj and x_proj weights, the residual rows and the previous out_proj's
    row-statistics partials (d/16 per row), gamma, conv taps, bias and ring;
    writes the z half, xs, the conv ring and the x_proj partials."""
    d, D, N, R = dims.d_model, dims.d_inner, dims.d_state, dims.dt_rank
    nx = R + 2 * N
    reads = 2 * D * d // 4 + nx * D // 4 + B * d * 4 + B * (d // 16) * 16 + d * 2 + D * 4 + D * 4 + B * 3 * D
    writes = B * D + B * D + B * 3 * D + B * (D // 16) * nx * 4
    return reads + writes


def cpu_baseline(params, threads):
    """Oracle (C, OpenMP) on a bounded sample: the full batch 8 x 2048-token
    prefill and 48 of the 256 decode steps of the same model (about 10-20 s on
    16 cores), the decode time extrapolated per step."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import oracle as O
    O.set_threads(threads)
    om = O.OracleModel(params)
    ids = np.random.default_rng(3).integers(0, params.dims.vocab_size, size=(8, 2048))
    t0 = time.perf_counter()
    logits, st = om.prefill(ids)
    t1 = time.perf_counter()
    tok = np.argmax(logits, axis=-1)
    steps = 48
    for _ in range(steps):
        logits, st = om.decode_step(tok, st)
        tok = np.argmax(logits, axis=-1)
    t2 = time.perf_counter()
    t_tok_prefill = (t1 - t0) / ids.size
    t_decode_step = (t2 - t1) / steps
    t_work = 8 * 2048 * t_tok_prefill + 256 * t_decode_step
    return {
        "value": (8 * 2048 + 8 * 256) / t_work, "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": "oracle C/OpenMP: batch 8 x 2048-token prefill + 48 decode steps of the d768x24 model "
                  f"({t2 - t0:.1f} s), decode extrapolated to 256 steps",
        "prefill_tok_s": 1.0 / t_tok_prefill, "decode_tok_s": 8.0 / t_decode_step,
    }


def cpu_model_name():
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_reference_structure(threads, dims, B=8, L=2048, n_dec=256, sub_layers=2):
    """The reference's own float inference structure on PyTorch-CPU
    (oracle/reference_cpu.py: per-timestep scan loop, fp32 F.linear BitLinear,
    decoding by re-running the whole prefix) on a declared subset: the first
    `sub_layers` of the 24 layers, timed over the full batch 8 x 2048 prefill
    and over one full-recompute decode step (a forward over 2049 positions).
    Scaling: layer time x (n_layer / sub_layers) + embedding and head time;
    the 256 decode steps cost sum over prefix lengths 2049..2304 of one
    forward each, taken as linear in the length (256 x t(2049) x 2176.5/2049)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import torch
    import reference_cpu as R
    torch.set_num_threads(threads)
    m = R.RefCpuModel(dims.d_model, sub_layers, dims.vocab_size, dims.d_state, dims.dt_rank, seed=3)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, dims.vocab_size, (B, L + 1), generator=g)

    def timed(tokens):
        with torch.no_grad():
            t0 = time.perf_counter()
            x = m.emb[tokens]
            for P in m.layers:
                x = m.block(P, x)
            t1 = time.perf_counter()
            R.bitlinear(R.bitshift_norm(x, m.gamma_f), m.w_head) * m.out_scale
            t2 = time.perf_counter()
        return t1 - t0, t2 - t1
    pl, ph = timed(ids[:, :L])
    dl, dh = timed(ids)
    scale = dims.n_layer / sub_layers
    t_prefill = pl * scale + ph
    t_step = dl * scale + dh
    t_decode = n_dec * t_step * (L + 1 + (n_dec - 1) / 2) / (L + 1)
    return {
        "value": (B * L + B * n_dec) / (t_prefill + t_decode), "unit": "tok/s", "cores": threads,
        "kind": "port", "prefill_tok_s": B * L / t_prefill, "decode_tok_s": B * n_dec / t_decode,
        "sample": f"reference float structure on PyTorch-CPU (oracle/reference_cpu.py), {sub_layers} of "
                  f"{dims.n_layer} layers: batch {B} x {L} prefill ({pl + ph:.1f} s) and one full-recompute decode "
                  f"step over {L + 1} positions ({dl + dh:.1f} s); layer time scaled x{scale:g}, decode steps "
                  f"summed over prefix lengths {L + 1}..{L + n_dec} as linear in the length",
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


def _decode_ready(run, dims, B):
    """A live batch-B decode workspace and state (prefill of 16 tokens + one
    decode step), the inputs of the decode stage kernels."""
    import numpy as np
    import torch
    from mamba_int import ops
    ids = torch.from_numpy(np.random.default_rng(5).integers(0, dims.vocab_size, size=(B, 16))).to("cuda:0")
    logits, state = run.prefill(ids)
    run.decode_step(ops.argmax(logits), state)
    torch.cuda.synchronize()
    return run._workspace(B), state


def in_proj_stage_launch(run, ws, state):
    """One launch of the decode in_proj stage kernel of layer 1 on live buffers
    (row statistics as the out_proj partials, as in layers 1..n-1 of a step)."""
    from mamba_int import ops
    ly = run.layers[1]
    return lambda: ops.norm_in_proj_conv(ws.r, ly.gamma, ly.w_in, ly.s_in, ly.conv_w, ly.conv_b, state.conv[1],
                                         ws.xs, ws.xz, row_stats=ws.parts, w_x=ly.w_x, xpart=ws.xpart)


def gemm_probe(shape=(4096, 768, 3072)):
    """For rocprofv3: 20 launches of a prefill GEMM (default: config 2, M 4096,
    K 768, N 3072; int8 requant out) on the MFMA tile path."""
    import numpy as np
    import torch
    from mamba_int import ops, pack_ternary
    rng = np.random.default_rng(1)
    M, K, N = shape
    a = torch.from_numpy(rng.integers(-127, 128, size=(M, K), dtype=np.int8)).to("cuda:0")
    wp = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(N, K), dtype=np.int8))).to("cuda:0")
    o = torch.empty((M, N), dtype=torch.int8, device="cuda:0")
    for _ in range(20):
        ops.bitlinear(a, wp, ops.OUT_INT8, N, shift=5, out=o, path="gemm")
    torch.cuda.synchronize()
    print(json.dumps({"gemm_probe": "done", "launches": 20, "int8_ops_per_launch": 2 * M * N * K}))


def pmc_probe():
    """For rocprofv3 --pmc: 20 launches of the dominant kernel at the bench's
    batch, then 3 device copies of 256 MiB (bytes known: the counter scale)."""
    import torch
    from mamba_int import ModelDims, init_random_params
    from mamba_int.model import IntegerMambaRunner
    dims = ModelDims(d_model=768, n_layer=24, vocab_size=32000, d_state=16, dt_rank=48)
    run = IntegerMambaRunner(init_random_params(dims, 3), device="cuda:0")
    ws, state = _decode_ready(run, dims, 8)
    fn = in_proj_stage_launch(run, ws, state)
    for _ in range(20):
        fn()
    x = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": "done", "kernel_launches": 20, "copy_bytes": 256 << 20, "copies": 3}))


def scan_probe():
    """For rocprofv3 --pmc: the scan kernels at their benchmark shapes, each
    launched a few times: the fused prefill block scan (B8, L2048, d_inner
    1536, N16), the config-4 chunked scan (B4, L8192, 24 heads of 64, N128,
    chunk 256) and the batch-64 decode scan step of the d2048 model (d_inner
    4096, N16, x_proj from four channel-quarter partials)."""
    import numpy as np
    import torch
    from mamba_int import ops, pack_ternary
    dev = "cuda:0"
    rng = np.random.default_rng(11)

    def t8(*shape, lo=-127, hi=127):
        return torch.from_numpy(rng.integers(lo, hi + 1, size=shape, dtype=np.int8)).to(dev)
    B, L, D, N, R = 8, 2048, 1536, 16, 48
    xs, dm, xp, z = t8(B, L, D, lo=0), t8(B, L, D, lo=-20, hi=20), t8(B, L, R + 2 * N), t8(B, L, 2 * D)
    base = torch.from_numpy(rng.integers(16384, 32001, size=(D, N), dtype=np.int32)).to(dev)
    h = torch.zeros((B, D, N), dtype=torch.int32, device=dev)
    yo = torch.empty((B, L, D), dtype=torch.int8, device=dev)
    for _ in range(5):
        ops.block_scan(xs, dm, xp, R, z, D, base, 15, 14, h_out=h, out=yo)
    B4, L4, H4, P4, N4 = 4, 8192, 24, 64, 128
    x4, b4, c4 = t8(B4, L4, H4, P4), t8(B4, L4, H4, N4), t8(B4, L4, H4, N4)
    n4 = torch.from_numpy(rng.integers(24576, 32768, size=(H4,), dtype=np.int32)).to(dev)
    for _ in range(3):
        ops.ssd_chunked_scan(x4, b4, c4, n4, 15, 256)
    m, D5, R5 = 64, 4096, 128
    xpart = torch.from_numpy(rng.integers(-3000, 3000, size=(m, 4, R5 + 32), dtype=np.int32)).to(dev)
    w_dt = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(D5, R5), dtype=np.int8))).to(dev)
    xs5, z5 = t8(m, D5, lo=0), t8(m, 2 * D5)
    base5 = torch.from_numpy(rng.integers(16384, 32001, size=(D5, 16), dtype=np.int32)).to(dev)
    h5 = torch.zeros((m, D5, 16), dtype=torch.int32, device=dev)
    yo5 = torch.empty((m, D5), dtype=torch.int8, device=dev)
    for _ in range(10):
        ops.xpart_dt_scan_step(xpart, 8, R5, w_dt, 6, xs5, z5, D5, base5, 15, 14, h5, yo5)
    torch.cuda.synchronize()
    print(json.dumps({"scan_probe": "done", "block_scan_launches": 5, "block_scan_updates": B * L * D * N,
                      "chunked_scan_launches": 3, "chunked_scan_updates": B4 * L4 * H4 * P4 * N4,
                      "decode_scan_step_launches": 10, "decode_scan_step_updates": m * D5 * 16}))


def decode5_probe():
    """For rocprofv3: the d2048 x 48 model (d_inner 4096, dt_rank 128) at batch
    64: a 16-token prefill, then 4 eager greedy decode steps (every layer's
    recurrent state, 805 MB in all, streams through HBM each step)."""
    import torch
    from mamba_int import ModelDims
    from mamba_int.model import IntegerMambaRunner, random_device_params
    dims = ModelDims(d_model=2048, n_layer=48, vocab_size=32000, d_state=16, dt_rank=128)
    run = IntegerMambaRunner(random_device_params(dims, 5, "cuda:0"), device="cuda:0")
    ids = torch.randint(0, 32000, (64, 16), device="cuda:0")
    logits, state = run.prefill(ids)
    run.decode_loop(logits, state, 4, use_graph=False)
    torch.cuda.synchronize()
    print(json.dumps({"decode5_probe": "done", "batch": 64, "decode_steps": 4}))


def kernel_table():
    """Per-config kernel timings: config-1 scan, config-2 GEMM and GEMV (weights
    rotated over 512 copies so the GEMV reads HBM, not the 256 MB MALL), the
    config-3 decode GEMVs, config-5 prefill and decode at batch 64, config-4
    chunked scan."""
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
                           "G_updates_s": 256 * 512 * 16 / ms / 1e6,
                           "roofline": {"bound": "latency (0.7 MB, 2.1 M updates per launch)", "achieved":
                                        byt / ms / 1e6, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                        "frac": byt / ms / 1e6 / HBM_PEAK_GBS}}
    # config 2: GEMM M4096 K768 N3072 -> int8, and GEMV M1
    M, K, N = 4096, 768, 3072
    a = t8(M, K)
    wp = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(N, K), dtype=np.int8))).to(dev)
    o8 = torch.empty((M, N), dtype=torch.int8, device=dev)
    ms = _time_kernel(lambda: ops.bitlinear(a, wp, ops.OUT_INT8, N, shift=5, out=o8, path="gemm"))
    tops = 2 * M * N * K / ms / 1e9
    out["config2_gemm"] = {"ms": ms, "TOPS": tops, "mfma_frac": tops / MFMA_I8_PEAK_TOPS,
                           "GB_s": 16318464 / ms / 1e6,
                           "roofline": {"bound": "mfma", "achieved": tops, "peak": MFMA_I8_PEAK_TOPS, "unit": "TOP/s",
                                        "frac": tops / MFMA_I8_PEAK_TOPS}}
    # the same kernel at the config-5 prefill in_proj shape (64 x 512 tokens,
    # d2048 -> 2 x 4096), where per-launch fixed costs matter least
    M5, K5, N5 = 32768, 2048, 8192
    a5 = t8(M5, K5)
    wp5 = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(N5, K5), dtype=np.int8))).to(dev)
    o5 = torch.empty((M5, N5), dtype=torch.int8, device=dev)
    ms5 = _time_kernel(lambda: ops.bitlinear(a5, wp5, ops.OUT_INT8, N5, shift=6, out=o5, path="gemm"), iters=5)
    tops5 = 2 * M5 * N5 * K5 / ms5 / 1e9
    out["config5_in_proj_gemm"] = {"ms": ms5, "TOPS": tops5, "mfma_frac": tops5 / MFMA_I8_PEAK_TOPS,
                                   "shape": "M32768 K2048 N8192 -> int8"}
    del a5, wp5, o5
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
    # the floor a single dependent launch cannot go below: the period of an
    # empty (one-element fill) kernel replayed the same way
    tiny = torch.zeros(1, device=dev)
    null_ms = _time_kernel(lambda: tiny.fill_(1.0), iters=copies)
    out["config2_gemv_m1"] = {"ms": ms, "GB_s": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                              "note": "weights rotated over 512 copies (302 MB > MALL); 0.59 MB is "
                                      f"{byt / HBM_PEAK_GBS / 1e3:.3f} us of HBM time, below the "
                                      f"{null_ms * 1e3:.2f} us period of an empty kernel: launch-latency bound",
                              "hbm_byte_time_us": byt / HBM_PEAK_GBS / 1e3,
                              "empty_kernel_period_us": null_ms * 1e3,
                              "roofline": {"bound": "hbm (latency-bound at this size)", "achieved": byt / ms / 1e6,
                                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                           "frac": byt / ms / 1e6 / HBM_PEAK_GBS}}
    # config-3 decode GEMVs at batch 8
    for name, (NN, KK) in {"in_proj": (3072, 768), "out_proj": (768, 1536), "lm_head": (32000, 768)}.items():
        w = torch.from_numpy(pack_ternary(rng.integers(-1, 2, size=(NN, KK), dtype=np.int8))).to(dev)
        a8 = t8(8, KK)
        o = torch.empty((8, NN), dtype=torch.int32, device=dev)
        ms = _time_kernel(lambda: ops.bitlinear(a8, w, ops.OUT_INT32, NN, out=o, path="gemv"))
        byt = NN * KK // 4 + 8 * KK + 8 * NN * 4
        out[f"config3_decode_{name}_gemv"] = {"ms": ms, "GB_s": byt / ms / 1e6, "bytes": byt}
    # config 5: d2048 x 48 (d_inner 4096, N 16, dt_rank 128), batch 64: 512-token
    # prefill and greedy decode steps (device-generated random weights)
    from mamba_int import ModelDims
    from mamba_int.model import IntegerMambaRunner, random_device_params
    dims5 = ModelDims(d_model=2048, n_layer=48, vocab_size=32000, d_state=16, dt_rank=128)
    run5 = IntegerMambaRunner(random_device_params(dims5, 5, dev), device=dev)
    ids5 = torch.randint(0, 32000, (64, 512), device=dev)
    lg5, st5 = run5.prefill(ids5)  # warm (workspaces, kernels)
    torch.cuda.synchronize()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    e0.record()
    lg5, st5 = run5.prefill(ids5)
    e1.record()
    nd = 32
    run5.decode_loop(lg5, st5, nd + 1)  # capture the decode graphs outside the timed steps
    torch.cuda.synchronize()
    e1b = torch.cuda.Event(enable_timing=True)
    e1b.record()
    run5.decode_loop(lg5, st5, nd + 1)
    e2.record()
    torch.cuda.synchronize()
    ms_pf, ms_dec = e0.elapsed_time(e1), e1b.elapsed_time(e2) / nd
    sb = decode_step_bytes(dims5, 64)
    out["config5_d2048x48_b64"] = {
        "prefill_ms_64x512": ms_pf, "prefill_tok_s": 64 * 512 / (ms_pf * 1e-3),
        "decode_ms_per_step": ms_dec, "decode_tok_s": 64 / (ms_dec * 1e-3),
        "decode_bytes_per_step": sb, "decode_GB_s": sb / (ms_dec * 1e-3) / 1e9,
        "decode_hbm_frac": sb / (ms_dec * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "roofline": {"bound": "hbm", "kernel": "whole decode step", "achieved": sb / (ms_dec * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": sb / (ms_dec * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "note": "device-generated random weights; decode steps include the host-side graph launch"}
    del run5, st5, lg5
    torch.cuda.empty_cache()
    # the shipped configuration (configs/config_mamba_integer_l4.json): multi-head
    # SSD blocks (24 heads of 64, d_state 64), d768 x 24, vocab 4096; batch 8 x
    # 2048 prefill, greedy decode steps, and the block scan alone
    from mamba_int import init_random_params
    dimsv = ModelDims(d_model=768, n_layer=24, vocab_size=4096, d_state=64, dt_rank=0, block="ssd", n_heads=24,
                      d_head=64)
    runv = IntegerMambaRunner(init_random_params(dimsv, 7), device=dev)
    idsv = torch.randint(0, 4096, (8, 2048), device=dev)
    lgv, stv = runv.prefill(idsv)
    torch.cuda.synchronize()
    e0.record()
    lgv, stv = runv.prefill(idsv)
    e1.record()
    runv.decode_loop(lgv, stv, nd + 1)  # capture the step graphs of the timed call's sizes
    torch.cuda.synchronize()
    e1b.record()
    runv.decode_loop(lgv, stv, nd + 1)
    e2.record()
    torch.cuda.synchronize()
    ms_pf, ms_dec = e0.elapsed_time(e1), e1b.elapsed_time(e2) / nd
    Bv, Lv, Dv, Wv = 8, 2048, dimsv.d_inner, dimsv.xp_width
    xsv, xpv, xzv = t8(Bv, Lv, Dv), t8(Bv, Lv, Wv), t8(Bv, Lv, 2 * Dv)
    tabv = runv.layers[0].decay_tab
    hv = torch.zeros((Bv, Dv, 64), dtype=torch.int32, device=dev)
    yv = torch.empty((Bv, Lv, Dv), dtype=torch.int8, device=dev)
    ms_scan = _time_kernel(lambda: ops.ssd_block_scan(xsv, xpv, xzv, Dv, tabv, 24, 64, 14, h_out=hv, out=yv),
                           iters=5, warmup=1)
    # each input read once, each output written once: xs, z half, yo; B, C, dt
    # columns of xp; the decay table; the final state
    scan_bytes = 3 * Bv * Lv * Dv + Bv * Lv * (2 * 24 * 64 + 24) + 24 * 255 * 4 + Bv * Dv * 64 * 4
    upd = Bv * Lv * Dv * 64
    out["shipped_ssd_d768x24_b8"] = {
        "prefill_ms_8x2048": ms_pf, "prefill_tok_s": 8 * 2048 / (ms_pf * 1e-3),
        "decode_ms_per_step": ms_dec, "decode_tok_s": 8 / (ms_dec * 1e-3),
        "ssd_scan_ms": ms_scan, "ssd_scan_bytes": scan_bytes, "ssd_scan_GB_s": scan_bytes / ms_scan / 1e6,
        "ssd_scan_hbm_frac": scan_bytes / ms_scan / 1e6 / HBM_PEAK_GBS, "ssd_scan_G_updates_s": upd / ms_scan / 1e6,
        "note": "random integer weights (spec section 7 initialisation); decode: chained step graphs, four kernels "
                "per layer"}
    del runv, stv, lgv
    torch.cuda.empty_cache()
    # config 4: B4 L8192 H24 P64 N128, chunk 256
    B, L, H, P, NS = 4, 8192, 24, 64, 128
    x4, b4, c4 = t8(B, L, H, P), t8(B, L, H, NS), t8(B, L, H, NS)
    n4 = torch.from_numpy(rng.integers(24576, 32768, size=(H,), dtype=np.int32)).to(dev)
    ms = _time_kernel(lambda: ops.ssd_chunked_scan(x4, b4, c4, n4, 15, 256), iters=3, warmup=1)
    byt = 452984928
    upd = B * L * H * P * NS
    out["config4_ssd"] = {"ms": ms, "GB_s": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                          "G_updates_s": upd / ms / 1e6,
                          "roofline": {"bound": "valu", "lane_ops_per_update": C4_LANE_OPS_PER_UPDATE,
                                       "achieved": C4_LANE_OPS_PER_UPDATE * upd / ms / 1e6, "peak": VALU_PEAK_GOPS,
                                       "unit": "G lane-ops/s",
                                       "frac": C4_LANE_OPS_PER_UPDATE * upd / ms / 1e6 / VALU_PEAK_GOPS}}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--kernels", action="store_true", help="(default) time each config's kernels")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-config kernel table")
    ap.add_argument("--pmc-probe", action="store_true", help="only the dominant kernel and a copy (for counters)")
    ap.add_argument("--gemm-probe", action="store_true", help="only the config-2 prefill GEMM (for counters)")
    ap.add_argument("--gemm-shape", default="4096,768,3072", help="M,K,N of --gemm-probe")
    ap.add_argument("--scan-probe", action="store_true", help="only the scan kernels at their benchmark shapes "
                    "(for counters)")
    ap.add_argument("--decode5-probe", action="store_true",
                    help="only 4 eager decode steps of the d2048 x 48 model at batch 64 (for a kernel trace)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: runs on one GPU only (the integer inference path has no multi-GPU code; "
              "each GPU would decode its own batch slice of a replicated model)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from mamba_int import ModelDims, init_random_params, _lib
    from mamba_int.model import IntegerMambaRunner

    _lib.load()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.gemm_probe:
        gemm_probe(tuple(int(v) for v in args.gemm_shape.split(",")))
        return
    if args.decode5_probe:
        decode5_probe()
        return
    if args.scan_probe:
        scan_probe()
        return
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

    # dominant kernel: the decode in_proj stage (24 launches per decode step);
    # per-launch period of back-to-back launches in a HIP graph, HIP events on
    # the launch stream (kernels inside the decode graphs cannot be bracketed
    # one by one)
    ws, dstate = _decode_ready(run, dims, B)
    dom_ms = _time_kernel(in_proj_stage_launch(run, ws, dstate), iters=100, warmup=3, reps=5)
    dom_bytes = in_proj_step_bytes(dims, B)
    dom_gbs = dom_bytes / (dom_ms * 1e-3) / 1e9
    # the x_proj partials are an intermediate the fusion itself creates (the
    # next stage sums them); without their writes the stage moves these bytes
    xpart_bytes = B * (dims.d_inner // 16) * (dims.dt_rank + 2 * dims.d_state) * 4
    dom_bytes_core = dom_bytes - xpart_bytes
    step_bytes = decode_step_bytes(dims, B)
    step_gbs = step_bytes / (ms_decode / NDEC * 1e-3) / 1e9

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
            "kernel": "decode in_proj stage: norm + in_proj GEMV + conv + squareplus + x_proj partials "
                      "(norm_gemv_kernel<1,true,false>, mi_norm_in_proj_conv_xpart), batch 8, 24 launches/step",
            "bound": "hbm", "achieved": dom_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": dom_gbs / HBM_PEAK_GBS, "traffic": IN_PROJ_STAGE_TRAFFIC_B8,
            "bytes_per_launch": dom_bytes, "avg_launch_ms": dom_ms,
            "bytes_per_launch_without_xproj_partials": dom_bytes_core,
            "frac_without_xproj_partials": dom_bytes_core / (dom_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "method": "period of 100 back-to-back launches in one HIP graph, HIP events on the launch stream",
        },
        "roofline_decode_step": {
            "bound": "hbm", "bytes_per_step": step_bytes, "achieved": step_gbs, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": step_gbs / HBM_PEAK_GBS,
        },
        "roofline_scan": {
            "kernel": "prefill fused block scan (model_scan_kernel<16,8,512,16>, the mixed 48-channel block), one launch per layer",
            "bound": "valu", "bytes_per_launch": sbytes, "avg_launch_ms": scan_avg_ms,
            "launches_timed": len(scan_ms), "hbm_GB_s": achieved, "hbm_frac": achieved / HBM_PEAK_GBS,
            "updates_per_s": updates / (scan_avg_ms * 1e-3),
            "lane_ops_per_update": SCAN_LANE_OPS_PER_UPDATE,
            "valu_frac": SCAN_LANE_OPS_PER_UPDATE * updates / (scan_avg_ms * 1e-3) / (VALU_PEAK_GOPS * 1e9),
        },
    }
    if not args.no_kernels:
        # configs 1, 2, 4, 5 and the shipped configuration, each against its roof
        line["kernels"] = kernel_table()
    if not args.no_cpu:
        threads = len(os.sched_getaffinity(0))
        base = cpu_baseline(params, threads)
        base["cpu_model"] = cpu_model_name()
        # the reference's own structure (float, per-step scan loop, full-recompute
        # decode) on the same cores, beside the integer oracle
        base["reference_structure"] = cpu_reference_structure(threads, dims)
        line["cpu_baseline"] = base
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
