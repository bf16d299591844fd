"""FWLoss forward+backward throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2] [--no-cpu-baseline]

A step is one fused forward+backward (``fw_forward_backward``: H, losses, mean, kappa and the dense
gradient) over one batch of synthetic logits resident in HBM.  The default workload is the headline
configuration N=65536, C=1000 fp32 (logits N(0,1), labels uniform).  Input/output buffer sets are
rotated between steps so the 256 MB Infinity Cache cannot hold a step's data from the previous use.

Prints one JSON line.  ``roofline.achieved`` = algorithmic bytes per launch (read logits once,
write the gradient once, read labels, write H/loss/kappa: 8*N*C + 20*N bytes) / the mean duration
of the op's row kernels, measured with one HIP event pair on their stream around K more launches of
the same op through the C ABI without the mean (whose one-block finishing kernel, about 2-5 us, the
timed steps add after the row kernels; region GPU time / K).  ``kernel_ms`` is the same for the
timed steps themselves.  ``roofline.traffic`` is the
HBM bytes per launch measured with rocprofv3 counters (profiles/<kernel>_<config>.md), or null.
``cpu_baseline`` times the reference's own CPU path (compiled into oracle/_ref) on this host's cores,
on the same host-generated inputs, as loss + full gradient per call (benchmarks/cpu_benchmarks/
bench_cpu_e2e.py:13-15); without oracle/_ref the C restatement is timed instead.
"""
import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "fast-familywise-loss_amd")
ORACLE = os.path.join(ROOT, "oracle")
for _p in (PKG, ORACLE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

DTYPE_NAME = {"f32": "fp32", "bf16": "bf16", "f16": "fp16", "f64": "fp64"}


def metric_for(N, C, dtype, dist=None):
    """The metric of the workload actually run: BASELINE.json's metric string for the headline, the
    same wording with this run's shape, dtype and input distribution otherwise."""
    m = f"rows/sec and achieved HBM GB/s (% of peak), fwd+bwd, N={N} C={C} {DTYPE_NAME[dtype]}"
    return m if dist is None else f"{m}, {dist}"
HBM_PEAK_GBS = 8000.0


ELEM_BYTES = {"f32": 4, "bf16": 2, "f16": 2, "f64": 8}


def alg_bytes(N, C, elem=4):
    # logits read once + gradient written once (the logits' element type) + int64 labels + H, loss
    # (f32) and kappa (i32)
    return 2 * elem * N * C + 8 * N + 12 * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2", choices=["cfg2", "cfg3", "cfg4", "cfg5"])
    ap.add_argument("--dist", default=None, choices=["gauss", "laplace", "mixture"],
                    help="logits from the reference harness's distributions (data_io.py:8-83) at the "
                         "configuration's shape instead of the configuration's own recipe")
    ap.add_argument("--sigma", type=float, default=1.0, help="--dist: the distributions' sigma")
    ap.add_argument("--rows", type=int, default=None,
                    help="rows of the batch (default: the configuration's N; few rows of a long "
                         "configuration run the split-row kernels)")
    ap.add_argument("--sets", type=int, default=3, help="rotated input/output buffer sets")
    ap.add_argument("--dtype", default="f32", choices=["f32", "bf16", "f16", "f64"],
                    help="element type of the logits and the gradient (decisions are fp32/fp64)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-two-op", action="store_true",
                    help="skip the timing of the reference harness's two-op sequence (profiling runs)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--copy-probe", action="store_true",
                    help="time a plain 1 GiB device copy instead (calibrates rocprof byte counters)")
    ap.add_argument("--op", default="loss", choices=["loss", "linear"],
                    help="loss: the FW loss on resident logits (the headline); linear: the LM head fused "
                         "with the loss (familywise_linear_loss) against the unfused F.linear + loss")
    ap.add_argument("--lm", default="8192,4096,128256,8192",
                    help="--op linear: tokens N, hidden size d, vocabulary V, chunk columns")
    return ap.parse_args()


def profile_for(kernel_tag, cfg):
    """(HBM bytes per launch, average kernel duration in ns) of the fused kernel from the rocprofv3
    summary committed under profiles/ (FETCH_SIZE and WRITE_SIZE passes, each scaled by what the
    counter reads for a plain copy; the kernel-trace average), or None where not profiled."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_{cfg}.md")
    if not os.path.isfile(path):
        return None, None
    with open(path) as f:
        text = f.read()
    m = re.search(r"^hbm_bytes_per_launch: (\d+)$", text, re.M)
    d = re.search(r"^avg_duration_ns: (\d+)$", text, re.M)
    return (int(m.group(1)) if m else None), (int(d.group(1)) if d else None)


def _median_time(call, seconds, min_calls):
    call()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_calls or (time.perf_counter() < t_end and len(times) < 5000):
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def cpu_baseline(z_np, y_np, seconds):
    """Time the reference CPU path (oracle/_ref) or the C restatement on the same inputs, on all
    of torch's threads and then on one thread (a shorter sample)."""
    import numpy as np
    import torch
    import oracle
    N, C = z_np.shape
    # every CPU of the process's affinity mask, within the CPU share the host grants this job
    # (OMP_NUM_THREADS, where the host sets it); both counts are reported
    affinity = len(os.sched_getaffinity(0))
    threads = affinity
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    ref = oracle.load_ref()
    nthreads = [threads]
    if ref is not None:
        Z = torch.from_numpy(z_np)
        Y = torch.from_numpy(y_np)

        def call():
            Zg = Z.detach().requires_grad_(True)
            loss = ref.familywise_loss(Zg, Y, 0)          # reduction "sum" (fwcpp.py:17)
            loss.backward()
            return Zg.grad
        kind, label = "reference", f"oracle/_ref {oracle.ref_variant()} (src/cpu/fw_cpu.cpp)"
    else:
        def call():
            return oracle.single_pass(z_np, y_np, scale=1.0, nthreads=nthreads[0])
        kind, label = "port", "oracle/fwl_oracle.c fwo_single_pass"
    med, times = _median_time(call, seconds, 10)
    # one thread: the reference splits rows with at::parallel_for, which follows torch's thread count
    torch.set_num_threads(1)
    nthreads[0] = 1
    try:
        med1, times1 = _median_time(call, seconds / 3, 3)
    finally:
        torch.set_num_threads(prev_threads)
    return {"value": N / med, "unit": "rows/s", "cores": threads, "affinity_cpus": affinity, "kind": kind,
            "sample": f"{label}: full {N}x{C} batch, loss + dense gradient per call, median of {len(times)} "
                      f"calls ({sum(times):.1f} s of CPU work), {threads} threads",
            "ms_per_call": med * 1e3, "gbps": alg_bytes(N, C) / med / 1e9,
            "one_thread": {"value": N / med1, "unit": "rows/s", "ms_per_call": med1 * 1e3,
                           "sample": f"median of {len(times1)} calls ({sum(times1):.1f} s), 1 thread"}}


def copy_probe(args):
    import torch
    n = 1 << 28  # 1 GiB of fp32
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        b.copy_(a)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    print(json.dumps({"probe": "copy", "bytes_per_launch_read": 4 * n, "bytes_per_launch_write": 4 * n,
                      "ms": dt * 1e3, "gbps": 8 * n / dt / 1e9}), flush=True)


MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}


def bench_linear(args):
    """One step = forward + backward (gradients of hidden and weight) of the FW loss of
    hidden @ weight.T, mean reduction.  The fused op computes the logits one vocabulary chunk at a
    time and derives both gradients from the sparse logit gradient; the unfused reference
    materialises the logits and back-propagates through two more GEMMs."""
    import numpy as np
    import torch
    import torch.nn.functional as F
    import fwloss
    N, d, V, chunk = (int(x) for x in args.lm.split(","))
    dname = args.dtype if any(a.startswith("--dtype") for a in sys.argv) else "bf16"   # LM heads run in bf16
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dname]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(N, d, device=dev, generator=g).to(dt).requires_grad_(True)
    w = (torch.randn(V, d, device=dev, generator=g) * (3.0 / d ** 0.5)).to(dt).requires_grad_(True)
    y = torch.randint(0, V, (N,), device=dev, generator=g)

    def fused():
        h.grad = None
        w.grad = None
        fwloss.familywise_linear_loss(h, w, y, "mean", chunk).backward()

    def unfused():
        h.grad = None
        w.grad = None
        fwloss.familywise_loss(F.linear(h, w), y, "mean").backward()

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, e0.elapsed_time(e1) / steps
    steps = min(args.steps, 20)
    warm = min(args.warmup, 3)
    wall_f, gpu_f = timed(fused, steps, warm)
    res = fwloss.linear_forward(h, w, y, chunk)
    n_over = int(res["overflow"].sum().item())
    wall_u, gpu_u = (None, None)
    if not args.no_two_op:
        wall_u, gpu_u = timed(unfused, max(1, steps // 2), 1)
    flops = 2.0 * N * V * d   # the logits GEMM: the only dense contraction of the fused step
    tf = flops / (gpu_f * 1e-3) / 1e12
    print(json.dumps({
        "metric": "tokens/s, FW loss of an LM head (hidden @ weight.T), fwd+bwd, fused vocabulary chunks",
        "value": N / wall_f, "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": wall_f * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dname, "data": "synthetic",
        "config": {"workload": f"LM head N={N} d={d} V={V} chunk={chunk} {dname}, labels uniform, mean reduction",
                   "N": N, "d": d, "V": V, "chunk": chunk, "op": "familywise_linear_loss",
                   "parallelism": "single GPU"},
        "gpu_ms_per_step": gpu_f, "overflow_rows": n_over,
        "unfused_ms_per_step": None if gpu_u is None else gpu_u,
        "speedup_vs_unfused": None if gpu_u is None else gpu_u / gpu_f,
        "roofline": {"bound": "mfma", "kernel": "whole step (logits GEMM per chunk + list merge + sparse grads)",
                     "achieved": tf, "peak": MFMA_PEAK_TFLOPS[dname], "unit": "TFLOP/s",
                     "frac": tf / MFMA_PEAK_TFLOPS[dname], "traffic": None, "flops": flops},
    }), flush=True)


def row_kernels_ms(sets, N, C, tdt, steps, stream):
    """Mean GPU time of the fused op's row kernels alone: K launches through the C ABI
    (fwl_forward_backward_ex) on the same rotated inputs with no mean requested, so that the op
    launches no finishing kernel; one HIP event pair around them on `stream`.  None for float64
    (another entry point)."""
    import torch
    import fwloss_capi as capi
    if tdt not in capi.DTYPES:
        return None
    dev = sets[0][0].device
    ws = capi.Workspace(dev)
    buf = ws.get(N, C)
    outs = [dict(H=torch.empty(N, device=dev), loss=torch.empty(N, device=dev),
                 kappa=torch.empty(N, dtype=torch.int32, device=dev),
                 grad=torch.empty((N, C), dtype=tdt, device=dev)) for _ in sets]
    P = capi._ptr
    s = capi.ctypes.c_void_p(stream.cuda_stream)

    def launch(i):
        zt, yt = sets[i % len(sets)]
        o = outs[i % len(sets)]
        rc = capi.lib().fwl_forward_backward_ex(capi.DTYPES[tdt], P(zt), C, P(yt), N, C, 1.0 / N, float(N), P(o["H"]),
                                                P(o["loss"]), None, None, P(o["kappa"]), P(o["grad"]), P(buf),
                                                buf.numel(), None, s)
        if rc != 0:
            raise RuntimeError(f"fwl_forward_backward_ex returned {rc}")
    for i in range(min(steps, 20)):
        launch(i)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(steps):
        launch(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def main():
    args = parse()
    if args.op == "linear":
        if args.gpus != 1:
            print("bench.py: this build runs on one GPU only", file=sys.stderr)
            sys.exit(2)
        bench_linear(args)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the row-sharded multi-GPU design is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import fwloss
    import fwloss_data

    if args.copy_probe:
        copy_probe(args)
        return

    dev = torch.device("cuda:0")
    if args.dist is None:
        z_np, y_np = fwloss_data.make(args.config, N=args.rows, seed=0)
        recipe = f"{args.config} recipe (fwloss_data.make)"
    else:
        shape = fwloss_data.CONFIGS[args.config]
        z_np, y_np = fwloss_data.make_dist(args.dist, args.rows or shape["N"], shape["C"], args.sigma, seed=0)
        recipe = f"{args.dist} sigma={args.sigma:g} (fwloss_data.make_dist, data_io.py:8-83)"
    N, C = z_np.shape
    cfg_tag = args.config if args.rows is None else f"{args.config}_{N}rows"
    if args.dist is not None:
        cfg_tag += f"_{args.dist}{args.sigma:g}"
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16, "f64": torch.float64}[args.dtype]
    sets = []
    for s in range(args.sets):
        zt = torch.from_numpy(z_np).to(dev).to(tdt) if s == 0 else sets[0][0].roll(s, dims=0).contiguous()
        yt = torch.from_numpy(y_np).to(dev) if s == 0 else sets[0][1].roll(s, dims=0).contiguous()
        sets.append((zt, yt))
    torch.cuda.synchronize()

    def step(i):
        zt, yt = sets[i % len(sets)]
        return fwloss.fw_forward_backward(zt, yt)

    for i in range(args.warmup):
        out = step(i)
    del out
    torch.cuda.synchronize()
    # One HIP event pair on the launch stream brackets the K launches: their mean duration is the
    # GPU time of the region / K, gaps between launches included.  (An event pair around every
    # launch adds about 7 us per step at cfg2 on MI355X: the event markers serialise the queue.)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    keep = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        o = step(i)
        keep.append(o[1])  # hold the losses so the allocator cannot reuse them within the region
        del o
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = ev0.elapsed_time(ev1) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    nbytes = alg_bytes(N, C, ELEM_BYTES[args.dtype])
    row_ms = row_kernels_ms(sets, N, C, tdt, args.steps, stream)
    achieved = nbytes / ((kern_ms if row_ms is None else row_ms) * 1e-3) / 1e9

    # the reference harness's two-op sequence (fp32 only), for comparison: the small ops below
    # K = 10000, the candidate-list ops above (benchmarks/cuda_benchmarks/CE_FW_perf.py:76-88)
    def two_op(i):
        zt, yt = sets[i % len(sets)]
        if C < 10000:
            H, losses, mean, kappa, sel = fwloss.fw_forward_small(zt, yt)
            return fwloss.fw_backward_small(yt, sel, kappa)
        H, losses, mean, kappa, cb, ci, cc = fwloss.fw_forward(zt, yt)
        return fwloss.fw_backward(zt, yt, H, kappa, cb, ci, cc)
    two_op_ms = None
    if args.dtype == "f32" and not args.no_two_op:
        for i in range(5):
            two_op(i)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for i in range(args.steps):
            two_op(i)
        torch.cuda.synchronize()
        two_op_ms = (time.perf_counter() - t1) * 1e3 / args.steps

    # the (dominant) kernel the automatic dispatch runs for this shape (16-byte aligned rows)
    unit = 16 // ELEM_BYTES[args.dtype]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if args.dtype == "f64":
        tag = "fwl_rows_f64"
    elif N <= 128 and C * ELEM_BYTES[args.dtype] >= 96 * 1024:
        tag = "fwl_split_chunks"
    elif (args.dtype == "f32" and ((N >= 384 and C >= 32000) or (C >= 8192 and N * C >= 32 << 20))) or \
            (args.dtype != "f32" and ((N >= 512 and C >= 65536) or (N >= 8 * cus and C >= 32000) or (N >= 16 * cus and C >= 28000) or
                                      (N >= 8 * cus and C >= 12000 and C % 2 == 1))):
        tag = "fwl_two_pass"      # the candidate-list read pass + fwl_fill_zero + fwl_scatter_support
    elif (C % unit == 0 and C // unit <= 64) or (C % unit != 0 and C <= 128):
        tag = "fwl_seg_rows"
    elif C <= 2048:
        tag = "fwl_wave_rows"
    elif C <= 8192 or (args.dtype != "f32" and C <= (65535 if C % unit == 0 else 28672) and N >= 1024):
        tag = "fwl_wave_stream_rows"
    else:
        tag = "fwl_block_rows"
    traffic, prof_ns = profile_for(tag, cfg_tag if args.dtype == "f32" else f"{cfg_tag}_{args.dtype}")
    result = {
        "metric": metric_for(N, C, args.dtype, None if args.dist is None else recipe),
        "value": N * args.steps / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {"workload": f"{cfg_tag} fused FW loss forward+backward, N={N} C={C} {args.dtype} logits "
                               f"({recipe}), labels uniform int64, buffers rotated over "
                               f"{args.sets} sets", "N": N, "C": C, "op": "fw_forward_backward",
                   "dist": args.dist or args.config, "sigma": args.sigma if args.dist else None,
                   "parallelism": "single GPU"},
        "gbps": nbytes / (ms_per_step * 1e-3) / 1e9,
        "hbm_frac": nbytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernel_ms": kern_ms,
        "row_kernels_ms": row_ms,
        "two_op_ms_per_step": two_op_ms,
        "roofline": {"bound": "hbm", "kernel": tag, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "alg_bytes": nbytes,
                     # the same fraction from the committed kernel-trace average (profiles/)
                     "frac_profiled": None if prof_ns is None else nbytes / prof_ns / HBM_PEAK_GBS},
    }
    if not args.no_cpu_baseline and args.dtype == "f32":
        result["cpu_baseline"] = cpu_baseline(z_np, y_np, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
