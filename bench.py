#!/usr/bin/env python3
"""Throughput benchmark of the KANLinear hot path on one MI355X.

Workload (the metric's config): a single
KANLinear(in=1024, out=1024, grid_size=10, spline_order=3) in fp32 on the
native gfx950 backend, N = 65536 samples, x ~ U(-1, 1) with
requires_grad=True, coef ~ N(0, 0.1), base_weight ~ U(+-1/32),
scaler ~ U(0.5, 1.5), target ~ N(0, 1); one step is
zero_grad -> forward -> MSE loss -> backward (dx, dcoef, dscaler, dbase_w),
so three dense-equivalent contractions of 2*N*O*I*(R+1) flops each.
Inputs are generated on the CPU with a seeded torch.Generator and moved to
the device before timing starts.

Prints one JSON line (the benchmark contract): whole-job samples/s, the
roofline of the dominant kernel (the MFMA contraction, timed live with HIP
events recorded by the library on the launch stream), a CPU baseline (the
ATen/MKL formulation of the reference's CPU path, csrc/kan_cpu.cpp, on the
host's cores, rank 0 only) and, under "other_configs", the same figures for
BASELINE.json's other single-GPU configs (c2, c4, c5), reported beside the
metric.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload c3|c3-nodx|c2|c4|c5|stream|refit|pinn|infer]
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd samples/s, KANLinear 1024→1024 G10 k3 N=64K; % MFMA/HBM roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_FP64_TFLOPS = 78.6  # FP64 MFMA and FP64 vector alike
PEAK_HBM_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_recorded.json")


def recorded_traffic(cfg):
    """(HBM bytes per launch of the config's dominant kernel, source) from the
    committed rocprofv3 --pmc summaries (FETCH_SIZE + WRITE_SIZE, calibrated
    on a 1 GiB copy); a recorded figure, not measured in this run."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            rec = json.load(f).get(cfg)
    except (OSError, ValueError):
        return None, None
    if not rec:
        return None, None
    return rec.get("hbm_bytes_per_launch"), ("recorded: %s (rocprofv3 --pmc FETCH_SIZE and "
                                              "WRITE_SIZE per dispatch, calibrated on a 1 GiB "
                                              "copy), not measured in this run" % rec["source"])


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3",
                    choices=["c3", "c3-nodx", "c2", "c4", "c5", "stream", "refit", "pinn",
                             "infer"],
                    help="c3 (the metric's config, default), c3-nodx (x without grad, the "
                         "reference benchmark's semantics), c2 (KAN([784,256,10])), c4 "
                         "(KAN([256,512,512,64]) with forward_with_regularization), c5 "
                         "(4096->256 G65, the kernel-limit layer), stream (HBM streaming "
                         "ceiling over a buffer of c3's augmented-basis size), refit "
                         "(update_grid of c4's 512->512 layer), pinn (Laplacian loss of "
                         "KAN([2,128,128,1]) through create_graph) or infer (c3's layer, "
                         "exported, inference forward); all but c3 are reported separately, "
                         "not the metric")
    ap.add_argument("--dtype", default="f32", choices=["f32", "f64"],
                    help="arithmetic type of c3, c3-nodx and c4 (the metric is f32; f64 lines "
                         "are reported against the FP64 peak)")
    ap.add_argument("--n", type=int, default=0, help="samples per step (default: the config's)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--native-only", action="store_true",
                    help="pinn: skip the reference formulation's run on the same GPU (for "
                         "profiling the native step alone)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="c3 only: skip the c2, c4 and c5 figures of the JSON line")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of each baseline sample (3 timed repetitions)")
    ap.add_argument("--no-graph", action="store_true",
                    help="c2: time eager steps instead of replays of the step captured in a "
                         "HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device-to-device copy (3 times); the HBM "
                         "counters of this known-size copy scale the counter readings of the "
                         "kernels")
    return ap.parse_args()


def copy_calibration():
    import torch
    n = 1 << 28  # 2^28 fp32 = 1 GiB
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "launches": 3}))


# ---------------------------------------------------------------------------
# workloads; the GPU parity tests build the same ones
# ---------------------------------------------------------------------------

def make_inputs(N, I, O, G, k, seed=0):
    """c3: seeded CPU draws in a fixed order: x, coef, base_weight, scaler, target."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(N, I, generator=g) * 2 - 1
    coef = torch.randn(O, I, G + k, generator=g) * 0.1
    bw = (torch.rand(O, I, generator=g) * 2 - 1) / (I ** 0.5)
    scaler = torch.rand(O, I, generator=g) + 0.5
    target = torch.randn(N, O, generator=g)
    return x, coef, bw, scaler, target


def build_c3(dev, N=65536, need_dx=True, dtype=None):
    """(layer on dev, x on dev with requires_grad=need_dx, target on dev,
    CPU copies of (x, coef, bw, scaler, target, grid)) for c3; dtype float64
    casts the same draws (layer, x and target) after they are made."""
    import torch
    from torchsplinekan_amd import KANLinear
    I = O = 1024
    G, k = 10, 3
    x, coef, bw, scaler, target = make_inputs(N, I, O, G, k, seed=0)
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    with torch.no_grad():
        L.spline_weight.copy_(coef)
        L.base_weight.copy_(bw)
        L.spline_scaler.copy_(scaler)
    grid_cpu = L.grid.detach().clone()
    dt = dtype or torch.float32
    L = L.to(dev, dt)
    xd = x.to(dev, dt).requires_grad_(need_dx)
    return L, xd, target.to(dev, dt), (x, coef, bw, scaler, target, grid_cpu)


def build_c2(dev, N=4096):
    """c2: KAN([784, 256, 10], G=5, k=3) fp32, uniform knots on [-1, 1];
    x ~ U(-1, 1) [N, 784]; coef ~ N(0, 0.1); base_weight Kaiming-uniform
    (the layer's default init, global seed 0); scaler = 1; target ~ N(0, 1).
    Returns (net on dev, x, target) with x and target on the CPU."""
    import torch
    from torchsplinekan_amd import KAN
    g = torch.Generator().manual_seed(2)
    x = torch.rand(N, 784, generator=g) * 2 - 1
    target = torch.randn(N, 10, generator=g)
    torch.manual_seed(0)
    net = KAN([784, 256, 10], grid_size=5, spline_order=3, backend="cuda")
    with torch.no_grad():
        for layer in net.layers:
            layer.spline_weight.normal_(0.0, 0.1, generator=g)
            layer.spline_scaler.fill_(1.0)
    return net.to(dev), x, target


def build_c4(dev, N=16384, dtype=None):
    """c4: KAN([256, 512, 512, 64], G=8, k=3) fp32; x [N, 256] from a
    4-component Gaussian mixture (means +-0.5, +-0.8, sd 0.1, equal weights);
    coef ~ N(0, 0.1); knots and coefficients then set by the network's
    update_grid on x (on the device: native Gram kernel + float64 device
    solve).  Returns (net on dev, x on dev, target on dev)."""
    import torch
    from torchsplinekan_amd import KAN
    widths = [256, 512, 512, 64]
    g = torch.Generator().manual_seed(0)
    means = torch.tensor([-0.8, -0.5, 0.5, 0.8])
    comp = torch.randint(0, 4, (N, widths[0]), generator=g)
    x = means[comp] + 0.1 * torch.randn(N, widths[0], generator=g)
    target = torch.randn(N, widths[-1], generator=g)
    torch.manual_seed(0)
    net = KAN(widths, grid_size=8, spline_order=3, backend="cuda")
    with torch.no_grad():
        for layer in net.layers:
            layer.spline_weight.normal_(0.0, 0.1, generator=g)
    dt = dtype or torch.float32
    net = net.to(dev, dt)
    xd = x.to(dev, dt)
    net.update_grid(xd)
    return net, xd, target.to(dev, dt)


def build_c5(dev, N=8192):
    """c5: KANLinear(4096 -> 256, G=65, k=3) fp32 (72 knots, R = 68) on uniform
    [-1, 1] knots; x ~ U(-1.1, 1.1) [N, 4096] (0.7 % of the inputs fall
    outside [t_0, t_71] and take the zero-basis path); coef ~ N(0, 0.05);
    base_weight and scaler from the layer's default init (global seed 0);
    target ~ N(0, 1).  Returns (layer on dev, x on the CPU, target on the CPU)."""
    import torch
    from torchsplinekan_amd import KANLinear
    g = torch.Generator().manual_seed(5)
    x = (torch.rand(N, 4096, generator=g) * 2 - 1) * 1.1
    target = torch.randn(N, 256, generator=g)
    torch.manual_seed(0)
    L = KANLinear(4096, 256, grid_size=65, spline_order=3, backend="cuda")
    with torch.no_grad():
        L.spline_weight.normal_(0.0, 0.05, generator=g)
    return L.to(dev), x, target


def contraction_flops(N, I, O, R):
    """Dense-equivalent flops of one contraction: 2 N O I (R + 1)."""
    return 2.0 * N * O * I * (R + 1)


# ---------------------------------------------------------------------------
# CPU baseline (the reference CPU path's formulation, csrc/kan_cpu.cpp)
# ---------------------------------------------------------------------------

def host_cpu():
    """lscpu-style facts of this host: model name, physical cores, logical
    CPUs, CPUs this process may run on, and the thread count the baseline
    uses (physical cores, capped by the CPU share and OMP_NUM_THREADS)."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model == "unknown":
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    core = val
                elif not key and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    logical = os.cpu_count() or 1
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = logical
    physical = len(cores) or logical
    threads = min(physical, share)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    return {"model": model, "physical_cores": physical, "logical_cpus": logical,
            "cpus_allowed": share, "threads": max(1, threads)}


def _median_reps(run_rows, total_rows, chunk, seconds):
    """Times run_rows(n0, n1) over the first rows of the workload: one
    untimed chunk, then the number of chunks that makes one repetition
    about seconds/3, three timed repetitions; -> (rows, median seconds,
    all repetition times)."""
    n1 = min(chunk, total_rows)
    t0 = time.perf_counter()
    run_rows(0, n1)
    per_chunk = time.perf_counter() - t0
    chunks = max(1, min(-(-total_rows // chunk), int(seconds / 3.0 / max(per_chunk, 1e-6))))
    rows = min(total_rows, chunks * chunk)
    reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        for a in range(0, rows, chunk):
            run_rows(a, min(a + chunk, rows))
        reps.append(time.perf_counter() - t0)
    return rows, statistics.median(reps), reps


def cpu_baseline_layers(layers, x, target, need_dx, seconds, chunk, label):
    """Forward + MSE + backward of a stack of KAN layers on the host through
    the ATen formulation of csrc/kan_cpu.cpp (the raw ops' CPU dispatch:
    dense Cox-de Boor basis, MKL GEMMs, analytic backward), on consecutive
    row chunks of the same inputs.  `layers` are (grid, bw, sw, scaler)
    float32 CPU tensors; the loss scale is the full batch's, so every chunk
    does the work it does inside the full step."""
    import torch
    from torchsplinekan_amd import _C
    info = host_cpu()
    prev = torch.get_num_threads()
    torch.set_num_threads(info["threads"])
    params = [(g, bw.clone().requires_grad_(), sw.clone().requires_grad_(),
               sc.clone().requires_grad_()) for g, bw, sw, sc in layers]
    scale = float(target.numel())

    def run_rows(n0, n1):
        h = x[n0:n1].clone().requires_grad_(need_dx)
        out = h
        for g, bw, sw, sc in params:
            out = _C.kan_apply(out, g, bw, sw, sc, 3, True)
        loss = ((out - target[n0:n1]) ** 2).sum() / scale
        loss.backward()
        for _, bw, sw, sc in params:
            bw.grad = sw.grad = sc.grad = None

    try:
        rows, med, reps = _median_reps(run_rows, x.shape[0], chunk, seconds)
    finally:
        torch.set_num_threads(prev)
    return {
        "value": rows / med, "unit": "samples/s", "cores": info["threads"], "kind": "port",
        "sample": (f"{label}: the ATen/MKL formulation of csrc/kan_cpu.cpp (raw-op CPU "
                   f"dispatch, torchsplinekan_amd/composite.py) fp32 fwd + MSE + bwd "
                   f"{'with' if need_dx else 'without'} dx on the first {rows} of "
                   f"{x.shape[0]} rows in {chunk}-row chunks; median of 3 repetitions "
                   f"({', '.join(f'{r:.2f}' for r in reps)} s)"),
        "host": info, "torch_threads": info["threads"],
    }


def cpu_baseline_c4(net_cpu, x, target, seconds, chunk=512):
    """c4 on the host through the reference backend (backend="reference" on
    CPU tensors: forward_with_regularization resolves reg_impl "auto" to the
    dense [n, O, I] edge tensor, spline_kan/kan_linear.py:398-422), on row
    chunks; the edge means are per chunk."""
    import torch
    info = host_cpu()
    prev = torch.get_num_threads()
    torch.set_num_threads(info["threads"])
    scale = float(target.numel())

    def run_rows(n0, n1):
        for p in net_cpu.parameters():
            p.grad = None
        y, reg = net_cpu.forward_with_regularization(x[n0:n1], 1e-2, 1e-2, reg_impl="auto")
        (((y - target[n0:n1]) ** 2).sum() / scale + reg).backward()

    try:
        rows, med, reps = _median_reps(run_rows, x.shape[0], chunk, seconds)
    finally:
        torch.set_num_threads(prev)
    return {
        "value": rows / med, "unit": "samples/s", "cores": info["threads"], "kind": "port",
        "sample": (f"c4 on the reference backend (torchsplinekan_amd/reference_backend.py, the "
                   f"restated spline_kan reference path) fp32 forward_with_regularization "
                   f"(reg_impl 'auto' -> dense on CPU) + MSE + backward on the first {rows} of "
                   f"{x.shape[0]} rows in {chunk}-row chunks (edge means per chunk); median of "
                   f"3 repetitions ({', '.join(f'{r:.2f}' for r in reps)} s)"),
        "host": info, "torch_threads": info["threads"],
    }


def _layer_tensors(layer):
    """(grid, base_weight, spline_weight, spline_scaler) as float32 CPU tensors."""
    f = lambda t: t.detach().float().cpu().clone()
    return f(layer.grid), f(layer.base_weight), f(layer.spline_weight), f(layer.spline_scaler)


# ---------------------------------------------------------------------------
# timed GPU steps
# ---------------------------------------------------------------------------

def timed_steps(step, steps, warmup, classes, params=(), timed=None):
    """warmup untimed steps, then `steps` timed ones between two device
    synchronisations with nothing else running (the library's per-launch
    timing off), then one more step for the memory figures and `steps`
    instrumented ones for the per-kernel times (HIP events the library
    records around each launch on its own stream).  timed: what the timed
    steps call instead of step (a graph replay of it); warmup, memory and
    the instrumented pass run step itself.
    -> (wall seconds of the timed steps, {class: (ms, launches, work)},
        memory figures)."""
    import torch
    from torchsplinekan_amd import _lib
    for _ in range(warmup):
        step()
    _lib.timing_enable(False)
    run = timed or step
    if timed is not None:
        for _ in range(warmup):
            run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    mem = measure_memory(step, params)
    _lib.timing_enable(True)
    torch.cuda.synchronize()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kern = {c: _lib.timing_read(c) for c in classes}
    _lib.timing_enable(False)
    return wall, kern, mem


def measure_memory(step, params):
    """Device memory of one step as the reference's benchmark measures it
    (benchmarks/bench_kan.py:308-329): gradients cleared, allocator peak
    reset, one step; the peak over the step, its increment over what was
    allocated before (parameters, inputs, targets), what the step leaves
    allocated, and the gradients' bytes."""
    import gc
    import torch
    for p in params:
        p.grad = None
    gc.collect()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated()
    after = torch.cuda.memory_allocated()
    grads = sum(p.grad.numel() * p.grad.element_size() for p in params if p.grad is not None)
    return {"peak_mem_bytes": peak, "baseline_bytes": base, "peak_increment_bytes": peak - base,
            "retained_after_bytes": after - base, "grad_bytes": grads,
            "method": "torch.cuda.max_memory_allocated over one step after "
                      "reset_peak_memory_stats (benchmarks/bench_kan.py:308-329); every "
                      "library workspace is a torch allocation"}


def _mfma_roofline(kern, cls, kernel_name, traffic=None, traffic_source=None,
                   peak=PEAK_FP32_MFMA_TFLOPS):
    ms, cnt, work = kern[cls]
    ach = work / (ms * 1e-3) / 1e12 if cnt else 0.0
    return {"bound": "mfma", "kernel": kernel_name, "achieved": ach,
            "peak": peak, "unit": "TFLOP/s", "frac": ach / peak,
            "traffic": traffic, "traffic_source": traffic_source,
            "flop_per_launch": work / max(cnt, 1), "avg_launch_ms": ms / max(cnt, 1),
            "launches": cnt}


def _line(metric, N, steps, warmup, wall, workload, roofline, kern, mem, **extra):
    line = {
        "metric": metric, "value": N * steps / wall, "unit": "samples/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": wall * 1e3 / steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded torch.Generator draws, random-init weights of the config)",
        "config": {"workload": workload}, "roofline": roofline,
        "kernels": {c: {"ms_per_step": v[0] / steps, "launches_per_step": v[1] / steps}
                    for c, v in kern.items()},
        "kernel_times": "from a separate instrumented pass of the same step count",
        "peak_mem_bytes": mem["peak_mem_bytes"], "memory": mem,
    }
    line.update(extra)
    return line


def run_c3(args, dev, steps, warmup, need_dx=True, f64=False):
    """c3: KANLinear(1024 -> 1024, G=10, k=3) fp32, N = 65536, fwd + MSE +
    bwd; with dx (three contractions: the metric's workload) or, as the
    reference's benchmark runs it (benchmarks/bench_kan.py:168-175), with x
    not requiring grad (two contractions).  f64: the same in float64 (the
    reference dispatches every kernel on both types), against the FP64 peak."""
    import torch
    import torch.nn.functional as F
    N = args.n or 65536
    L, xd, td, cpu_inputs = build_c3(dev, N, need_dx, torch.float64 if f64 else None)
    I, O, R = L.in_features, L.out_features, L.grid_size + L.spline_order
    torch.cuda.synchronize()

    def step():
        for p in L.parameters():
            p.grad = None
        xd.grad = None
        y = L(xd)
        loss = F.mse_loss(y, td)
        loss.backward()

    wall, kernels, mem = timed_steps(step, steps, warmup,
                                     ("contraction", "basis", "basis_grad", "other"),
                                     list(L.parameters()) + [xd])
    if L.last_backend != "cuda":
        raise RuntimeError("the timed steps did not run on the native backend")
    # per-step spans with events on the step's stream, outside the timed region
    stream = torch.cuda.current_stream(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    step_ms = [a.elapsed_time(b) for a, b in ev]

    tag = ("c3" if need_dx else "c3-nodx") + ("-f64" if f64 else "")
    traffic, source = recorded_traffic(tag)
    roof = _mfma_roofline(kernels, "contraction",
                          "%s (%s MFMA contraction; average over the forward, parameter%s "
                          "launches)" % ("gemm_pipe_kernel",
                                         "fp64" if f64 else "fp32",
                                         " and input" if need_dx else ""),
                          traffic, source, PEAK_FP64_TFLOPS if f64 else PEAK_FP32_MFMA_TFLOPS)
    b_ms, b_cnt, b_work = kernels["basis"]
    g_ms, g_cnt, g_work = kernels["basis_grad"]
    c_ms = kernels["contraction"][0]
    gbps = lambda w, ms, n: (w / n) / (ms / n * 1e-3) / 1e9 if n else None
    line = {
        "metric": (METRIC if need_dx and not f64 else
                   "fwd+bwd samples/s, KANLinear 1024->1024 G10 k3 N=64K%s%s"
                   % ("" if need_dx else ", x without grad (2 contractions)",
                      ", float64" if f64 else "")),
        "value": N * steps / wall,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": wall * 1e3 / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if f64 else "f32",
        "data": "synthetic (seeded torch.Generator draws, random-init weights of the config)",
        "config": {
            "workload": ("c3: KANLinear(1024->1024, grid_size=10, spline_order=3) %s, N=%d, "
                         "fwd + MSE + bwd %s" % ("fp64" if f64 else "fp32", N,
                                                 "with dx (3 contractions)" if need_dx
                                                 else "without dx (2 contractions; the "
                                                 "reference benchmark's fwd_bwd)")),
            "in_features": I, "out_features": O, "grid_size": L.grid_size,
            "spline_order": L.spline_order, "samples_per_step": N, "x_requires_grad": need_dx,
        },
        "roofline": roof,
        "step_ms_median_events": statistics.median(step_ms),
        "kernels": {
            "basis": {"avg_ms": b_ms / max(b_cnt, 1), "launches": b_cnt,
                      "GB/s": gbps(b_work, b_ms, b_cnt)},
            "basis_grad": {"avg_ms": g_ms / max(g_cnt, 1), "launches": g_cnt,
                           "GB/s": gbps(g_work, g_ms, g_cnt)},
            "contraction_ms_per_step": c_ms / steps,
            "other_ms_per_step": kernels["other"][0] / steps,
        },
        "kernel_times": "from a separate instrumented pass of the same step count",
        "peak_mem_bytes": mem["peak_mem_bytes"],
        "memory": mem,
    }
    if not args.no_cpu_baseline and not f64:
        x, coef, bw, scaler, target, grid = cpu_inputs
        line["cpu_baseline"] = cpu_baseline_layers([(grid, bw, coef, scaler)], x, target, need_dx,
                                                   args.cpu_seconds, 2048, "c3")
    return line


def capture_step(step):
    """The step captured once in a HIP graph (torch.cuda.CUDAGraph, warmed up
    on a side stream of default priority) -> a function that replays it.
    Every launch of the native path goes to the current stream and nothing in
    it synchronises with the host, so a replay runs the step's kernels
    without its host work (tests/test_gpu_graph.py checks replays of c2's
    step, F.mse_loss included, against eager steps bit for bit; torch's
    multi-block means over larger outputs are not replay-safe on this ROCm
    build, so a step with one stays eager)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    return graph.replay


def graph_step(args, step, steps, warmup):
    """(replay, extra fields of the JSON line): unless --no-graph, the eager
    step's time per step (warmup, then `steps` timed) and a replay of the
    step captured in a HIP graph; (None, {}) with --no-graph."""
    import torch
    if args.no_graph:
        return None, {}
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager = (time.perf_counter() - t0) * 1e3 / steps
    return capture_step(step), {"step": "HIP graph replay of the captured step",
                                "eager_ms_per_step": eager}


def run_c2(args, dev, steps, warmup):
    """c2: KAN([784, 256, 10]) G5 k3 fp32, N = 4096, fwd + MSE + bwd (x
    without grad, the network input of a classifier).  Its kernels take
    about 0.5 ms per step, close to what the host needs to issue them from
    Python, so on a slow host eager steps measure the host: the timed steps
    replay the step captured in a HIP graph (the same kernels on the same
    inputs, nothing skipped), and the eager figure is reported beside it
    (eager_ms_per_step; --no-graph times eager steps)."""
    import torch
    import torch.nn.functional as F
    N = args.n or 4096
    net, x, target = build_c2(dev, N)
    xd, td = x.to(dev), target.to(dev)

    def step():
        for p in net.parameters():
            p.grad = None
        F.mse_loss(net(xd), td).backward()

    replay, extra = graph_step(args, step, steps, warmup)
    wall, kern, mem = timed_steps(step, steps, warmup,
                                  ("contraction", "basis", "basis_grad", "other"),
                                  list(net.parameters()), timed=replay)
    if any(l.last_backend != "cuda" for l in net.layers):
        raise RuntimeError("c2 did not run on the native backend")
    line = _line("fwd+bwd samples/s, KAN([784,256,10]) G5 k3 N=4096", N, steps, warmup, wall,
                 "c2: KAN([784,256,10], G=5, k=3) fp32, N=%d, fwd + MSE + bwd (x without "
                 "grad)%s" % (N, "" if replay is None else ", replayed from a HIP graph"),
                 _mfma_roofline(kern, "contraction", "contraction: gemm_pipe_kernel (fp32 MFMA; "
                                "forward and parameter products of the first layer) and the "
                                "thin-product kernels (thin_wide_cols/thin_wide_rows/"
                                "thin_short_k: forward, parameter and input products of the "
                                "10-wide output layer)", *recorded_traffic("c2")), kern, mem,
                 **extra)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_layers(
            [_layer_tensors(l) for l in net.layers], x, target, False, args.cpu_seconds, 1024,
            "c2")
    return line


def run_c4(args, dev, steps, warmup):
    """c4: KAN([256, 512, 512, 64]) G8 k3 fp32 with update_grid knots, N =
    16384; one step is forward_with_regularization(1e-2, 1e-2, "auto") + MSE
    + backward (x without grad)."""
    import torch
    import torch.nn.functional as F
    N = args.n or 16384
    f64 = getattr(args, "dtype", "f32") == "f64"
    net, xd, td = build_c4(dev, N, torch.float64 if f64 else None)

    def step():
        for p in net.parameters():
            p.grad = None
        y, reg = net.forward_with_regularization(xd, 1e-2, 1e-2, reg_impl="auto")
        (F.mse_loss(y, td) + reg).backward()

    wall, kern, mem = timed_steps(step, steps, warmup, ("edge", "edge_grad", "basis",
                                                        "basis_grad", "contraction", "other"),
                                  list(net.parameters()))
    if any(l.last_backend != "cuda" for l in net.layers):
        raise RuntimeError("c4 did not run the fused native path")
    # dominant kernel class: the edge-statistic backward on FP32 MFMA (fused
    # kernel for the layers that need both gradient sides: phi once plus two
    # products, 6 n O I (R+1) flops; parameter kernel for the first layer,
    # whose input needs no gradient: 4 n O I (R+1))
    if f64:
        roof = _mfma_roofline(kern, "edge_grad", "edge_param_mfma64_kernel + "
                              "edge_input_mfma64_kernel (fp64 MFMA): mean|phi| backward, "
                              "4 n O I (R+1) flops per launch",
                              None, None, PEAK_FP64_TFLOPS)
    else:
        roof = _mfma_roofline(kern, "edge_grad", "edge_bwd_mfma_kernel (both gradient sides, "
                              "dL/dy folded in; edge_bwd_stage_kernel for the 64-wide layer) + "
                              "edge_param_mfma_kernel (first layer): mean|phi| backward",
                              *recorded_traffic("c4"))
    e_ms, e_cnt, e_work = kern["edge"]
    line = _line("fwd+bwd samples/s, KAN([256,512,512,64]) G8 k3 N=16K forward_with_regularization"
                 + (", float64" if f64 else ""), N, steps, warmup, wall,
                 "c4: KAN([256,512,512,64], G=8, k=3) %s, N=%d, update_grid knots, "
                 "forward_with_regularization(1e-2, 1e-2, 'auto') + MSE + backward"
                 % ("fp64" if f64 else "fp32", N), roof,
                 kern, mem, edge_forward_tflops=e_work / (e_ms * 1e-3) / 1e12 if e_cnt else 0.0)
    if f64:
        line["dtype"] = "f64"
    if not args.no_cpu_baseline and not f64:
        from torchsplinekan_amd import KAN
        net_cpu = KAN([256, 512, 512, 64], grid_size=8, spline_order=3, backend="reference")
        net_cpu.load_state_dict({k_: v.detach().cpu() for k_, v in net.state_dict().items()})
        line["cpu_baseline"] = cpu_baseline_c4(net_cpu, xd.cpu(), td.cpu(), args.cpu_seconds)
    return line


def run_c5(args, dev, steps, warmup):
    """c5: KANLinear(4096 -> 256, G=65, k=3) fp32, N = 8192, fwd + MSE + bwd
    with dx (three contractions of K = 4096 x 69 = 282624)."""
    import torch
    import torch.nn.functional as F
    N = args.n or 8192
    L, x, target = build_c5(dev, N)
    xd, td = x.to(dev).requires_grad_(), target.to(dev)

    def step():
        for p in L.parameters():
            p.grad = None
        xd.grad = None
        F.mse_loss(L(xd), td).backward()

    wall, kern, mem = timed_steps(step, steps, warmup,
                                  ("contraction", "basis", "basis_grad", "other"),
                                  list(L.parameters()) + [xd])
    if L.last_backend != "cuda":
        raise RuntimeError("c5 did not run on the native backend")
    line = _line("fwd+bwd samples/s, KANLinear 4096->256 G65 k3 N=8192", N, steps, warmup, wall,
                 "c5: KANLinear(4096->256, G=65, k=3) fp32, N=%d, x ~ U(-1.1, 1.1), fwd + MSE "
                 "+ bwd with dx (3 contractions)" % N,
                 _mfma_roofline(kern, "contraction", "gemm_pipe_kernel (fp32 MFMA contraction; "
                                "forward, parameter and input products)", *recorded_traffic("c5")),
                 kern, mem)
    b_ms, b_cnt, b_work = kern["basis"]
    if b_cnt:
        line["basis_GBps"] = b_work / max(b_cnt, 1) / (b_ms / b_cnt * 1e-3) / 1e9
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_layers([_layer_tensors(L)], x, target, True,
                                                   args.cpu_seconds, 256, "c5")
    return line


def bench_refit(args):
    """KANLinear(512 -> 512, G=8, k=3) fp32 update_grid on N=16384 samples
    from c4's Gaussian mixture: device refit (native Gram kernel + float64
    device solve) timed over `steps` calls; the reference's CPU path
    (dense curve tensor + per-feature lstsq) timed on a subset of the
    features, with the subset stated."""
    import torch
    from torchsplinekan_amd import KANLinear
    from torchsplinekan_amd.reference_backend import ReferenceKANLayer
    N, I, O, G, k = (args.n or 16384), 512, 512, 8, 3
    g = torch.Generator().manual_seed(0)
    means = torch.tensor([-0.8, -0.5, 0.5, 0.8])
    x = means[torch.randint(0, 4, (N, I), generator=g)] + 0.1 * torch.randn(N, I, generator=g)
    coef = torch.randn(O, I, G + k, generator=g) * 0.1
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    xd = x.cuda()

    def fresh():
        with torch.no_grad():
            L.spline_weight.copy_(coef)
            L._copy_grid_(L._ref._uniform_grid(*L._ref.grid_range).to(L.grid.device))

    L = L.cuda()
    for _ in range(max(args.warmup, 1)):
        fresh()
        L.update_grid(xd)
    torch.cuda.synchronize()
    times = []
    for _ in range(args.steps):
        fresh()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        L.update_grid(xd)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    dev_ms = statistics.median(times) * 1e3
    # reference path on the CPU: update_grid of a layer holding the first i_sub features
    i_sub = 16
    ref = ReferenceKANLayer(i_sub, O, grid_size=G, spline_order=k)
    with torch.no_grad():
        ref.spline_weight.copy_(coef[:, :i_sub])
    t0 = time.perf_counter()
    ref.update_grid(x[:, :i_sub])
    cpu_s = time.perf_counter() - t0
    line = {
        "metric": "update_grid ms, KANLinear 512->512 G8 k3 fp32, N=16384 (c4 middle layer)",
        "value": dev_ms, "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "dtype": "f32 (refit solves in f64)",
        "data": "synthetic (c4 Gaussian mixture, seeded)",
        "config": {"workload": "refit: KANLinear(512->512, G=8, k=3).update_grid(x[16384, 512])"},
        "cpu_reference": {"seconds": cpu_s, "features": i_sub, "per_feature_ms": cpu_s * 1e3 / i_sub,
                          "est_full_layer_s": cpu_s * I / i_sub, "threads": torch.get_num_threads(),
                          "sample": f"ReferenceKANLayer.update_grid on the first {i_sub} of {I} "
                                    "features (dense [O, B, I] curves + per-feature CPU lstsq)"},
    }
    print(json.dumps(line), flush=True)


def bench_pinn(args):
    """Physics-informed step (README's higher-order use, in 2-D): KAN([2, 128,
    128, 1], G=8, k=3) in fp64 on N=16384 collocation points; one step is
    u = net(x), grad u and the Laplacian u_xx + u_yy through create_graph,
    loss = mean((lap - f)^2), loss.backward().  The native recorded backward
    (basis derivatives of any order on the device kernels) is timed, then the
    reference's recorded-backward formulation (kan_backward_composite with the
    dense differentiable recurrences, csrc/kan_cpu.cpp:301-345) on the same
    GPU, then the reference backend on the CPU for a bounded sample."""
    import torch
    from torchsplinekan_amd import KAN, _C, _lib
    from torchsplinekan_amd import composite as cmp
    dev = torch.device("cuda", 0)
    N = args.n or 16384
    widths, G, k = [2, 128, 128, 1], 8, 3
    g = torch.Generator().manual_seed(0)
    x = torch.rand(N, 2, generator=g, dtype=torch.float64) * 1.8 - 0.9
    f = torch.sin(3 * x[:, :1]) * torch.cos(2 * x[:, 1:])
    torch.manual_seed(0)
    net = KAN(widths, grid_size=G, spline_order=k, backend="cuda").double()
    with torch.no_grad():
        for layer in net.layers:
            layer.spline_weight.normal_(0.0, 0.1, generator=g)
    ref_state = {n_: t.clone() for n_, t in net.state_dict().items()}
    net = net.to(dev)
    xd, fd = x.to(dev), f.to(dev)

    def step(model, xx, ff):
        for p in model.parameters():
            p.grad = None
        xg = xx.clone().requires_grad_()
        u = model(xg)
        gu = torch.autograd.grad(u.sum(), xg, create_graph=True)[0]
        lap = (torch.autograd.grad(gu[:, 0].sum(), xg, create_graph=True)[0][:, 0]
               + torch.autograd.grad(gu[:, 1].sum(), xg, create_graph=True)[0][:, 1])
        loss = ((lap.unsqueeze(1) - ff) ** 2).mean()
        loss.backward()
        return loss

    def timed(n_steps):
        for _ in range(args.warmup):
            step(net, xd, fd)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_steps):
            step(net, xd, fd)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_steps

    native_s = timed(args.steps)
    # per-kernel times from a separate instrumented pass
    _lib.timing_enable(True)
    timed(args.steps)
    kern = {c: _lib.timing_read(c) for c in ("basis", "basis_grad", "contraction", "other")}
    _lib.timing_enable(False)
    # the reference's recorded backward (dense differentiable recurrences) on the same GPU
    dense_s = float("nan")
    if not args.native_only:
        native_fn = _C.kan_backward_composite_device
        _C.kan_backward_composite_device = cmp.kan_backward_composite
        try:
            dense_s = timed(max(2, args.steps // 2))
        finally:
            _C.kan_backward_composite_device = native_fn
    cpu = None
    if not args.no_cpu_baseline:
        ref = KAN(widths, grid_size=G, spline_order=k, backend="reference").double()
        ref.load_state_dict(ref_state)
        n_cpu = 1024
        t0 = time.perf_counter()
        step(ref, x[:n_cpu], f[:n_cpu])
        cpu_s = time.perf_counter() - t0
        cpu = {"value": n_cpu / cpu_s, "unit": "samples/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": f"one step of the reference backend (backend="
               f"'reference', dense recurrences, torch CPU) on the first {n_cpu} of {N} points, "
               f"{cpu_s:.2f} s"}
    line = {
        "metric": "PINN step samples/s, KAN([2,128,128,1]) G8 k3 fp64 N=16K, Laplacian loss",
        "value": N / native_s, "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": native_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic (x ~ U(-0.9, 0.9)^2 seeded, f = sin(3x) cos(2y))",
        "config": {"workload": "pinn: KAN([2,128,128,1], G=8, k=3) fp64, N=%d, u -> grad u -> "
                               "Laplacian (create_graph) -> MSE -> backward" % N},
        "reference_formulation_same_gpu": {"ms_per_step": dense_s * 1e3,
                                           "speedup": dense_s / native_s,
                                           "what": "kan_backward_composite with the dense "
                                                   "differentiable recurrences (the reference's "
                                                   "create_graph path) on this GPU"},
        "kernels": {k_: {"ms_per_step": v[0] / (args.steps + args.warmup),
                         "launches_per_step": v[1] / (args.steps + args.warmup)}
                    for k_, v in kern.items()},
        "kernel_times": "from a separate instrumented pass (its warmup and timed steps)",
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_infer(args):
    """Inference forward of c3's layer (KANLinear(1024->1024, G=10, k=3) fp32,
    exported: scaler folded, frozen, eval): throughput at N=65536 and latency
    at small batches, through kan_hip_infer with the packed weight kept,
    against the training-path forward op (kan_hip_forward: packs the weight
    and runs the product unsplit on every call)."""
    import torch
    from torchsplinekan_amd import KANLinear, _C, _lib
    dev = torch.device("cuda", 0)
    I = O = 1024
    G, k = 10, 3
    g = torch.Generator().manual_seed(0)
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    with torch.no_grad():
        L.spline_weight.normal_(0.0, 0.1, generator=g)
        L.spline_scaler.uniform_(0.5, 1.5, generator=g)
    E = L.export_inference().to(dev)
    empty = torch.empty(0, device=dev)

    def ev_median(fn, reps):
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
        return statistics.median(times)

    lat = {}
    with torch.no_grad():
        for n in (1, 16, 256, 4096):
            x = (torch.rand(n, I, generator=g) * 2 - 1).to(dev)
            f_inf = lambda: E(x)
            f_fwd = lambda: _C.kan_forward(x, E.grid, E.base_weight, E.spline_weight, empty, k,
                                           False)
            for _ in range(3):
                f_inf()
                f_fwd()
            lat[str(n)] = {"infer_ms": ev_median(f_inf, 30), "training_forward_op_ms":
                           ev_median(f_fwd, 30)}
        N = 65536
        x = (torch.rand(N, I, generator=g) * 2 - 1).to(dev)
        for _ in range(args.warmup):
            E(x)
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            E(x)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / args.steps
        c_ms, c_cnt, c_work = _lib.timing_read("contraction")
        b_ms, b_cnt, _ = _lib.timing_read("basis")
        _lib.timing_enable(False)
        fwd_ms = ev_median(lambda: _C.kan_forward(x, E.grid, E.base_weight, E.spline_weight,
                                                   empty, k, False), max(args.steps, 3))
    ach = c_work / (c_ms * 1e-3) / 1e12 if c_cnt else 0.0
    line = {
        "metric": "inference samples/s, KANLinear 1024->1024 G10 k3 fp32 (exported), N=64K",
        "value": N / wall, "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (x ~ U(-1, 1) seeded; coef ~ N(0, 0.1), scaler ~ U(0.5, 1.5) folded)",
        "config": {"workload": "infer: c3 layer exported, no autograd; latency at n = 1, 16, "
                               "256, 4096"},
        "roofline": {"bound": "mfma", "kernel": "gemm_pipe_kernel (NT, packed weight)",
                     "achieved": ach, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": ach / PEAK_FP32_MFMA_TFLOPS, "traffic": None,
                     "avg_launch_ms": c_ms / max(c_cnt, 1), "launches": c_cnt},
        "basis_ms": b_ms / max(b_cnt, 1),
        "training_forward_op_ms_at_64K": fwd_ms,
        "latency_ms": lat,
    }
    print(json.dumps(line), flush=True)



def bench_stream(args):
    """HBM streaming ceilings of this GPU for buffers of c3's size: float4
    write, read and copy kernels (kan_hip_stream_probe) over a buffer of the
    c3 augmented basis' size (65536 x 14336 fp32 = 3.76 GB), and the write
    pattern of the basis kernel on that layout (row segments), each timed
    with the library's HIP events; the basis kernels' GB/s are judged against
    these."""
    import torch
    from torchsplinekan_amd import _C, _lib
    dev = torch.device("cuda", 0)
    nbytes = 65536 * 14336 * 4
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    b = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    out = {}
    rows = nbytes // (14336 * 4)
    for mode, name, moved in ((0, "write", nbytes), (1, "read", nbytes), (2, "copy", 2 * nbytes),
                              (3, "basis_row_segments", nbytes),
                              (4, "one_segment_per_workgroup_write", nbytes),
                              (5, "one_segment_per_workgroup_read", nbytes + rows * 1024 * 4),
                              (6, "basis_row_segments_one_step", nbytes),
                              (7, "workgroup_segments_4_rows", nbytes),
                              (8, "workgroup_segments_16_rows", nbytes),
                              (9, "one_segment_per_wave_workgroup_write", nbytes),
                              (10, "two_segments_per_workgroup_read", nbytes + rows * 1024 * 4)):
        for _ in range(args.warmup):
            _C.stream_probe(mode, a, b)
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        for _ in range(args.steps):
            _C.stream_probe(mode, a, b)
        torch.cuda.synchronize()
        ms, cnt, _ = _lib.timing_read("stream")
        _lib.timing_enable(False)
        avg = ms / max(cnt, 1)
        out[name] = {"avg_ms": avg, "GB/s": moved / (avg * 1e-3) / 1e9,
                     "frac_of_8TBps": moved / (avg * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "bytes_per_launch": moved, "launches": cnt}
    line = {"metric": "HBM streaming GB/s (float4 kernels, c3 augmented-basis-sized buffer)",
            "value": out["write"]["GB/s"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "higher_is_better": True, "dtype": "f32",
            "data": "synthetic", "config": {"workload": "stream: %d-byte buffer" % nbytes},
            "modes": out}
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the sample axis would shard over GPUs, with one all-reduce of the parameter "
              "gradients per step)", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return

    import torch
    import torch.nn.functional as F

    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    single = {"c2": run_c2, "c4": run_c4, "c5": run_c5}
    if args.workload in single:
        print(json.dumps(single[args.workload](args, dev, args.steps, args.warmup)), flush=True)
        return
    other = {"stream": bench_stream, "infer": bench_infer, "pinn": bench_pinn,
             "refit": bench_refit}
    if args.workload in other:
        other[args.workload](args)
        return

    line = run_c3(args, dev, args.steps, args.warmup, need_dx=args.workload == "c3",
                  f64=args.dtype == "f64")
    if args.workload == "c3" and args.dtype == "f32" and not args.no_other_configs and not args.n:
        torch.cuda.empty_cache()
        line["other_configs"] = {}
        nodx = lambda a, d, st, w: run_c3(a, d, st, w, need_dx=False)
        c3_64 = lambda a, d, st, w: run_c3(a, d, max(3, st // 4), min(w, 2), f64=True)

        def c4_64(a, d, st, w):
            a64 = argparse.Namespace(**vars(a))
            a64.dtype = "f64"
            return run_c4(a64, d, st, w)

        for name, fn in (("c3-nodx", nodx), ("c2", run_c2), ("c4", run_c4), ("c5", run_c5),
                         ("c3-f64", c3_64), ("c4-f64", c4_64)):
            try:
                line["other_configs"][name] = fn(args, dev, args.steps, args.warmup)
            except Exception as exc:  # reported in the line; the metric stands on its own
                line["other_configs"][name] = {"error": f"{type(exc).__name__}: {exc}"}
            torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
