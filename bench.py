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
events recorded by the library on the launch stream) and a CPU baseline
(the numpy oracle on a bounded sample of the same workload, rank 0 only).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3|c3-nodx]
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
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3",
                    choices=["c3", "c3-nodx", "c4", "refit", "pinn", "infer"],
                    help="c3 (the metric's config, default), c3-nodx (x without grad, the "
                         "reference benchmark's semantics), c4 (KAN([256,512,512,64]) with "
                         "forward_with_regularization), refit (update_grid of c4's 512->512 "
                         "layer), pinn (Laplacian loss of KAN([2,128,128,1]) through "
                         "create_graph) or infer (c3's layer, exported, inference forward: "
                         "throughput at N=65536 and latency at small batches); these are "
                         "reported separately, not the metric")
    ap.add_argument("--n", type=int, default=65536, help="samples per step (default: config's 65536)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the baseline sample")
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


def make_inputs(N, I, O, G, k, seed=0):
    """Seeded CPU draws in a fixed order: x, coef, base_weight, scaler, target."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(N, I, generator=g) * 2 - 1
    coef = torch.randn(O, I, G + k, generator=g) * 0.1
    bw = (torch.rand(O, I, generator=g) * 2 - 1) / (I ** 0.5)
    scaler = torch.rand(O, I, generator=g) + 0.5
    target = torch.randn(N, O, generator=g)
    return x, coef, bw, scaler, target


def cpu_baseline(x, coef, bw, scaler, target, grid, k, need_dx, seconds):
    """The numpy oracle (restatement of the reference CPU path: basis
    recurrence, BLAS GEMMs, analytic backward) timed on this host on
    consecutive 1024-row chunks of the same workload until `seconds` of work
    are done; returns samples/s, BLAS threads and the sample description."""
    import numpy as np
    from oracle import kan_oracle as ko
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()
                       if p.get("user_api") == "blas"] or [1])
    except Exception:  # threadpoolctl missing: report the env setting
        threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    N, O = target.shape
    gridn = grid.numpy()
    sw, bwn, sc = coef.numpy(), bw.numpy(), scaler.numpy()
    chunk = 1024
    done, t_total = 0, 0.0
    for n0 in range(0, N, chunk):
        xs = x[n0:n0 + chunk].numpy()
        ts = target[n0:n0 + chunk].numpy()
        t0 = time.perf_counter()
        y, H = ko.kan_forward(xs, gridn, bwn, sw, sc, k)
        D = (np.float32(2.0) / np.float32(N * O)) * (y - ts)
        if need_dx:
            ko.kan_backward(D, xs, gridn, bwn, sw, sc, k, basis=H)
        else:
            ko.kan_backward_params(D, xs, bwn, sw, sc, H)
        t_total += time.perf_counter() - t0
        done += xs.shape[0]
        if t_total >= seconds:
            break
    return {
        "value": done / t_total,
        "unit": "samples/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"numpy oracle (oracle/kan_oracle.py) fp32 fwd+MSE+bwd of the first {done} of "
                   f"{N} rows in {chunk}-row chunks, {t_total:.1f} s; BLAS threads={threads}, "
                   f"elementwise work single-threaded; host {os.cpu_count()} logical CPUs"),
    }


def bench_c4(args):
    """KAN([256, 512, 512, 64], grid_size=8, spline_order=3) fp32, knots from
    update_grid on x drawn from a 4-component Gaussian mixture (means +-0.5,
    +-0.8, sd 0.1), N=16384; one step is forward_with_regularization(1e-2,
    1e-2, reg_impl="auto") + MSE + backward (x without grad)."""
    import torch
    import torch.nn.functional as F
    from torchsplinekan_amd import KAN, _lib
    dev = torch.device("cuda", 0)
    N, widths = args.n if args.n != 65536 else 16384, [256, 512, 512, 64]
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
    net = net.to(dev)
    xd, td = x.to(dev), target.to(dev)
    net.update_grid(xd)          # before timing (least squares on the host)

    def step():
        for p in net.parameters():
            p.grad = None
        y, reg = net.forward_with_regularization(xd, 1e-2, 1e-2, reg_impl="auto")
        (F.mse_loss(y, td) + reg).backward()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if any(l.last_backend != "cuda" for l in net.layers):
        raise RuntimeError("c4 did not run the fused native path")
    kern = {c: _lib.timing_read(c) for c in ("edge", "edge_grad", "basis", "basis_grad",
                                             "contraction", "other")}
    _lib.timing_enable(False)
    e_ms, e_cnt, e_work = kern["edge"]
    eg_ms, eg_cnt, eg_work = kern["edge_grad"]
    c_ms, c_cnt, c_work = kern["contraction"]
    ach = e_work / (e_ms * 1e-3) / 1e12 if e_cnt else 0.0
    ach_g = eg_work / (eg_ms * 1e-3) / 1e12 if eg_cnt else 0.0
    ach_c = c_work / (c_ms * 1e-3) / 1e12 if c_cnt else 0.0
    line = {
        "metric": "fwd+bwd samples/s, KAN([256,512,512,64]) G8 k3 N=16K forward_with_regularization",
        "value": N * args.steps / wall, "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (Gaussian-mixture x, seeded; knots from update_grid)",
        "config": {"workload": "c4: KAN([256,512,512,64], G=8, k=3) fp32, N=%d, "
                               "forward_with_regularization(1e-2, 1e-2, 'auto') + MSE + backward" % N},
        # dominant kernel class: the edge-statistic backward on FP32 MFMA
        # (fused kernel for layers that need both gradient sides: phi once
        # plus two products, 6 n O I (R+1) flops; parameter kernel for the
        # first layer, whose input needs no gradient: 4 n O I (R+1))
        "roofline": {"bound": "mfma",
                     "kernel": "edge_bwd_mfma_kernel (both gradient sides) + edge_param_mfma_kernel "
                               "(first layer): mean|phi| backward",
                     "achieved": ach_g, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": ach_g / PEAK_FP32_MFMA_TFLOPS, "traffic": None,
                     "flop_per_launch": eg_work / max(eg_cnt, 1),
                     "avg_launch_ms": eg_ms / max(eg_cnt, 1), "launches": eg_cnt},
        "kernels": {k_: {"ms_per_step": v[0] / args.steps, "launches_per_step": v[1] / args.steps}
                    for k_, v in kern.items()},
        "edge_forward_tflops": ach,
        "contraction_tflops": ach_c,
    }
    print(json.dumps(line), flush=True)


def bench_refit(args):
    """KANLinear(512 -> 512, G=8, k=3) fp32 update_grid on N=16384 samples
    from c4's Gaussian mixture: device refit (native Gram kernel + float64
    device solve) timed over `steps` calls; the reference's CPU path
    (dense curve tensor + per-feature lstsq) timed on a subset of the
    features, with the subset stated."""
    import torch
    from torchsplinekan_amd import KANLinear
    from torchsplinekan_amd.reference_backend import ReferenceKANLayer
    N, I, O, G, k = (args.n if args.n != 65536 else 16384), 512, 512, 8, 3
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
    N = args.n if args.n != 65536 else 16384
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

    _lib.timing_enable(True)
    native_s = timed(args.steps)
    kern = {c: _lib.timing_read(c) for c in ("basis", "basis_grad", "contraction", "other")}
    _lib.timing_enable(False)
    # the reference's recorded backward (dense differentiable recurrences) on the same GPU
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
        "kernels": {k_: {"ms_per_step": v[0] / args.steps, "launches_per_step": v[1] / args.steps}
                    for k_, v in kern.items()},
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
    from torchsplinekan_amd import KANLinear, _lib

    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.workload == "c4":
        bench_c4(args)
        return
    if args.workload == "infer":
        bench_infer(args)
        return
    if args.workload == "pinn":
        bench_pinn(args)
        return
    if args.workload == "refit":
        bench_refit(args)
        return

    I = O = 1024
    G, k = 10, 3
    N = args.n
    need_dx = args.workload == "c3"
    x, coef, bw, scaler, target = make_inputs(N, I, O, G, k, seed=0)
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    with torch.no_grad():
        L.spline_weight.copy_(coef)
        L.base_weight.copy_(bw)
        L.spline_scaler.copy_(scaler)
    grid_cpu = L.grid.detach().clone()
    L = L.to(dev)
    xd = x.to(dev).requires_grad_(need_dx)
    td = target.to(dev)
    torch.cuda.synchronize()

    def step():
        for p in L.parameters():
            p.grad = None
        xd.grad = None
        y = L(xd)
        loss = F.mse_loss(y, td)
        loss.backward()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    _lib.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if L.last_backend != "cuda":
        raise RuntimeError("the timed steps did not run on the native backend")
    step_ms = [a.elapsed_time(b) for a, b in ev]
    kernels = {}
    for cls in ("contraction", "basis", "basis_grad", "other"):
        ms, cnt, work = _lib.timing_read(cls)
        kernels[cls] = (ms, cnt, work)
    _lib.timing_enable(False)

    ms_per_step = wall * 1e3 / args.steps
    value = N * args.steps / wall

    c_ms, c_cnt, c_work = kernels["contraction"]
    c_avg_ms = c_ms / max(c_cnt, 1)
    c_flop = c_work / max(c_cnt, 1)
    achieved = c_flop / (c_avg_ms * 1e-3) / 1e12 if c_cnt else 0.0
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "contraction_c3_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    b_ms, b_cnt, b_work = kernels["basis"]
    g_ms, g_cnt, g_work = kernels["basis_grad"]

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.Generator draws, random-init weights of the config)",
        "config": {
            "workload": ("c3: KANLinear(1024->1024, grid_size=10, spline_order=3) fp32, N=%d, "
                         "fwd + MSE + bwd %s" % (N, "with dx (3 contractions)" if need_dx
                                                 else "without dx (2 contractions)")),
            "in_features": I, "out_features": O, "grid_size": G, "spline_order": k,
            "samples_per_step": N, "x_requires_grad": need_dx,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_pipe_kernel (fp32 MFMA contraction; average over the forward, parameter and input launches)",
            "achieved": achieved,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_FP32_MFMA_TFLOPS,
            "traffic": traffic,
            "flop_per_launch": c_flop,
            "avg_launch_ms": c_avg_ms,
            "launches": c_cnt,
        },
        "step_ms_median_events": statistics.median(step_ms),
        "kernels": {
            "basis": {"avg_ms": b_ms / max(b_cnt, 1), "launches": b_cnt,
                      "GB/s": (b_work / max(b_cnt, 1)) / (b_ms / max(b_cnt, 1) * 1e-3) / 1e9
                      if b_cnt else None},
            "basis_grad": {"avg_ms": g_ms / max(g_cnt, 1), "launches": g_cnt,
                           "GB/s": (g_work / max(g_cnt, 1)) / (g_ms / max(g_cnt, 1) * 1e-3) / 1e9
                           if g_cnt else None},
            "contraction_ms_per_step": c_ms / args.steps,
            "other_ms_per_step": kernels["other"][0] / args.steps,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(x, coef, bw, scaler, target, grid_cpu, k, need_dx,
                                            args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
