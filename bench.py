#!/usr/bin/env python3
"""Benchmark of the OmniMatch HAL hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]

Headline (the `value`): fp32 GEMM 4096x4096x4096, row-major A[M,K] x B[K,N]
(CPUBackend::matmul's layout), inputs resident in HBM; one step = one GEMM;
value = TFLOP/s over the timed steps (HIP events on the library stream).
Second metric in the same line (`resnet18_conv`): the ResNet-18 conv stack
forward at batch 32, 224x224 (20 convs, each conv + BN-inference + ReLU fused),
as images/s.

Also reported:
  roofline      — fp32 MFMA roof for the GEMM kernel (achieved = 2MNK / average
                  launch time, peak 157.3 TFLOP/s), traffic from the committed
                  rocprofv3 FETCH_SIZE / WRITE_SIZE counters when present;
  cpu_baseline  — the reference CPUBackend itself (oracle/_ref, built from the
                  reference sources) timed on this host's cores on a bounded
                  sample of the same workloads;
  parity        — sampled rows of the timed GEMM and two sampled images of the
                  conv stack against float64 (K-scaled error, bar 1e-4).
Only one GPU is used: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK_FP32 = 157.3e12      # MI355X dense fp32 MFMA, FLOP/s
PEAK_HBM = 8.0e12         # bytes/s
M = N = K = 4096


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 counter summary, if any."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            d = json.load(f)
        return d.get(name, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def bench_gemm(om, steps: int, warmup: int):
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    import oracle as O
    A = O.randn((M, K), 11)
    B = O.randn((K, N), 12)
    dA, dB = om.DeviceBuffer.from_numpy(A), om.DeviceBuffer.from_numpy(B)
    dC = om.DeviceBuffer.empty((M, N))
    H = om.HIPBackend
    for _ in range(warmup):
        H.matmul(dA, dB, dC, M, K, N)
    om.synchronize()
    timer = StreamTimer(om.stream_handle())
    t0 = time.perf_counter()
    timer.start()
    for _ in range(steps):
        H.matmul(dA, dB, dC, M, K, N)
    timer.stop()
    ms_total = timer.ms()
    om.synchronize()
    wall = time.perf_counter() - t0
    ms = ms_total / steps
    flops = 2.0 * M * N * K
    # parity on sampled rows (float64 brute force, K-scaled bound)
    C = dC.numpy()
    rows = np.r_[0:4, 2046:2050, 4092:4096]
    C64, bound = O.gemm_f64(A[rows], B)
    err = O.normalized_error(C[rows], C64, bound)
    return ms, flops, wall, err


def bench_resnet18(om, steps: int, warmup: int, batch: int = 32):
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    from resnet_shapes import conv_bytes, conv_flops, out_hw, resnet18_convs
    import oracle as O
    H = om.HIPBackend
    layers = []
    for li, (name, cin, h, w, cout, k, s, p) in enumerate(resnet18_convs()):
        fan_in = cin * k * k
        bnd = np.sqrt(6.0 / fan_in)
        x = O.randn((batch, cin, h, w), 100 + li)
        wt = O.uniform((cout, cin, k, k), 200 + li, -bnd, bnd)
        g, b = O.uniform((cout,), 300 + li, 0.5, 1.5), O.randn((cout,), 400 + li, 0.1)
        m, v = O.randn((cout,), 500 + li, 0.1), O.uniform((cout,), 600 + li, 0.5, 1.5)
        ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
        dev = dict(x=om.DeviceBuffer.from_numpy(x), w=om.DeviceBuffer.from_numpy(wt),
                   g=om.DeviceBuffer.from_numpy(g), b=om.DeviceBuffer.from_numpy(b),
                   m=om.DeviceBuffer.from_numpy(m), v=om.DeviceBuffer.from_numpy(v),
                   y=om.DeviceBuffer.empty((batch, cout, ho, wo)))
        layers.append(((name, cin, h, w, cout, k, s, p), dev, (x, wt, g, b, m, v)))

    def forward():
        for (name, cin, h, w, cout, k, s, p), d, _ in layers:
            H.conv2dBiasBnAct(d["x"], d["w"], None, d["g"], d["b"], d["m"], d["v"], 1e-5, 1, d["y"],
                              batch, cin, h, w, cout, k, k, s, p)

    for _ in range(warmup):
        forward()
    om.synchronize()
    timer = StreamTimer(om.stream_handle())
    timer.start()
    for _ in range(steps):
        forward()
    timer.stop()
    ms = timer.ms() / steps
    # per-layer times (for the roofline table)
    per = []
    for (shape, d, _) in layers:
        name, cin, h, w, cout, k, s, p = shape
        t = StreamTimer(om.stream_handle())
        reps = max(3, steps // 2)
        t.start()
        for _ in range(reps):
            H.conv2dBiasBnAct(d["x"], d["w"], None, d["g"], d["b"], d["m"], d["v"], 1e-5, 1, d["y"],
                              batch, cin, h, w, cout, k, k, s, p)
        t.stop()
        lms = t.ms() / reps
        f, by = conv_flops(shape, batch), conv_bytes(shape, batch)
        roof = max(f / PEAK_FP32, by / PEAK_HBM) * 1e3
        per.append({"layer": name, "ms": round(lms, 4), "tflops": round(f / lms / 1e9, 1),
                    "roof_frac": round(roof / lms, 3)})
    flops = sum(conv_flops(sh, batch) for sh, _, _ in layers)
    roof_ms = sum(max(conv_flops(sh, batch) / PEAK_FP32, conv_bytes(sh, batch) / PEAK_HBM) for sh, _, _ in layers) * 1e3
    # parity: two images of three layers against float64
    errs = []
    for idx in (0, 9, 19):
        (name, cin, h, w, cout, k, s, p), d, (x, wt, g, b, m, v) = layers[idx]
        y = d["y"].numpy()[[0, batch - 1]]
        o64, bound = O.conv_f64(x[[0, batch - 1]], wt, None, s, p, gamma=g, beta=b, mean=m, var=v, act=1)
        errs.append(O.normalized_error(y, o64, bound))
    return ms, flops, roof_ms, per, max(errs)


def cpu_baseline_gemm(budget_s: float = 10.0):
    """Reference CPUBackend::matmul (oracle/_ref) on 4096^3: one warm-up, then
    repeated for about budget_s seconds; the median run is reported."""
    import oracle as O
    backend = "reference" if O.ref_lib() is not None else "oracle"
    A, B = O.randn((M, K), 11), O.randn((K, N), 12)
    O.matmul(A, B, backend=backend)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t = time.perf_counter()
        O.matmul(A, B, backend=backend)
        times.append(time.perf_counter() - t)
    dt = float(np.median(times))
    return backend, 2.0 * M * N * K / dt / 1e12, dt, len(times)


def cpu_baseline_resnet18(batch: int = 32, budget_s: float = 10.0):
    """Reference conv2d -> batchNorm2d(eval) -> relu over the 20 ResNet-18 convs
    at the benchmark batch, repeated for about budget_s seconds (median pass)."""
    import oracle as O
    from resnet_shapes import resnet18_convs
    backend = "reference" if O.ref_lib() is not None else "oracle"
    data = []
    for li, (name, cin, h, w, cout, k, s, p) in enumerate(resnet18_convs()):
        data.append(((s, p), O.randn((batch, cin, h, w), 100 + li), O.randn((cout, cin, k, k), 200 + li, 0.05),
                     O.uniform((cout,), 300 + li, 0.5, 1.5), O.randn((cout,), 400 + li, 0.1),
                     O.randn((cout,), 500 + li, 0.1), O.uniform((cout,), 600 + li, 0.5, 1.5)))

    def one_pass():
        t0 = time.perf_counter()
        for (s, p), x, wt, g, b, m, v in data:
            y = O.conv2d(x, wt, None, s, p, backend=backend)
            y, _, _ = O.batchnorm2d_eval(y, g, b, m, v, backend=backend)
            O.relu(y, backend=backend)
        return time.perf_counter() - t0

    one_pass()
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        times.append(one_pass())
    dt = float(np.median(times))
    return backend, batch / dt, dt, len(times)


def traffic_probe():
    """The dispatch sequence the HBM-traffic counter passes profile: a 256 MiB
    device copy (calibration), three 4096^3 NN GEMMs, one ResNet-18 conv stack
    pass at batch 32 (each layer once), one dispatch at a time."""
    import omnimatchdeeplearningtool_amd as om
    from resnet_shapes import out_hw, resnet18_convs
    om.init(0)
    H = om.HIPBackend
    n = 64 << 20
    src, dst = om.DeviceBuffer.empty((n,)), om.DeviceBuffer.empty((n,))
    H.fillValue(src, n, 1.0)
    om.synchronize()
    H.copy(src, dst, n)
    om.synchronize()
    A = om.DeviceBuffer.from_numpy(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32))
    B = om.DeviceBuffer.from_numpy(np.random.default_rng(2).standard_normal((K, N), dtype=np.float32))
    C = om.DeviceBuffer.empty((M, N))
    for _ in range(3):
        H.matmul(A, B, C, M, K, N)
    om.synchronize()
    bs = 32
    for name, cin, h, w, cout, k, s, p in resnet18_convs():
        ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
        x = om.DeviceBuffer.empty((bs * cin * h * w,))
        H.fillValue(x, bs * cin * h * w, 0.1)
        wt = om.DeviceBuffer.empty((cout * cin * k * k,))
        H.fillValue(wt, cout * cin * k * k, 0.01)
        bn = [om.DeviceBuffer.empty((cout,)) for _ in range(4)]
        for d in bn:
            H.fillValue(d, cout, 1.0)
        y = om.DeviceBuffer.empty((bs * cout * ho * wo,))
        om.synchronize()
        H.conv2dBiasBnAct(x, wt, None, bn[0], bn[1], bn[2], bn[3], 1e-5, 1, y, bs, cin, h, w, cout, k, k, s, p)
        om.synchronize()
    log("traffic probe done")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the dispatch sequence profiled for HBM traffic (no JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the HAL path runs on a single "
              f"MI355X and multi-GPU runs are not part of this build.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    if args.traffic_probe:
        traffic_probe()
        return

    import omnimatchdeeplearningtool_amd as om
    om.init(0)
    dev = om.device_name(0)
    log(f"device {dev}")

    log(f"gemm 4096^3 NN: warmup {args.warmup}, steps {args.steps}")
    ms, flops, wall, gemm_err = bench_gemm(om, args.steps, args.warmup)
    tflops = flops / ms / 1e9
    log(f"gemm {ms:.4f} ms/step  {tflops:.1f} TFLOP/s  parity {gemm_err:.2e}")

    log("resnet18 conv stack b32")
    r_steps = max(5, args.steps // 2)
    r_ms, r_flops, r_roof_ms, per, conv_err = bench_resnet18(om, r_steps, max(2, args.warmup))
    img_s = 32.0 / (r_ms / 1e3)
    log(f"resnet18 {r_ms:.3f} ms/batch  {img_s:.0f} img/s  roof frac {r_roof_ms / r_ms:.3f}  parity {conv_err:.2e}")

    cpu = None
    cpu_r18 = None
    if rank == 0 and not args.no_cpu:
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        log(f"cpu baseline (reference CPUBackend, {threads} threads)")
        kind, cpu_tf, cpu_dt, n1 = cpu_baseline_gemm()
        cpu = {"value": round(cpu_tf, 4), "unit": "TFLOP/s", "cores": threads,
               "kind": "reference" if kind == "reference" else "port",
               "sample": f"median of {n1} runs of the 4096^3 NN fp32 GEMM ({cpu_dt:.2f} s each) after one warm-up: "
                         f"CPUBackend::matmul (AVX2 4x8 FMA + OpenMP) compiled from the reference sources"}
        kind2, r18_ips, r18_dt, n2 = cpu_baseline_resnet18()
        cpu_r18 = {"value": round(r18_ips, 3), "unit": "img/s", "cores": threads,
                   "kind": "reference" if kind2 == "reference" else "port",
                   "sample": f"median of {n2} passes of batch 32 through the 20 ResNet-18 convs "
                             f"(conv2d -> batchNorm2d(eval) -> relu, {r18_dt:.2f} s each) after one warm-up"}
        log(f"cpu gemm {cpu_tf * 1e3:.1f} GFLOP/s, cpu resnet18 {r18_ips:.3f} img/s")

    gemm_kernel_ms = ms
    traffic = _traffic("gemm_f32_4096_nn")
    line = {
        "metric": "fp32 GEMM TFLOP/s @4096³ (% MFMA peak); ResNet-18 conv fwd img/s b32",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) matrices; seeded N(0,1) images, Kaiming-uniform weights, seeded BN stats)",
        "config": {"workload": "fp32 GEMM 4096x4096x4096, row-major A[M,K] x B[K,N] (CPUBackend::matmul layout)",
                   "M": M, "N": N, "K": K, "layout": "NN", "device": dev},
        "pct_mfma_peak": round(100.0 * tflops * 1e12 / PEAK_FP32, 1),
        "roofline": {"bound": "mfma", "achieved": round(flops / gemm_kernel_ms / 1e9, 2), "peak": 157.3,
                     "unit": "TFLOP/s", "frac": round(flops / gemm_kernel_ms / 1e9 / 157.3, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "parity": {"gemm_sampled_rows_max_err": gemm_err, "conv_sampled_max_err": conv_err, "tol": 1e-4},
        "resnet18_conv": {"value": round(img_s, 1), "unit": "img/s", "batch": 32, "ms_per_batch": round(r_ms, 4),
                          "tflops": round(r_flops / r_ms / 1e9, 2),
                          "roofline": {"bound": "mfma (per-layer max(flops/157.3T, bytes/8TB/s))",
                                       "roof_ms": round(r_roof_ms, 4), "frac": round(r_roof_ms / r_ms, 4)},
                          "layers": per, "cpu_baseline": cpu_r18},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
