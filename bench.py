#!/usr/bin/env python3
"""Benchmark of the OmniMatch HAL hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]

Headline (the `value`): fp32 GEMM 4096x4096x4096, row-major A[M,K] x B[K,N]
(CPUBackend::matmul's layout), inputs resident in HBM; one step = one GEMM;
value = TFLOP/s over the timed steps (HIP events on the library stream). It is
timed right after the fp32 GEMM sweep, whose last shapes are 8192^3: an idle
MI355X runs its first ~20 ms of load at lower clocks.
Second metric in the same line (`resnet18_conv`): the ResNet-18 conv stack
forward at batch 32, 224x224 (20 convs, each conv + BN-inference + ReLU fused),
as images/s over eager launches (the same 20 launches replayed from a
captured HIP graph are timed beside it).

Also reported:
  roofline      — fp32 MFMA roof for the GEMM kernel (achieved = 2MNK / average
                  launch time, peak 157.3 TFLOP/s); traffic is read from the
                  committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
                  (profiles/traffic.json), not measured in this run, and
                  roofline.traffic_source says so;
  cpu_baseline  — the reference CPUBackend itself (oracle/_ref, built from the
                  reference sources) timed on this host's cores on a bounded
                  sample of the same workloads;
  parity        — every leg's sampled outputs against float64 or the reference
                  chain on the CPU: rows of the timed GEMM and of each sweep
                  shape, two images of three layers of each conv stack, the
                  network logits, each op and weight gradient of the training
                  step, rows / batches of every ViT GEMM, two images of the
                  fused attention and of the attention layer, and every layer,
                  gradient and the loss of the MLP step (bars in parity.bars).
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

from omnimatchdeeplearningtool_amd import synthetic as syn   # noqa: E402  (seeded inputs)

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


GEMM_ROWS = np.r_[0:4, 2046:2050, 4092:4096]   # rows of the 4096^3 product checked on the CPU


def settle(om, fn, seconds: float = 0.03) -> None:
    """Runs fn back to back for at least `seconds`, untimed: an MI355X that has been
    idle needs about 20 ms of load before its clocks settle, and every leg but the
    headline starts after host set-up (the headline keeps exactly its W warm-up steps:
    it follows the sweep with no idle gap). Calls go out in doubling batches between
    waits, so launches of a few microseconds also keep the GPU busy."""
    t0 = time.perf_counter()
    batch = 1
    while time.perf_counter() - t0 < seconds:
        for _ in range(batch):
            fn()
        om.synchronize()
        batch = min(2 * batch, 1024)


def read_rows(om, buf, rows, ncols: int, dtype=np.float32) -> np.ndarray:
    """Rows `rows` of a row-major device matrix with ncols columns (only those bytes cross PCIe)."""
    out = np.empty((len(rows), ncols), dtype)
    nb = ncols * out.itemsize
    for i, r in enumerate(rows):
        om.call("omHipCopyD2H", out[i].ctypes.data, buf.ptr + int(r) * nb, nb)
    return out


def gemm_inputs(om):
    """The headline GEMM's seeded inputs, uploaded to HBM."""
    A = syn.randn((M, K), 11)
    B = syn.randn((K, N), 12)
    return om.DeviceBuffer.from_numpy(A), om.DeviceBuffer.from_numpy(B), om.DeviceBuffer.empty((M, N))


def bench_gemm(om, bufs, steps: int, warmup: int):
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    dA, dB, dC = bufs
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
    return ms, flops, wall, read_rows(om, dC, GEMM_ROWS, N)


# (M, N, K); the cubes last, so the sweep ends with 8192^3 launches (the
# headline GEMM is timed right after it, on clocks that are already up)
GEMM_SWEEP = [(128, 4096, 4096), (8192, 256, 2048), (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
              (4096, 4096, 4096), (8192, 8192, 8192)]


def bench_gemm_sweep(om, steps: int, warmup: int):
    """The fp32 GEMM sweep in both layouts: row-major A x B and A x B^T (Linear weight)."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    H = om.HIPBackend
    timer = StreamTimer(om.stream_handle())
    out, samples = [], []
    for (m, n, k) in GEMM_SWEEP:
        A = syn.randn((m, k), 21 + m)
        dA = om.DeviceBuffer.from_numpy(A)
        dC = om.DeviceBuffer.empty((m, n))
        reps = max(3, min(steps, int(2e12 / (2.0 * m * n * k))))   # about 2 TFLOP of work per shape
        for layout in ("NN", "NT"):
            B = syn.randn((k, n) if layout == "NN" else (n, k), 22 + n)
            dB = om.DeviceBuffer.from_numpy(B)
            f = (lambda: H.matmul(dA, dB, dC, m, k, n)) if layout == "NN" else (lambda: H.matmulTransB(dA, dB, dC, m, k, n))
            settle(om, f)   # the inputs were made on the host meanwhile: the GPU sat idle
            for _ in range(warmup):
                f()
            om.synchronize()
            timer.start()
            for _ in range(reps):
                f()
            timer.stop()
            ms = timer.ms() / reps
            rows = np.unique(np.r_[0, m // 2, m - 1])
            samples.append(((m, n, k, layout), rows, read_rows(om, dC, rows, n)))
            tf = 2.0 * m * n * k / ms / 1e9
            out.append({"M": m, "N": n, "K": k, "layout": layout, "ms": round(ms, 4), "tflops": round(tf, 1),
                        "frac_of_157_3": round(tf / 157.3, 3), "parity": None})
            log(f"gemm sweep {m}x{n}x{k} {layout}: {ms:.4f} ms  {tf:.1f} TFLOP/s")
            dB.free()
        dA.free(); dC.free()
    return out, samples


RESNET18_CHECKED = (0, 9, 19)   # layers whose outputs (two images) are checked on the CPU


def resnet18_layer_inputs(li: int, batch: int):
    """Seeded input, Kaiming-uniform weight and BN vectors of ResNet-18 conv layer li."""
    from resnet_shapes import resnet18_convs
    name, cin, h, w, cout, k, s, p = resnet18_convs()[li]
    bnd = np.sqrt(6.0 / (cin * k * k))
    x = syn.randn((batch, cin, h, w), 100 + li)
    wt = syn.uniform((cout, cin, k, k), 200 + li, -bnd, bnd)
    g, b = syn.uniform((cout,), 300 + li, 0.5, 1.5), syn.randn((cout,), 400 + li, 0.1)
    m, v = syn.randn((cout,), 500 + li, 0.1), syn.uniform((cout,), 600 + li, 0.5, 1.5)
    return x, wt, g, b, m, v


def resnet18_setup(om, batch: int = 32):
    """The 20 ResNet-18 conv layers' seeded inputs, uploaded to HBM."""
    from resnet_shapes import out_hw, resnet18_convs
    layers = []
    for li, (name, cin, h, w, cout, k, s, p) in enumerate(resnet18_convs()):
        x, wt, g, b, m, v = resnet18_layer_inputs(li, batch)
        ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
        dev = dict(x=om.DeviceBuffer.from_numpy(x), w=om.DeviceBuffer.from_numpy(wt),
                   g=om.DeviceBuffer.from_numpy(g), b=om.DeviceBuffer.from_numpy(b),
                   m=om.DeviceBuffer.from_numpy(m), v=om.DeviceBuffer.from_numpy(v),
                   y=om.DeviceBuffer.empty((batch, cout, ho, wo)))
        layers.append(((name, cin, h, w, cout, k, s, p), dev, (x, wt, g, b, m, v)))
    return layers


def bench_resnet18(om, layers, steps: int, warmup: int, batch: int = 32):
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    from resnet_shapes import conv_bytes, conv_flops
    H = om.HIPBackend

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
    # The same 20 launches replayed from a captured HIP graph (the kernels and
    # their work are unchanged; the host launch cost and the gaps between
    # launches go), timed straight after the eager passes; the replays'
    # outputs are compared with an eager pass's bit for bit at the end, once
    # every timing is done (the read-backs would leave the GPU idle).
    graph = om.Graph(forward)
    for _ in range(warmup):
        graph.launch()
    om.synchronize()
    timer.start()
    for _ in range(steps):
        graph.launch()
    timer.stop()
    graph_ms = timer.ms() / steps
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
    return ms, flops, roof_ms, per, graph_ms, (forward, graph)


def resnet18_checks(om, layers, run, batch: int = 32):
    """After the timed GPU legs: the graph replay's outputs against an eager
    pass's, bit for bit (every output is overwritten per pass), and two images
    of three layers kept for the CPU check."""
    forward, graph = run
    forward()
    eager_out = [d["y"].numpy() for _, d, _ in layers]
    graph.launch()
    om.synchronize()
    same = all(np.array_equal(d["y"].numpy().view(np.uint32), e.view(np.uint32))
               for (_, d, _), e in zip(layers, eager_out))
    graph.destroy()
    # outputs of two images of three layers, checked on the CPU
    samples = []
    for idx in RESNET18_CHECKED:   # images 0 and batch-1 only (the next leg starts with no long host gap)
        y = layers[idx][1]["y"]
        per_img = int(np.prod(y.shape[1:]))
        samples.append((idx, read_rows(om, y, [0, batch - 1], per_img).reshape((2,) + tuple(y.shape[1:]))))
    return samples, same


def bench_resnet18_net(om, steps: int, warmup: int, batch: int = 32):
    """The whole ResNet-18 at batch 32: fused inference forward, and one training
    step (forward with batch statistics + backward to every weight)."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    from resnet_net import GpuResNet18, forward_flops, make_params
    P = make_params(seed=1)
    img = syn.randn((batch, 3, 224, 224), 900)
    d_img = om.DeviceBuffer.from_numpy(img)
    timer = StreamTimer(om.stream_handle())
    net = GpuResNet18(om, P, batch)
    settle(om, lambda: net.forward(d_img))
    for _ in range(warmup):
        logits = net.forward(d_img)
    om.synchronize()
    timer.start()
    for _ in range(steps):
        net.forward(d_img)
    timer.stop()
    fwd_ms = timer.ms() / steps
    got = logits.numpy()[:2]
    # training step
    tnet = GpuResNet18(om, P, batch, train=True)
    g_logits = om.DeviceBuffer.from_numpy(syn.randn((batch, 1000), 901, 0.01))
    settle(om, lambda: (tnet.forward_train(d_img), tnet.backward(g_logits)))
    for _ in range(max(1, warmup // 2)):
        tnet.forward_train(d_img)
        tnet.backward(g_logits)
    om.synchronize()
    tsteps = max(3, steps // 2)
    timer.start()
    for _ in range(tsteps):
        tnet.forward_train(d_img)
        tnet.backward(g_logits)
    timer.stop()
    train_ms = timer.ms() / tsteps
    fl = forward_flops(batch)
    stem = 2.0 * batch * 64 * 112 * 112 * 3 * 49
    train_fl = 3.0 * fl - stem        # forward + input gradients (none for the image) + weight gradients
    # the last timed step's forward state and weight gradients, for the CPU check
    train_state = (tnet.forward_state(img), tnet.grads())
    return fwd_ms, fl, got, train_ms, train_fl, train_state


def bench_infer_pipeline(om, n_img: int = 512, batch: int = 32, reps: int = 3):
    """EngineBridge::inferBatch on this backend: n_img host images (pageable, float32 in
    [0, 1]) -> ImageNet normalisation, ResNet-18 forward, softmax / argmax per image, in
    batches of 32 with the upload of each batch overlapping the previous batch's compute.
    Also the device-resident forward alone, eager and replayed from a captured graph."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    from resnet_net import make_params, pack_params
    P = make_params(seed=1)
    net = om.ResNet18Infer(pack_params(P), 1000, batch)
    imgs = syn.uniform((n_img, 3, 224, 224), 905, 0.0, 1.0)
    net.infer_batch(imgs[:2 * batch], batch)        # warm-up: tables, workspaces, staging
    wall = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cls, conf, _ = net.infer_batch(imgs, batch, with_probs=False)
        wall.append(time.perf_counter() - t0)
    pipe_s = float(np.median(wall))
    # device-resident forward of one batch: eager, then a captured graph
    d_in = om.DeviceBuffer.from_numpy(syn.randn((batch, 3, 224, 224), 906))
    d_log = om.DeviceBuffer.empty((batch, 1000))
    timer = StreamTimer(om.stream_handle())
    steps = 20
    net.forward(d_in, d_log, batch)
    om.synchronize()
    timer.start()
    for _ in range(steps):
        net.forward(d_in, d_log, batch)
    timer.stop()
    eager_ms = timer.ms() / steps
    graph = om.Graph(lambda: net.forward(d_in, d_log, batch))
    graph.launch()
    om.synchronize()
    timer.start()
    for _ in range(steps):
        graph.launch()
    timer.stop()
    graph_ms = timer.ms() / steps
    return {"images": n_img, "batch": batch, "img_s": round(n_img / pipe_s, 1),
            "ms_per_batch": round(pipe_s / (n_img / batch) * 1e3, 4),
            "scope": "host float32 images (pageable) -> page-locked staging -> transfer stream -> ImageNet "
                     "normalisation -> ResNet-18 forward -> logits to the host -> softmax / argmax per image",
            "resident_forward": {"ms": round(eager_ms, 4), "img_s": round(batch / eager_ms * 1e3, 1)},
            "resident_forward_graph": {"ms": round(graph_ms, 4), "img_s": round(batch / graph_ms * 1e3, 1)},
            "host_link_bytes_per_batch": batch * 3 * 224 * 224 * 4}


def cpu_baseline_resnet18_net(n_img: int = 2, reps: int = 3):
    from resnet_net import cpu_forward, cpu_train_step, make_params
    import oracle as O
    kind = "reference" if O.ref_lib() is not None else "oracle"
    P = make_params(seed=1)
    img = O.randn((n_img, 3, 224, 224), 900)
    g = O.randn((n_img, 1000), 901, 0.01)
    cpu_forward(P, img, backend=kind)
    f, t = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        cpu_forward(P, img, backend=kind)
        f.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        cpu_train_step(P, img, g, backend=kind)
        t.append(time.perf_counter() - t0)
    return kind, n_img / float(np.median(f)), n_img / float(np.median(t)), float(np.median(f)), float(np.median(t))


RESNET50_CHECKED = (0, 26, 52)   # layers whose outputs (two images) are checked on the CPU


def resnet50_layer_inputs(li: int, batch: int):
    """Seeded input, Kaiming-uniform weight and BN vectors of ResNet-50 conv layer li."""
    from resnet_shapes import resnet50_convs
    name, cin, h, w, cout, k, s, p = resnet50_convs()[li]
    bnd = np.sqrt(6.0 / (cin * k * k))
    x = syn.randn((batch, cin, h, w), 700 + li)
    wt = syn.uniform((cout, cin, k, k), 800 + li, -bnd, bnd)
    bn = (syn.uniform((cout,), 900 + li, 0.5, 1.5), syn.randn((cout,), 1000 + li, 0.1),
          syn.randn((cout,), 1100 + li, 0.1), syn.uniform((cout,), 1200 + li, 0.5, 1.5))
    return x, wt, bn


def resnet50_setup(om, batch: int = 64):
    """The 53 ResNet-50 conv layers' seeded inputs, uploaded to HBM."""
    from resnet_shapes import out_hw, resnet50_convs
    layers = []
    for li, (name, cin, h, w, cout, k, s, p) in enumerate(resnet50_convs()):
        ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
        xh, wh, bnh = resnet50_layer_inputs(li, batch)
        x, wt = om.DeviceBuffer.from_numpy(xh), om.DeviceBuffer.from_numpy(wh)
        bn = [om.DeviceBuffer.from_numpy(a) for a in bnh]
        y = om.DeviceBuffer.empty((batch, cout, ho, wo))
        layers.append(((name, cin, h, w, cout, k, s, p), x, wt, bn, y))
    return layers


def resnet50_samples(om, layers, batch: int = 64):
    """Images 0 and batch-1 of the checked layers' outputs (every output is overwritten per pass)."""
    out = []
    for li in RESNET50_CHECKED:
        y = layers[li][4]
        per_img = int(np.prod(y.shape[1:]))
        out.append((li, read_rows(om, y, [0, batch - 1], per_img).reshape((2,) + tuple(y.shape[1:]))))
    return out


def bench_resnet50(om, layers, steps: int, warmup: int, batch: int = 64):
    """ResNet-50 conv stack forward (53 convs, fused conv+BN+ReLU) at batch 64."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    from resnet_shapes import conv_bytes, conv_flops
    H = om.HIPBackend

    def forward():
        for (name, cin, h, w, cout, k, s, p), x, wt, bn, y in layers:
            H.conv2dBiasBnAct(x, wt, None, bn[0], bn[1], bn[2], bn[3], 1e-5, 1, y, batch, cin, h, w, cout, k, k, s, p)

    for _ in range(warmup):
        forward()
    om.synchronize()
    timer = StreamTimer(om.stream_handle())
    timer.start()
    for _ in range(steps):
        forward()
    timer.stop()
    ms = timer.ms() / steps
    flops = sum(conv_flops(sh, batch) for sh, *_ in layers)
    roof_ms = sum(max(conv_flops(sh, batch) / PEAK_FP32, conv_bytes(sh, batch) / PEAK_HBM) for sh, *_ in layers) * 1e3
    return ms, flops, roof_ms


def vit_gemm_shapes(batch: int = 64, tokens: int = 197, d: int = 768, heads: int = 12, proj_nt: bool = False):
    """(name, batch, M, N, K, transB) of the ViT-B/16 GEMMs: the projections x[T,in] x W
    with W stored [in, out] as the reference's Linear keeps it (linear.ixx:31, :52; NN), or
    with proj_nt W stored [out, in] (NT); attention Q.K^T (transB) and P.V."""
    T = batch * tokens
    dh = d // heads
    return [("qkv", 1, T, 3 * d, d, proj_nt), ("out_proj", 1, T, d, d, proj_nt), ("fc1", 1, T, 4 * d, d, proj_nt),
            ("fc2", 1, T, d, 4 * d, proj_nt), ("qk_t", batch * heads, tokens, tokens, dh, True),
            ("pv", batch * heads, tokens, dh, tokens, False)]


def bench_vit_half(om, steps: int, warmup: int, bf16: bool, proj_nt: bool = False):
    """The ViT-B/16 GEMM set (batch 64, 197 tokens) with fp16 / bf16 inputs, fp32 accumulate,
    projections in the NN (reference) or NT weight layout. With NN, also the fused attention
    and the whole attention layer (MultiHeadAttention::forward: QKV Linear with bias, fused
    attention, output Linear with bias)."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    H = om.HIPBackend
    dt = 1 if bf16 else 0
    bufs = []
    rng = np.random.default_rng(5)
    for name, b, m, n, k, tb in vit_gemm_shapes(proj_nt=proj_nt):
        a = rng.standard_normal(b * m * k, dtype=np.float32)
        w = (rng.standard_normal(b * n * k, dtype=np.float32) * (0.02 if b == 1 else 1.0)).astype(np.float32)
        da, dw = om.DeviceBuffer.from_numpy(a), om.DeviceBuffer.from_numpy(w)
        ha, hw = om.DeviceBuffer.empty((a.size,), np.uint16), om.DeviceBuffer.empty((w.size,), np.uint16)
        H.convertToHalf(da, ha, a.size, bf16=bf16)
        H.convertToHalf(dw, hw, w.size, bf16=bf16)
        c = om.DeviceBuffer.empty((b * m * n,))
        bufs.append((name, b, m, n, k, tb, ha, hw, c))

    def run(item):
        name, b, m, n, k, tb, ha, hw, c = item
        H.gemmStridedBatchedHalf(dt, 0, tb, b, m, n, k, ha, k, m * k, hw, k if tb else n, n * k, c, n, m * n)

    per = []
    total_ms = 0.0
    flops_total = 0.0
    settle(om, lambda: [run(item) for item in bufs])
    for item in bufs:
        for _ in range(warmup):
            run(item)
        om.synchronize()
        t = StreamTimer(om.stream_handle())
        t.start()
        for _ in range(steps):
            run(item)
        t.stop()
        ms = t.ms() / steps
        name, b, m, n, k = item[:5]
        f = 2.0 * b * m * n * k
        flops_total += f
        total_ms += ms
        per.append({"gemm": name, "shape": [b, m, n, k], "ms": round(ms, 4), "tflops": round(f / ms / 1e9, 1)})
    # sampled outputs for the CPU check: rows 0, M/2, M-1 of a projection, the first and last
    # batch of an attention product (each launch overwrites its whole C)
    samples = {}
    for name, b, m, n, k, tb, ha, hw, c in bufs:
        if b == 1:
            rows = [0, m // 2, m - 1]
            samples[name] = (rows, read_rows(om, c, rows, n))
        else:
            samples[name] = ([0, b - 1], read_rows(om, c, [0, b - 1], m * n).reshape(2, m, n))
    if proj_nt:
        return total_ms, flops_total, per, None, None, samples
    # Fused attention on the QKV projection's output layout [T, 3*768] (split + softmax(QK^T/8) V + merge),
    # replacing the two batched products above plus the softmax between them.
    batch, tokens, heads, dh = 64, 197, 12, 64
    T = batch * tokens
    qkv = om.DeviceBuffer.empty((T * 3 * heads * dh,), np.uint16)
    src = om.DeviceBuffer.from_numpy((rng.standard_normal(T * 3 * heads * dh, dtype=np.float32) * 0.5))
    H.convertToHalf(src, qkv, T * 3 * heads * dh, bf16=bf16)
    ctx = om.DeviceBuffer.empty((T * heads * dh,), np.uint16)
    settle(om, lambda: H.attentionHalf(qkv, ctx, batch, tokens, heads, dh, 0.125, bf16=bf16, outHalf=True))
    for _ in range(warmup):
        H.attentionHalf(qkv, ctx, batch, tokens, heads, dh, 0.125, bf16=bf16, outHalf=True)
    om.synchronize()
    t = StreamTimer(om.stream_handle())
    t.start()
    for _ in range(steps):
        H.attentionHalf(qkv, ctx, batch, tokens, heads, dh, 0.125, bf16=bf16, outHalf=True)
    t.stop()
    attn_ms = t.ms() / steps
    attn_bytes = 2.0 * T * 3 * heads * dh + 2.0 * T * heads * dh   # qkv read + context written (half)
    attn_flops = 4.0 * batch * heads * tokens * tokens * dh
    fused = {"op": "attention_fused", "shape": [batch, tokens, heads, dh], "ms": round(attn_ms, 4),
             "hbm_gb_s": round(attn_bytes / attn_ms / 1e6, 1), "frac_of_8000_gb_s": round(attn_bytes / attn_ms / 8e9, 4),
             "tflops": round(attn_flops / attn_ms / 1e9, 1),
             "replaces_ms": round(sum(x["ms"] for x in per if x["gemm"] in ("qk_t", "pv")), 4)}
    # The whole attention layer: x [T, 768] half -> out [T, 768] fp32 (three launches).
    d = heads * dh
    x = om.DeviceBuffer.empty((T * d,), np.uint16)
    H.convertToHalf(om.DeviceBuffer.from_numpy(rng.standard_normal(T * d, dtype=np.float32)), x, T * d, bf16=bf16)
    wq = om.DeviceBuffer.empty((d * 3 * d,), np.uint16)
    H.convertToHalf(om.DeviceBuffer.from_numpy(rng.standard_normal(d * 3 * d, dtype=np.float32) * 0.036), wq,
                    d * 3 * d, bf16=bf16)
    wo = om.DeviceBuffer.empty((d * d,), np.uint16)
    H.convertToHalf(om.DeviceBuffer.from_numpy(rng.standard_normal(d * d, dtype=np.float32) * 0.036), wo, d * d,
                    bf16=bf16)
    bq = om.DeviceBuffer.from_numpy(rng.standard_normal(3 * d, dtype=np.float32) * 0.1)
    bo = om.DeviceBuffer.from_numpy(rng.standard_normal(d, dtype=np.float32) * 0.1)
    y = om.DeviceBuffer.empty((T * d,))

    def layer():
        H.multiHeadAttentionHalf(x, wq, bq, wo, bo, y, batch, tokens, heads, dh, bf16=bf16)

    settle(om, layer)
    for _ in range(warmup):
        layer()
    om.synchronize()
    t = StreamTimer(om.stream_handle())
    t.start()
    for _ in range(steps):
        layer()
    t.stop()
    mha_ms = t.ms() / steps
    mha_flops = 2.0 * T * d * 3 * d + attn_flops + 2.0 * T * d * d
    mha = {"op": "multi_head_attention_forward", "shape": [batch, tokens, heads, dh], "ms": round(mha_ms, 4),
           "tflops": round(mha_flops / mha_ms / 1e9, 1),
           "launches": "QKV Linear (+bias, half out) -> fused attention (half out) -> output Linear (+bias, fp32 out)"}
    # images 0 and 63 of the fused attention's context (half) and of the layer's output
    imgs = [0, batch - 1]
    samples["attention_fused"] = (imgs, read_rows(om, ctx, imgs, tokens * d, np.uint16).reshape(2, tokens, d))
    samples["attention_layer"] = (imgs, read_rows(om, y, imgs, tokens * d).reshape(2, tokens, d))
    return total_ms, flops_total, per, fused, mha, samples


def bench_mlp(om, steps: int, warmup: int, batch: int = 128):
    """MLP 784-256-128-10 (ReLU) training step, fp32, batch 128, labels uniform in 0..9:
    each hidden Linear (+ ReLU) is one fused launch; the classifier head — its Linear,
    softmax, cross-entropy and their backward (dW, db, dA gated by the ReLU below) — one
    launch (omHipLinearSoftmaxCrossEntropyStep); each hidden layer's backward one launch
    (omHipLinearBackward: the reference's TN / NT products for dW and dA, the bias gradient
    of AddBiasBackward and the ReLU gate of the layer below, each element equal to the
    separate entries'). Five launches. No optimizer update."""
    from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
    H = om.HIPBackend
    dims = [784, 256, 128, 10]
    x = om.DeviceBuffer.from_numpy(syn.uniform((batch, 784), 1))
    labels = syn.rng(2).integers(0, 10, batch)
    T = om.DeviceBuffer.from_numpy(np.eye(10, dtype=np.float32)[labels])
    Ws = [om.DeviceBuffer.from_numpy(syn.uniform((i, o), 10 + j, -np.sqrt(6 / i), np.sqrt(6 / i)))
          for j, (i, o) in enumerate(zip(dims[:-1], dims[1:]))]
    bs = [om.DeviceBuffer.from_numpy(np.zeros(o, np.float32)) for o in dims[1:]]
    z = [om.DeviceBuffer.empty((batch, o)) for o in dims[1:]]
    a = [x] + [om.DeviceBuffer.empty((batch, o)) for o in dims[1:-1]]
    g = [om.DeviceBuffer.empty((batch, o)) for o in dims[1:]]
    gA = [om.DeviceBuffer.empty((batch, i)) for i in dims[:-1]]
    gW = [om.DeviceBuffer.empty((i, o)) for i, o in zip(dims[:-1], dims[1:])]
    gb = [om.DeviceBuffer.empty((o,)) for o in dims[1:]]
    loss = om.DeviceBuffer.empty((1,))

    def step():
        # forward of the hidden layers: one fused launch per layer, act(x W + b), keeping
        # only the activation, whose sign is the ReLU gate of the backward
        for j in range(2):
            i, o = dims[j], dims[j + 1]
            H.linearBiasAct(a[j], Ws[j], bs[j], a[j + 1], batch, i, o, 1)
        # the classifier head in one launch: logits, softmax + cross-entropy, (p - t) / batch,
        # the head's dW, db and dA gated by the ReLU output below it
        H.linearSoftmaxCrossEntropyStep(a[2], Ws[2], bs[2], T, a[2], z[2], loss, g[2], gW[2], gb[2], g[1], batch,
                                        dims[2], dims[3])
        for j in reversed(range(2)):
            i, o = dims[j], dims[j + 1]
            # dW = A^T G, db = column sums of G, dA = G W^T (as the reference, every layer);
            # above the first layer dA goes through the ReLU gate below it (a > 0 exactly
            # where x W + b > 0) straight into that layer's output gradient
            H.linearBackward(a[j], g[j], Ws[j], a[j] if j > 0 else None, gW[j], gb[j],
                             g[j - 1] if j > 0 else gA[0], batch, i, o)

    settle(om, step)
    for _ in range(warmup):
        step()
    om.synchronize()
    t = StreamTimer(om.stream_handle())
    t.start()
    for _ in range(steps):
        step()
    t.stop()
    ms = t.ms() / steps
    # The same step replayed from a captured graph (its kernels unchanged; the
    # per-launch host cost is gone). Every output is overwritten per step, so
    # the replay's results must equal the eager step's bit for bit.
    outs = gW + [gA[0]] + g + gb + [loss]
    eager_out = [d.numpy().copy() for d in outs]
    graph = om.Graph(step)
    graph.launch()
    om.synchronize()
    same = all(np.array_equal(d.numpy(), e) for d, e in zip(outs, eager_out))
    t.start()
    for _ in range(steps):
        graph.launch()
    t.stop()
    graph_ms = t.ms() / steps
    flops = sum(3 * 2.0 * batch * i * o for i, o in zip(dims[:-1], dims[1:]))
    # the step's state for the CPU check (every buffer is rewritten each step)
    state = {"a": [a[j].numpy() for j in (1, 2)], "z3": z[2].numpy(), "g": [d.numpy() for d in g],
             "gW": [d.numpy() for d in gW], "gb": [d.numpy() for d in gb], "gA0": gA[0].numpy(),
             "loss": float(eager_out[-1][0]), "labels": labels}
    return ms, flops, graph_ms, same, float(eager_out[-1][0]), state


# ---- CPU checks of the GPU legs' results (run with the CPU baseline leg) ----
# Each regenerates its leg's seeded inputs and compares the sampled GPU outputs
# with the oracle's float64 result under the K-scaled bound.

def cpu_check_gemm(c_rows) -> float:
    import oracle as O
    A, B = syn.randn((M, K), 11), syn.randn((K, N), 12)
    C64, bound = O.gemm_f64(A[GEMM_ROWS], B)
    return O.normalized_error(c_rows, C64, bound)


def cpu_check_sweep(sweep: list, samples: list) -> None:
    import oracle as O
    for entry, ((m, n, k, layout), rows, c_rows) in zip(sweep, samples):
        A = syn.randn((m, k), 21 + m)
        B = syn.randn((k, n) if layout == "NN" else (n, k), 22 + n)
        C64, bound = O.gemm_f64(A[rows], B, transB=(layout == "NT"))
        entry["parity"] = O.normalized_error(c_rows, C64, bound)


def cpu_check_resnet18(samples: list, batch: int = 32) -> float:
    import oracle as O
    from resnet_shapes import resnet18_convs
    errs = []
    for li, y in samples:
        name, cin, h, w, cout, k, s, p = resnet18_convs()[li]
        x, wt, g, b, m, v = resnet18_layer_inputs(li, batch)
        o64, bound = O.conv_f64(x[[0, batch - 1]], wt, None, s, p, gamma=g, beta=b, mean=m, var=v, act=1)
        errs.append(O.normalized_error(y, o64, bound))
    return max(errs)


def cpu_check_resnet50(samples: list, batch: int = 64) -> float:
    import oracle as O
    from resnet_shapes import resnet50_convs
    errs = []
    for li, y in samples:
        name, cin, h, w, cout, k, s, p = resnet50_convs()[li]
        x, wt, (g, b, m, v) = resnet50_layer_inputs(li, batch)
        o64, bound = O.conv_f64(x[[0, batch - 1]], wt, None, s, p, gamma=g, beta=b, mean=m, var=v, act=1)
        errs.append(O.normalized_error(y, o64, bound))
    return max(errs)


def _half_round(x, bf16: bool) -> np.ndarray:
    import oracle as O
    return O.bf16_round(x) if bf16 else np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def cpu_check_vit(vit_samples: dict) -> dict:
    """The ViT legs' sampled outputs against float64 on the same rounded inputs (the seeded
    draws of bench_vit_half regenerated in the same order): projection rows and attention
    product batches K-scaled (bar 1e-4: fp32 accumulate of exact half products), the fused
    attention's half context per element against sum_j P_ij |V_jd| (bar 2e-3 fp16, 1.2e-2
    bf16) and the attention layer's output against ((B_ctx + |ctx|) |W_out| + |b_out|)
    (bar 2u + 1e-4, u = 2^-11 fp16, 2^-8 bf16)."""
    import oracle as O
    rng = np.random.default_rng(5)
    draws = []
    for name, b, m, n, k, tb in vit_gemm_shapes():
        a = rng.standard_normal(b * m * k, dtype=np.float32)
        w = (rng.standard_normal(b * n * k, dtype=np.float32) * (0.02 if b == 1 else 1.0)).astype(np.float32)
        draws.append((name, b, m, n, k, a, w))
    batch, tokens, heads, dh = 64, 197, 12, 64
    T, d = batch * tokens, heads * dh
    qkv = (rng.standard_normal(T * 3 * d, dtype=np.float32) * 0.5)
    x = rng.standard_normal(T * d, dtype=np.float32)
    wq = rng.standard_normal(d * 3 * d, dtype=np.float32) * 0.036
    wo = rng.standard_normal(d * d, dtype=np.float32) * 0.036
    bq = rng.standard_normal(3 * d, dtype=np.float32) * 0.1
    bo = rng.standard_normal(d, dtype=np.float32) * 0.1
    out = {}
    for bf, (nn_smp, nt_smp) in vit_samples.items():
        tag = "bf16" if bf else "fp16"
        worst = 0.0
        for layout, smp in (("NN", nn_smp), ("NT", nt_smp)):
            for name, b, m, n, k, a, w in draws:
                picks, got = smp[name]
                ar, wr = _half_round(a, bf).reshape(b, m, k), _half_round(w, bf)
                tb = name == "qk_t" or (layout == "NT" and b == 1)
                wr = wr.reshape(b, n, k) if tb else wr.reshape(b, k, n)
                for i, pk in enumerate(picks):
                    if b == 1:
                        A, W, g = ar[0][[pk]], wr[0], got[i][None, :]
                    else:
                        A, W, g = ar[pk], wr[pk], got[i]
                    C64, bound = O.gemm_f64(A, W, transB=tb)
                    worst = max(worst, O.normalized_error(g, C64, bound))
        out[tag + "_gemms_max_err"] = worst
        # fused attention (half context) and the attention layer, images 0 and 63
        imgs, ctx = nn_smp["attention_fused"]
        ctx = (ctx.astype(np.uint32) << 16).view(np.float32) if bf else ctx.view(np.float16).astype(np.float32)
        qr = _half_round(qkv, bf).reshape(batch, tokens, 3 * d)
        e = 0.0
        for i, img in enumerate(imgs):
            ref64, bnd = O.attention_f64(qr[img], 1, tokens, heads, dh, 0.125)
            e = max(e, O.normalized_error(ctx[i], ref64, bnd))
        out[tag + "_attention_fused_err"] = e
        _, y = nn_smp["attention_layer"]
        xr = _half_round(x, bf).reshape(batch, tokens, d)
        wqr, wor = _half_round(wq, bf).reshape(d, 3 * d).astype(np.float64), _half_round(wo, bf).reshape(d, d).astype(np.float64)
        scale = float(np.float32(1.0 / np.sqrt(np.float32(dh))))
        e = 0.0
        for i, img in enumerate(imgs):
            q64 = xr[img].astype(np.float64) @ wqr + bq.astype(np.float64)
            ctx64, bctx = O.attention_f64(_half_round(q64.astype(np.float32), bf), 1, tokens, heads, dh, scale)
            o64 = ctx64 @ wor + bo.astype(np.float64)
            bnd = (bctx + np.abs(ctx64)) @ np.abs(wor) + np.abs(bo.astype(np.float64))
            e = max(e, O.normalized_error(y[i], o64, bnd))
        out[tag + "_attention_layer_err"] = e
    return out


def cpu_check_mlp(st: dict, batch: int = 128) -> dict:
    """The MLP step layer by layer in float64 on the GPU's own inputs to each op (so a ReLU
    input within rounding of 0 takes the GPU's side): each layer's output and each gradient
    K-scaled (bar 1e-4), the loss against the oracle's softmax + cross-entropy of the GPU
    logits (relative 1e-5) and the logit gradient (p - t) / batch (relative Frobenius 1e-5)."""
    import oracle as O
    dims = [784, 256, 128, 10]
    x = syn.uniform((batch, 784), 1).astype(np.float64)
    Ws = [syn.uniform((i, o), 10 + j, -np.sqrt(6 / i), np.sqrt(6 / i)).astype(np.float64)
          for j, (i, o) in enumerate(zip(dims[:-1], dims[1:]))]
    T = np.eye(10, dtype=np.float32)[st["labels"]]
    acts = [x] + [a.astype(np.float64) for a in st["a"]]
    errs = []
    for j in range(3):                       # act(a_j W_j + 0), biases are zero
        ref = acts[j] @ Ws[j]
        bound = np.abs(acts[j]) @ np.abs(Ws[j])
        got = st["a"][j] if j < 2 else st["z3"]
        errs.append(O.normalized_error(got, np.maximum(ref, 0) if j < 2 else ref, bound))
    p = O.softmax(st["z3"])
    loss_err = abs(st["loss"] - O.cross_entropy(p, T)) / abs(st["loss"])
    glogit_err = O.frobenius_rel(st["g"][2], O.cross_entropy_softmax_backward(p, T))
    for j in range(3):
        g = st["g"][j].astype(np.float64)
        errs.append(O.normalized_error(st["gW"][j], acts[j].T @ g, np.abs(acts[j]).T @ np.abs(g)))
        errs.append(O.normalized_error(st["gb"][j], g.sum(axis=0), np.abs(g).sum(axis=0)))
        dA = g @ Ws[j].T
        bound = np.abs(g) @ np.abs(Ws[j]).T
        if j > 0:
            gate = st["a"][j - 1] > 0
            errs.append(O.normalized_error(st["g"][j - 1], np.where(gate, dA, 0.0), bound))
        else:
            errs.append(O.normalized_error(st["gA0"], dA, bound))
    return {"layers_and_gradients_max_err": max(errs), "loss_rel_err": loss_err, "grad_logits_rel_err": glogit_err}


def cpu_check_resnet18_train(state) -> dict:
    """The timed b32 training step: each forward op against the CPU op on the GPU's own input
    to it (relative Frobenius, bar 1e-4), and every weight gradient against the reference
    backward replayed on the GPU's forward state (bar 1e-3)."""
    import oracle as O
    from resnet_net import conv_list, cpu_backward, cpu_forward_local, make_params
    f, grads = state
    P = make_params(seed=1)
    g_logits = syn.randn((32, 1000), 901, 0.01)
    local = cpu_forward_local(P, f)
    op_err = max(O.frobenius_rel(f[k].reshape(v.shape), v) for k, v in local.items())
    del local
    ref = cpu_backward(P, f, g_logits)
    g_err = max(O.frobenius_rel(grads[n].reshape(ref[n].shape), ref[n])
                for n in [c for c, *_ in conv_list()] + ["fc.w", "fc.b"])
    return {"forward_ops_max_rel_err": op_err, "weight_grads_max_rel_err": g_err}


def cpu_check_resnet18_net(logits2) -> float:
    import oracle as O
    from resnet_net import cpu_forward, make_params
    img2 = syn.randn((32, 3, 224, 224), 900)[:2]
    return O.frobenius_rel(logits2, cpu_forward(make_params(seed=1), img2))


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


def cpu_baseline_resnet50(n_img: int = 2):
    """Reference conv2d -> batchNorm2d(eval) -> relu over the 53 ResNet-50 convs, n_img images (one pass)."""
    import oracle as O
    from resnet_shapes import resnet50_convs
    backend = "reference" if O.ref_lib() is not None else "oracle"
    t_total = 0.0
    for li, (name, cin, h, w, cout, k, s, p) in enumerate(resnet50_convs()):
        x, wt = O.randn((n_img, cin, h, w), 700 + li), O.randn((cout, cin, k, k), 800 + li, 0.05)
        g, b = O.uniform((cout,), 900 + li, 0.5, 1.5), O.randn((cout,), 1000 + li, 0.1)
        m, v = O.randn((cout,), 1100 + li, 0.1), O.uniform((cout,), 1200 + li, 0.5, 1.5)
        t = time.perf_counter()
        y = O.conv2d(x, wt, None, s, p, backend=backend)
        y, _, _ = O.batchnorm2d_eval(y, g, b, m, v, backend=backend)
        O.relu(y, backend=backend)
        t_total += time.perf_counter() - t
    return backend, n_img / t_total, t_total


def cpu_baseline_vit():
    """Reference matmul / batchedMatmul (+ transpose2d for the B^T operands) on one image's
    share of the ViT GEMM set (197 tokens), fp32 on fp16-rounded inputs."""
    import oracle as O
    backend = "reference" if O.ref_lib() is not None else "oracle"
    flops = 0.0
    t_total = 0.0
    for name, b, m, n, k, tb in vit_gemm_shapes(batch=1):
        a = O.randn((b, m, k), 1).astype(np.float16).astype(np.float32)
        w = O.randn((b, n, k) if tb else (b, k, n), 2).astype(np.float16).astype(np.float32)
        t = time.perf_counter()
        for i in range(b):
            wi = O.transpose2d(w[i], backend=backend) if tb else w[i]
            O.matmul(a[i], wi, backend=backend)
        t_total += time.perf_counter() - t
        flops += 2.0 * b * m * n * k
    return backend, flops / t_total / 1e12, t_total


def cpu_baseline_mlp(reps: int = 20):
    """The MLP fwd+bwd step as the reference computes it (matmul, addBias, relu;
    MatMulBackward's explicit transposes + matmul for dA and dW on every layer)."""
    import oracle as O
    backend = "reference" if O.ref_lib() is not None else "oracle"
    dims = [784, 256, 128, 10]
    x = O.uniform((128, 784), 1)
    Ws = [O.uniform((i, o), 10 + j, -0.1, 0.1) for j, (i, o) in enumerate(zip(dims[:-1], dims[1:]))]
    T = np.eye(10, dtype=np.float32)[O.rng(2).integers(0, 10, 128)]

    def step():
        acts, pre = [x], []
        for j, W in enumerate(Ws):
            z = O.add_bias(O.matmul(acts[-1], W, backend=backend), np.zeros(W.shape[1], np.float32), backend=backend)
            pre.append(z)
            if j < 2:
                acts.append(O.relu(z, backend=backend))
        p = O.softmax(pre[-1], backend=backend)
        O.cross_entropy(p, T, backend=backend)
        g = O.cross_entropy_softmax_backward(p, T, backend=backend)
        for j in reversed(range(3)):
            O.matmul(O.transpose2d(acts[j], backend=backend), g, backend=backend)
            O.add_bias_backward(g, g.shape[0], g.shape[1])
            gA = O.matmul(g, O.transpose2d(Ws[j], backend=backend), backend=backend)
            if j > 0:
                g = O.relu_backward(pre[j - 1], gA, backend=backend)

    step()
    t = time.perf_counter()
    for _ in range(reps):
        step()
    dt = (time.perf_counter() - t) / reps
    return backend, dt * 1e3


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


def workload_probe(name: str):
    """A short dispatch sequence for kernel-trace profiling (no JSON):
    resnet18_train — three ResNet-18 b32 training steps; vit_attention — ten fused
    attentions (ViT-B/16 b64, fp16) after the ten Q.K^T / P.V batched products they replace;
    vit_gemms — each ViT-B/16 b64 GEMM (fp16, fp32 output) three times;
    half_power — the fp16 GEMM on constant and on random operands (same kernel and shape);
    mlp — thirty MLP 784-256-128-10 b128 training steps after five untimed ones."""
    import omnimatchdeeplearningtool_amd as om
    om.init(0)
    H = om.HIPBackend
    if name == "resnet18_train":
        from resnet_net import GpuResNet18, make_params
        img = om.DeviceBuffer.from_numpy(syn.randn((32, 3, 224, 224), 900))
        g = om.DeviceBuffer.from_numpy(syn.randn((32, 1000), 901, 0.01))
        net = GpuResNet18(om, make_params(seed=1), 32, train=True)
        for _ in range(3):
            net.forward_train(img)
            net.backward(g)
    elif name == "vit_attention":
        T, S, heads, dh, b = 64 * 197, 197, 12, 64, 64
        src = om.DeviceBuffer.from_numpy(syn.randn((T * 3 * heads * dh,), 5, 0.5))
        qkv = om.DeviceBuffer.empty((T * 3 * heads * dh,), np.uint16)
        H.convertToHalf(src, qkv, T * 3 * heads * dh)
        ctx = om.DeviceBuffer.empty((T * heads * dh,), np.uint16)
        q = om.DeviceBuffer.empty((b * heads * S * dh,), np.uint16)
        sc = om.DeviceBuffer.empty((b * heads * S * S,))
        pv = om.DeviceBuffer.empty((b * heads * S * dh,))
        p16 = om.DeviceBuffer.empty((b * heads * S * S,), np.uint16)
        for _ in range(10):
            H.gemmStridedBatchedHalf(0, 0, 1, b * heads, S, S, dh, q, dh, S * dh, q, dh, S * dh, sc, S, S * S)
            H.gemmStridedBatchedHalf(0, 0, 0, b * heads, S, dh, S, p16, S, S * S, q, dh, S * dh, pv, dh, S * dh)
        for _ in range(10):
            H.attentionHalf(qkv, ctx, b, S, heads, dh, 0.125, outHalf=True)
    elif name == "vit_gemms":
        # A 256 MiB device copy (the calibration of the traffic counters), then the ViT-B/16
        # b64 GEMM set (fp16 inputs, fp32 output, projections NN), each GEMM three times after
        # a 30 ms warm-up of the whole set, one after another.
        n = 64 << 20
        src, dst = om.DeviceBuffer.empty((n,)), om.DeviceBuffer.empty((n,))
        H.fillValue(src, n, 1.0)
        om.synchronize()
        H.copy(src, dst, n)
        om.synchronize()
        src.free(); dst.free()
        bufs = []
        for gname, b, m, n, k, tb in vit_gemm_shapes():
            a = om.DeviceBuffer.from_numpy(syn.randn((b * m * k,), 31))
            w = om.DeviceBuffer.from_numpy(syn.randn((b * n * k,), 32, 0.02 if b == 1 else 1.0))
            ha, hw = om.DeviceBuffer.empty((b * m * k,), np.uint16), om.DeviceBuffer.empty((b * n * k,), np.uint16)
            H.convertToHalf(a, ha, b * m * k)
            H.convertToHalf(w, hw, b * n * k)
            a.free(); w.free()
            bufs.append((gname, b, m, n, k, tb, ha, hw, om.DeviceBuffer.empty((b * m * n,))))
        run = lambda it: H.gemmStridedBatchedHalf(0, 0, it[5], it[1], it[2], it[3], it[4], it[6], it[4], it[2] * it[4],
                                                  it[7], it[4] if it[5] else it[3], it[3] * it[4], it[8], it[3],
                                                  it[2] * it[3])
        settle(om, lambda: [run(it) for it in bufs])
        for it in bufs:
            for _ in range(3):
                run(it)
            om.synchronize()
            log(f"vit_gemms {it[0]} done")
    elif name == "half_power":
        # One kernel and one shape (fp16 NT 8192^3, A times its own transpose), two
        # operand sets: every element 1.0, and N(0,1). The instruction stream is the
        # same; only the bit activity of the data differs. Blocks of ten launches
        # alternate after a warm-up so the clock ramp of an idle GPU is not counted.
        from omnimatchdeeplearningtool_amd.hiptime import StreamTimer
        n = 8192
        sets = {}
        for tag, host in (("ones", np.ones(n * n, np.float32)), ("randn", syn.randn((n * n,), 11))):
            src = om.DeviceBuffer.from_numpy(host)
            sets[tag] = om.DeviceBuffer.empty((n * n,), np.uint16)
            H.convertToHalf(src, sets[tag], n * n)
            src.free()
        c = om.DeviceBuffer.empty((n * n,))
        run = lambda a: H.gemmStridedBatchedHalf(0, 0, 1, 1, n, n, n, a, n, 0, a, n, 0, c, n, 0)
        for _ in range(20):
            run(sets["randn"])
        om.synchronize()
        for tag in ("ones", "randn", "ones", "randn"):
            t = StreamTimer(om.stream_handle())
            t.start()
            for _ in range(10):
                run(sets[tag])
            t.stop()
            ms = t.ms() / 10
            log(f"half_power {tag}: {ms * 1e3:.1f} us per launch, {2.0 * n ** 3 / ms / 1e9:.0f} TFLOP/s")
    elif name == "mlp":
        ms = bench_mlp(om, 30, 5)[0]
        log(f"mlp step {ms * 1e3:.1f} us")
    else:
        raise SystemExit(f"unknown probe {name}")
    om.synchronize()
    log(f"probe {name} done")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--probe", choices=["resnet18_train", "vit_attention", "half_power", "vit_gemms", "mlp"],
                    help="run only a short dispatch sequence for kernel-trace profiling (no JSON line)")
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
    if args.probe:
        workload_probe(args.probe)
        return

    import omnimatchdeeplearningtool_amd as om
    om.init(0)
    dev = om.device_name(0)
    log(f"device {dev}")

    # The headline GEMM is timed right after the sweep (whose last shapes are
    # the 8192^3 products), and the two conv stacks right after it, all inputs
    # uploaded before the sweep: an MI355X that has been idle needs about 20
    # ms of load before its clocks settle (4096^3 with 5 warm-up launches after
    # 0.5 s idle: 129-132 TFLOP/s; after 30 ms of other GEMMs, or with 25
    # warm-up launches: 140), and host work between the legs (generating the
    # next leg's inputs) would leave it idle again.
    gemm_bufs = gemm_inputs(om)
    r18_layers = resnet18_setup(om, 32)
    r50_layers = resnet50_setup(om, 64)
    sweep, sweep_samples = bench_gemm_sweep(om, args.steps, 2)

    log(f"gemm 4096^3 NN: warmup {args.warmup}, steps {args.steps} (timed right after the sweep)")
    ms, flops, wall, gemm_rows = bench_gemm(om, gemm_bufs, args.steps, args.warmup)
    tflops = flops / ms / 1e9
    log(f"gemm {ms:.4f} ms/step  {tflops:.1f} TFLOP/s")

    log("resnet18 conv stack b32")
    r_steps = max(5, args.steps // 2)
    r_ms, r_flops, r_roof_ms, per, r_graph_ms, r18_run = bench_resnet18(om, r18_layers, r_steps, max(2, args.warmup))
    img_s = 32.0 / (r_ms / 1e3)
    log(f"resnet18 {r_ms:.3f} ms/batch  {img_s:.0f} img/s  roof frac {r_roof_ms / r_ms:.3f}; graph replay "
        f"{r_graph_ms:.3f} ms, roof frac {r_roof_ms / r_graph_ms:.3f}")

    log("resnet50 conv stack b64")
    r50_ms, r50_flops, r50_roof = bench_resnet50(om, r50_layers, max(3, args.steps // 10), 1)
    log(f"resnet50 {r50_ms:.3f} ms/batch  {64 / r50_ms * 1e3:.0f} img/s  roof frac {r50_roof / r50_ms:.3f}")
    r50_samples = resnet50_samples(om, r50_layers)
    del r50_layers
    conv_samples, r_graph_same = resnet18_checks(om, r18_layers, r18_run)
    log(f"resnet18 graph replay bit-identical to eager: {r_graph_same}")

    log("resnet18 network b32 (inference forward, training step)")
    n_fwd_ms, n_fl, n_logits2, n_train_ms, n_train_fl, n_train_state = bench_resnet18_net(om, max(5, args.steps // 5), 2)
    log(f"resnet18 net forward {n_fwd_ms:.3f} ms  {32 / n_fwd_ms * 1e3:.0f} img/s; "
        f"train step {n_train_ms:.3f} ms  {32 / n_train_ms * 1e3:.0f} img/s")

    log("resnet18 inferBatch pipeline (host images -> classes)")
    infer = bench_infer_pipeline(om)
    log(f"inferBatch {infer['img_s']:.0f} img/s end to end; resident forward {infer['resident_forward']['ms']:.3f} ms, "
        f"graph replay {infer['resident_forward_graph']['ms']:.3f} ms")

    vit = {}
    vit_samples = {}
    for bf in (False, True):
        v_ms, v_flops, v_per, v_fused, v_mha, v_smp = bench_vit_half(om, max(5, args.steps // 5), 2, bf)
        t_ms, t_flops, t_per, _, _, t_smp = bench_vit_half(om, max(5, args.steps // 5), 2, bf, proj_nt=True)
        vit_samples[bf] = (v_smp, t_smp)
        lin_ms = sum(x["ms"] for x in v_per if x["gemm"] not in ("qk_t", "pv"))
        vit["bf16" if bf else "fp16"] = {"layout": "projections NN: W stored [in, out] as Linear keeps it",
                                         "ms_per_set": round(v_ms, 4), "tflops": round(v_flops / v_ms / 1e9, 1),
                                         "frac_of_2516_tflops": round(v_flops / v_ms / 1e9 / 2516.6, 4), "gemms": v_per,
                                         "nt": {"ms_per_set": round(t_ms, 4), "tflops": round(t_flops / t_ms / 1e9, 1),
                                                "frac_of_2516_tflops": round(t_flops / t_ms / 1e9 / 2516.6, 4),
                                                "gemms": t_per},
                                         "attention_fused": v_fused,
                                         "ms_per_layer_fused": round(lin_ms + v_fused["ms"], 4),
                                         "attention_layer": v_mha}
        log(f"vit {'bf16' if bf else 'fp16'} NN {v_ms:.3f} ms  {v_flops / v_ms / 1e9:.1f} TFLOP/s (NT {t_ms:.3f} ms "
            f"{t_flops / t_ms / 1e9:.1f}); fused attention {v_fused['ms'] * 1e3:.1f} us ({v_fused['hbm_gb_s']:.0f} GB/s) "
            f"replaces {v_fused['replaces_ms'] * 1e3:.1f} us of Q.K^T + P.V; attention layer {v_mha['ms'] * 1e3:.1f} us "
            f"{v_mha['tflops']:.1f} TFLOP/s")
        for x in v_per:
            log(f"  {x['gemm']:8s} NN {x['ms'] * 1e3:8.1f} us {x['tflops']:7.1f} TF")
    mlp_ms, mlp_flops, mlp_graph_ms, mlp_graph_same, mlp_loss, mlp_state = bench_mlp(om, max(20, args.steps), 5)
    log(f"mlp step {mlp_ms * 1e3:.1f} us (graph replay {mlp_graph_ms * 1e3:.1f} us, bit-identical {mlp_graph_same}),"
        f" loss {mlp_loss:.4f}")

    cpu = None
    cpu_r18 = None
    cpu_extra = {}
    gemm_err = conv_err = n_err = r50_err = None
    vit_err, mlp_err, train_err = {}, {}, {}
    if rank == 0 and not args.no_cpu:
        log("cpu checks of the sampled GPU results (oracle, float64)")
        gemm_err = cpu_check_gemm(gemm_rows)
        cpu_check_sweep(sweep, sweep_samples)
        conv_err = cpu_check_resnet18(conv_samples)
        r50_err = cpu_check_resnet50(r50_samples)
        n_err = cpu_check_resnet18_net(n_logits2)
        vit_err = cpu_check_vit(vit_samples)
        mlp_err = cpu_check_mlp(mlp_state)
        train_err = cpu_check_resnet18_train(n_train_state)
        log(f"parity: gemm {gemm_err:.2e}, sweep max {max(e['parity'] for e in sweep):.2e}, conv {conv_err:.2e}, "
            f"resnet50 {r50_err:.2e}, network logits {n_err:.1e}, vit {vit_err}, mlp {mlp_err}, train {train_err}")
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
        k50, ips50, dt50 = cpu_baseline_resnet50()
        cpu_extra["resnet50"] = {"value": round(ips50, 3), "unit": "img/s", "cores": threads, "kind": k50 if k50 == "reference" else "port",
                                 "sample": f"2 images through the 53 ResNet-50 convs ({dt50:.2f} s, one pass)"}
        kv, tfv, dtv = cpu_baseline_vit()
        cpu_extra["vit"] = {"value": round(tfv, 4), "unit": "TFLOP/s", "cores": threads, "kind": kv if kv == "reference" else "port",
                            "sample": f"one image's share of the ViT GEMM set (197 tokens, fp16-rounded fp32 inputs), {dtv:.2f} s"}
        kn, n_fwd_ips, n_train_ips, n_fdt, n_tdt = cpu_baseline_resnet18_net()
        cpu_extra["resnet18_net"] = {"kind": kn if kn == "reference" else "port", "cores": threads,
                                     "forward_img_s": round(n_fwd_ips, 3), "train_img_s": round(n_train_ips, 3),
                                     "sample": f"2 images, median of 3: inference forward {n_fdt:.2f} s, "
                                               f"training step {n_tdt:.2f} s (reference CPUBackend chain)"}
        km, msm = cpu_baseline_mlp()
        cpu_extra["mlp"] = {"value": round(msm, 3), "unit": "ms/step", "cores": threads, "kind": km if km == "reference" else "port",
                            "sample": "mean of 20 MLP fwd+bwd steps after one warm-up"}

    del n_train_state
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
                   "M": M, "N": N, "K": K, "layout": "NN", "device": dev,
                   "timed": "right after the fp32 GEMM sweep (last shape 8192^3), inputs uploaded before it: "
                            "an idle MI355X needs ~20 ms of load before its clocks settle"},
        "pct_mfma_peak": round(100.0 * tflops * 1e12 / PEAK_FP32, 1),
        "roofline": {"bound": "mfma", "achieved": round(flops / gemm_kernel_ms / 1e9, 2), "peak": 157.3,
                     "unit": "TFLOP/s", "frac": round(flops / gemm_kernel_ms / 1e9 / 157.3, 4),
                     "traffic": traffic,
                     "traffic_source": "profiles/traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE passes over "
                                       "`bench.py --traffic-probe`, copy-calibrated (recorded, not measured in this run)"},
        "cpu_baseline": cpu,
        "gemm_sweep": sweep,
        "parity": {"gemm_sampled_rows_max_err": gemm_err, "conv_sampled_max_err": conv_err, "tol": 1e-4,
                   "resnet50_conv_sampled_max_err": r50_err,
                   "resnet18_network_logits_rel_err": n_err,
                   "resnet18_train_step": train_err,
                   "vit": vit_err,
                   "mlp_step": mlp_err,
                   "bars": {"gemm, conv, resnet50, vit gemms, mlp layers and gradients": "1e-4 K-scaled (float64)",
                            "resnet18 logits": "1e-4 relative Frobenius",
                            "train step": "forward ops 1e-4, weight gradients 1e-3 relative Frobenius",
                            "attention fused (half context)": "2e-3 fp16 / 1.2e-2 bf16 of sum_j P_ij |V_jd|",
                            "attention layer": "2u + 1e-4 of (B_ctx + |ctx|) |W_out| + |b_out|",
                            "mlp loss, logit gradient": "1e-5 relative"}},
        "resnet18_conv": {"value": round(img_s, 1), "unit": "img/s", "batch": 32, "ms_per_batch": round(r_ms, 4),
                          "launch": "eager: 20 conv launches on the library stream",
                          "tflops": round(r_flops / r_ms / 1e9, 2),
                          "roofline": {"bound": "mfma (per-layer max(flops/157.3T, bytes/8TB/s))",
                                       "roof_ms": round(r_roof_ms, 4), "frac": round(r_roof_ms / r_ms, 4)},
                          "graph_replay": {"ms_per_batch": round(r_graph_ms, 4),
                                           "img_s": round(32.0 / r_graph_ms * 1e3, 1),
                                           "roof_frac": round(r_roof_ms / r_graph_ms, 4),
                                           "bit_identical_to_eager": bool(r_graph_same)},
                          "layers": per, "cpu_baseline": cpu_r18},
        "resnet18_network": {"batch": 32, "data": "synthetic images N(0,1), Kaiming-uniform weights, seeded BN",
                             "forward": {"ms": round(n_fwd_ms, 4), "img_s": round(32 / n_fwd_ms * 1e3, 1),
                                         "tflops": round(n_fl / n_fwd_ms / 1e9, 2),
                                         "frac_of_157_3": round(n_fl / n_fwd_ms / 1e9 / 157.3, 4),
                                         "logits_rel_err_vs_cpu_chain": n_err},
                             "train_step": {"ms": round(n_train_ms, 4), "img_s": round(32 / n_train_ms * 1e3, 1),
                                            "tflops": round(n_train_fl / n_train_ms / 1e9, 2),
                                            "frac_of_157_3": round(n_train_fl / n_train_ms / 1e9 / 157.3, 4),
                                            "scope": "forward with batch statistics + backward to every weight; "
                                                     "no optimizer update"},
                             "cpu_baseline": cpu_extra.get("resnet18_net")},
        "resnet18_infer_pipeline": infer,
        "resnet50_conv": {"value": round(64 / r50_ms * 1e3, 1), "unit": "img/s", "batch": 64, "ms_per_batch": round(r50_ms, 4),
                          "tflops": round(r50_flops / r50_ms / 1e9, 2),
                          "roofline": {"roof_ms": round(r50_roof, 4), "frac": round(r50_roof / r50_ms, 4)},
                          "cpu_baseline": cpu_extra.get("resnet50")},
        "vit_b16_gemms": {"batch": 64, "tokens": 197, "hidden": 768, "heads": 12, **vit,
                          "cpu_baseline": cpu_extra.get("vit")},
        "mlp_784_256_128_10": {"batch": 128, "us_per_step": round(mlp_ms * 1e3, 2),
                               "gflops": round(mlp_flops / mlp_ms / 1e6, 1),
                               "graph_replay": {"us_per_step": round(mlp_graph_ms * 1e3, 2),
                                                "bit_identical_to_eager": bool(mlp_graph_same)},
                               "loss": round(mlp_loss, 5),
                               "scope": "forward, softmax + cross-entropy on labels uniform in 0..9, backward "
                                        "(dW, db, dA every layer, ReLU gates); no optimizer update",
                               "cpu_baseline": cpu_extra.get("mlp")},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
