"""Writes tests/golden/reference_cpubackend.npz: input/output vectors produced by
the reference CPUBackend itself (oracle/_ref/libomref_reference.so, compiled
from src/hal/om.hal.cpu_backend.ixx + om.hal.simd.ixx by `make -C oracle ref`).

    python tests/golden/make_golden.py

The fixture pins the oracle restatement bit-for-bit on machines where the
reference cannot be built (the GPU box). Inputs are seeded; every output is a
call into the compiled reference, never into the oracle.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402


def main() -> None:
    R = O.ref_lib()
    if R is None:
        raise SystemExit("oracle/_ref/libomref_reference.so is not built (make -C oracle ref)")
    out = {}

    def put(name, **arrs):
        for k, v in arrs.items():
            out[f"{name}.{k}"] = np.asarray(v)

    # matmul: 4x8 tiles, row remainder, column remainder (N % 8), M < 4 path
    for (m, k, n) in [(37, 29, 53), (4, 8, 8), (3, 5, 7), (1, 17, 9), (12, 64, 24), (2, 2, 2)]:
        A, B = O.randn((m, k), 10 * m + k), O.randn((k, n), 10 * n + k)
        put(f"matmul_{m}x{k}x{n}", A=A, B=B, C=O.matmul(A, B, backend="reference"))
    # known answers of test_tensor_ops.cpp:55-82 through the compiled reference
    put("matmul_ka1", A=np.array([[1, 2], [3, 4]], np.float32), B=np.array([[5, 6], [7, 8]], np.float32),
        C=O.matmul(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32), backend="reference"))
    # batched
    A, B = O.randn((3, 5, 7), 31), O.randn((3, 7, 9), 32)
    put("batched_3x5x7x9", A=A, B=B, C=O.batched_matmul(A, B, backend="reference"))
    # transpose
    T = O.randn((13, 7), 33)
    put("transpose_13x7", A=T, B=O.transpose2d(T, backend="reference"))
    # MatMulBackward composition (autograd.ixx:261-286) with reference transpose2d + matmul
    G, A, B = O.randn((6, 5), 34), O.randn((6, 4), 35), O.randn((4, 5), 36)
    dA = O.matmul(G, O.transpose2d(B, backend="reference"), backend="reference")
    dB = O.matmul(O.transpose2d(A, backend="reference"), G, backend="reference")
    put("matmul_backward_6x4x5", G=G, A=A, B=B, dA=dA, dB=dB)
    # im2col + conv2d (with bias), stride 2 pad 1 and stride 1 pad 0
    x = O.randn((2, 3, 9, 9), 40)
    w = O.randn((4, 3, 3, 3), 41)
    bias = O.randn((4,), 42)
    put("im2col_3x9x9_k3s2p1", x=x[0], col=O.im2col(x[0], 3, 3, 1, 2, backend="reference"))
    put("conv_2x3x9x9_4_k3s2p1", x=x, w=w, bias=bias, y=O.conv2d(x, w, bias, 2, 1, backend="reference"))
    w5 = O.randn((5, 3, 5, 5), 43)
    put("conv_2x3x9x9_5_k5s1p0", x=x, w=w5, y=O.conv2d(x, w5, None, 1, 0, backend="reference"))
    # batchNorm2d eval and training
    xb = O.randn((2, 3, 4, 5), 44)
    g, b = O.uniform((3,), 45, 0.5, 1.5), O.randn((3,), 46, 0.1)
    m, v = O.randn((3,), 47, 0.1), O.uniform((3,), 48, 0.5, 1.5)
    y, sm, si = O.batchnorm2d_eval(xb, g, b, m, v, backend="reference")
    put("bn_eval", x=xb, gamma=g, beta=b, mean=m, var=v, y=y, savedMean=sm, savedInvStd=si)
    y, rm, rv, sm, si = O.batchnorm2d_train(xb, g, b, m, v, backend="reference")
    put("bn_train", x=xb, gamma=g, beta=b, mean=m, var=v, y=y, runMean=rm, runVar=rv, savedMean=sm, savedInvStd=si)
    # relu / reluBackward with special values
    z = np.concatenate([np.array([np.nan, -0.0, 0.0, -1, 1, np.inf, -np.inf, 1e-45, -1e-45], np.float32),
                        O.randn((23,), 49)])
    gz = O.randn(z.shape, 50)
    put("relu", x=z, y=O.relu(z, backend="reference"), g=gz, gi=O.relu_backward(z, gz, backend="reference"))
    # addBias
    A = O.randn((5, 11), 51)
    bb = O.randn((11,), 52)
    put("add_bias", A=A, bias=bb, out=O.add_bias(A, bb, backend="reference"))

    # training path: conv gradients (stride 1 and 2), BN backward
    xg = O.randn((2, 3, 9, 9), 60)
    wg = O.randn((4, 3, 3, 3), 61)
    for (s, p) in [(1, 1), (2, 1)]:
        Ho = (9 + 2 * p - 3) // s + 1
        go = O.randn((2, 4, Ho, Ho), 62 + s)
        gi = O.conv2d_backward_input(go, wg, 9, 9, s, p, backend="reference")
        gw, gb = O.conv2d_backward_weight(xg, go, 3, 3, s, p, backend="reference")
        put(f"conv_bwd_s{s}p{p}", x=xg, w=wg, gO=go, gI=gi, gW=gw, gB=gb)
    xb2 = O.randn((3, 4, 5, 6), 64)
    g2, b2 = O.uniform((4,), 65, 0.5, 1.5), O.randn((4,), 66, 0.1)
    _, _, _, sm2, si2 = O.batchnorm2d_train(xb2, g2, b2, np.zeros(4, np.float32), np.ones(4, np.float32),
                                            backend="reference")
    gy = O.randn(xb2.shape, 67)
    gi, gg, gbt = O.batchnorm2d_backward(gy, xb2, sm2, si2, g2, backend="reference")
    put("bn_backward", x=xb2, gO=gy, mean=sm2, invStd=si2, gamma=g2, gI=gi, gGamma=gg, gBeta=gbt)
    # pooling (with ties and padding) and add
    xp = O.randn((2, 3, 11, 11), 68)
    xp[0, 0, :4, :4] = 1.0                                    # ties: the first maximum wins
    y, idx = O.maxpool2d(xp, 3, 2, 1, backend="reference")
    gp = O.randn(y.shape, 69)
    put("maxpool_k3s2p1", x=xp, y=y, idx=idx, gO=gp, gI=O.maxpool2d_backward(gp, idx, 11, 11, backend="reference"))
    ya = O.avgpool2d(xp, 3, 2, 1, backend="reference")
    put("avgpool_k3s2p1", x=xp, y=ya, gO=gp, gI=O.avgpool2d_backward(gp, 11, 11, 3, 2, 1, backend="reference"))
    yad = O.adaptive_avgpool2d(xp, 3, 4, backend="reference")
    gad = O.randn(yad.shape, 70)
    put("adaptive_3x4", x=xp, y=yad, gO=gad, gI=O.adaptive_avgpool2d_backward(gad, 11, 11, backend="reference"))
    a1, a2 = O.randn((37,), 71), O.randn((37,), 72)
    put("add", a=a1, b=a2, out=O.add(a1, a2, backend="reference"))

    # softmax rows with ties, large magnitudes, -inf and a NaN first element
    sm = O.randn((6, 13), 73, 4.0)
    sm[1, :5] = 2.5                                           # tied maxima
    sm[2] *= 40.0                                             # exp underflows for most of the row
    sm[3, 4] = -np.inf
    sm[4, 0] = np.nan
    sm[5, 7] = np.nan                                         # skipped by the max scan
    put("softmax_6x13", x=sm, y=O.softmax(sm, backend="reference"))
    # attention core after the QKV projection, from the reference's transpose / batchedMatmul / softmax
    B_, S_, H_, D_ = 2, 7, 3, 4
    qkv = O.randn((B_ * S_, 3 * H_ * D_), 74)
    put("attention_2x7x3x4", qkv=qkv, out=O.attention(qkv, B_, S_, H_, D_, 0.5, backend="reference"))
    # cross-entropy (clamped zero probability, a row with two targets) and its joint gradient
    p = O.softmax(O.randn((5, 10), 75, 3.0), backend="reference")
    p[1, 3] = 0.0
    t = np.zeros((5, 10), np.float32)
    t[np.arange(5), [2, 3, 9, 0, 4]] = 1.0
    t[4, 7] = 0.75
    put("cross_entropy_5x10", p=p, t=t, loss=np.float32(O.cross_entropy(p, t, backend="reference")),
        grad=O.cross_entropy_softmax_backward(p, t, backend="reference"))

    path = os.path.join(HERE, "reference_cpubackend.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
