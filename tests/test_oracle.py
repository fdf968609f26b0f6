"""Pins the oracle (CPU restatement of the reference CPUBackend) — CPU only.

Checks, in order of strength:
  1. golden vectors written by the compiled reference CPUBackend
     (tests/golden/reference_cpubackend.npz): bit-exact;
  2. the reference's own known-answer tests (test_tensor_ops.cpp:55-82,
     test_phase5.cpp:206-222, test_nn.cpp:34-48, test_conv.cpp:21-49);
  3. the compiled reference on fresh seeded inputs, when oracle/_ref is built;
  4. float64 brute force within the K-scaled bound, plus closed forms
     (identity, transpose identity, linearity, all-ones conv interior = sum of
     weights, BN closed form) chosen so a dropped term, a wrong index or a
     transposed operand fails.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "reference_cpubackend.npz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------- 1. golden
def test_golden_matmul(gold):
    names = sorted({k.split(".")[0] for k in gold if k.startswith("matmul_") and k.endswith(".C")})
    assert len(names) >= 6
    for n in names:
        C = O.matmul(gold[f"{n}.A"], gold[f"{n}.B"])
        assert np.array_equal(bits(C), bits(gold[f"{n}.C"])), n


def test_golden_batched_transpose_backward(gold):
    assert np.array_equal(bits(O.batched_matmul(gold["batched_3x5x7x9.A"], gold["batched_3x5x7x9.B"])),
                          bits(gold["batched_3x5x7x9.C"]))
    assert np.array_equal(O.transpose2d(gold["transpose_13x7.A"]), gold["transpose_13x7.B"])
    dA, dB = O.matmul_backward(gold["matmul_backward_6x4x5.G"], gold["matmul_backward_6x4x5.A"],
                               gold["matmul_backward_6x4x5.B"])
    assert np.array_equal(bits(dA), bits(gold["matmul_backward_6x4x5.dA"]))
    assert np.array_equal(bits(dB), bits(gold["matmul_backward_6x4x5.dB"]))


def test_golden_conv(gold):
    assert np.array_equal(O.im2col(gold["im2col_3x9x9_k3s2p1.x"], 3, 3, 1, 2), gold["im2col_3x9x9_k3s2p1.col"])
    g = "conv_2x3x9x9_4_k3s2p1"
    y = O.conv2d(gold[f"{g}.x"], gold[f"{g}.w"], gold[f"{g}.bias"], 2, 1)
    assert np.array_equal(bits(y), bits(gold[f"{g}.y"]))
    g = "conv_2x3x9x9_5_k5s1p0"
    assert np.array_equal(bits(O.conv2d(gold[f"{g}.x"], gold[f"{g}.w"], None, 1, 0)), bits(gold[f"{g}.y"]))


def test_golden_bn(gold):
    p = [gold[f"bn_eval.{k}"] for k in ("x", "gamma", "beta", "mean", "var")]
    y, sm, si = O.batchnorm2d_eval(*p)
    for a, k in zip((y, sm, si), ("y", "savedMean", "savedInvStd")):
        assert np.array_equal(bits(a), bits(gold[f"bn_eval.{k}"])), k
    p = [gold[f"bn_train.{k}"] for k in ("x", "gamma", "beta", "mean", "var")]
    res = O.batchnorm2d_train(*p)
    for a, k in zip(res, ("y", "runMean", "runVar", "savedMean", "savedInvStd")):
        assert np.array_equal(bits(a), bits(gold[f"bn_train.{k}"])), k


def test_golden_relu_bias(gold):
    assert np.array_equal(bits(O.relu(gold["relu.x"])), bits(gold["relu.y"]))
    assert np.array_equal(bits(O.relu_backward(gold["relu.x"], gold["relu.g"])), bits(gold["relu.gi"]))
    assert np.array_equal(bits(O.add_bias(gold["add_bias.A"], gold["add_bias.bias"])), bits(gold["add_bias.out"]))


def test_golden_training(gold):
    for g, (s, p) in (("conv_bwd_s1p1", (1, 1)), ("conv_bwd_s2p1", (2, 1))):
        gi = O.conv2d_backward_input(gold[f"{g}.gO"], gold[f"{g}.w"], 9, 9, s, p)
        assert np.array_equal(bits(gi), bits(gold[f"{g}.gI"])), g
        gw, gb = O.conv2d_backward_weight(gold[f"{g}.x"], gold[f"{g}.gO"], 3, 3, s, p)
        assert np.array_equal(bits(gw), bits(gold[f"{g}.gW"])), g
        assert np.array_equal(bits(gb), bits(gold[f"{g}.gB"])), g
    k = "bn_backward"
    res = O.batchnorm2d_backward(gold[f"{k}.gO"], gold[f"{k}.x"], gold[f"{k}.mean"], gold[f"{k}.invStd"],
                                 gold[f"{k}.gamma"])
    for a, n in zip(res, ("gI", "gGamma", "gBeta")):
        assert np.array_equal(bits(a), bits(gold[f"{k}.{n}"])), n


def test_golden_pooling(gold):
    k = "maxpool_k3s2p1"
    y, idx = O.maxpool2d(gold[f"{k}.x"], 3, 2, 1)
    assert np.array_equal(bits(y), bits(gold[f"{k}.y"])) and np.array_equal(idx, gold[f"{k}.idx"])
    assert np.array_equal(bits(O.maxpool2d_backward(gold[f"{k}.gO"], idx, 11, 11)), bits(gold[f"{k}.gI"]))
    k = "avgpool_k3s2p1"
    assert np.array_equal(bits(O.avgpool2d(gold[f"{k}.x"], 3, 2, 1)), bits(gold[f"{k}.y"]))
    assert np.array_equal(bits(O.avgpool2d_backward(gold[f"{k}.gO"], 11, 11, 3, 2, 1)), bits(gold[f"{k}.gI"]))
    k = "adaptive_3x4"
    assert np.array_equal(bits(O.adaptive_avgpool2d(gold[f"{k}.x"], 3, 4)), bits(gold[f"{k}.y"]))
    assert np.array_equal(bits(O.adaptive_avgpool2d_backward(gold[f"{k}.gO"], 11, 11)), bits(gold[f"{k}.gI"]))
    assert np.array_equal(bits(O.add(gold["add.a"], gold["add.b"])), bits(gold["add.out"]))


# ---------------------------------------------------------- 2. known answers
def test_known_answers():
    assert O.matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]])).tolist() == [[19, 22], [43, 50]]
    assert O.matmul(np.arange(1, 7).reshape(2, 3), np.arange(7, 13).reshape(3, 2)).tolist() == [[58, 64], [139, 154]]
    assert np.all(O.batched_matmul(np.ones((2, 3, 4)), np.ones((2, 4, 5))) == 4.0)
    # Linear with zero input and zero bias -> 0 (test_nn.cpp:34-48)
    y = O.add_bias(O.matmul(np.zeros((2, 4)), O.randn((4, 3), 1)), np.zeros(3))
    assert np.all(y == 0)
    # Conv2d(1,4,3,s1,p1) on ones(1,1,8,8): shape (1,4,8,8), interior = sum(w); p0 -> (1,4,6,6)
    w = O.randn((4, 1, 3, 3), 2)
    y = O.conv2d(np.ones((1, 1, 8, 8), np.float32), w, None, 1, 1)
    assert y.shape == (1, 4, 8, 8)
    s = w.reshape(4, -1).astype(np.float64).sum(1)
    assert np.allclose(y[0, :, 1:7, 1:7], s[:, None, None], atol=1e-6)
    assert O.conv2d(np.ones((1, 1, 8, 8), np.float32), w, None, 1, 0).shape == (1, 4, 6, 6)


def test_degenerate_dims_zero_output():
    C = np.full((3, 4), 7, np.float32)
    O.lib().omrefMatmul(O._p(O.randn((3, 2), 1)), O._p(O.randn((2, 4), 2)), O._p(C), 3, 0, 4)
    assert np.all(C == 0)


# ------------------------------------------------ 3. compiled reference, fresh
ref_built = pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (needs the reference tree)")


@ref_built
@pytest.mark.parametrize("M,K,N", [(5, 9, 17), (64, 147, 100), (130, 257, 31), (4, 1, 8), (9, 300, 1)])
def test_vs_reference_matmul(M, K, N):
    A, B = O.randn((M, K), M), O.randn((K, N), N)
    assert np.array_equal(bits(O.matmul(A, B)), bits(O.matmul(A, B, backend="reference")))


@ref_built
@pytest.mark.parametrize("geom", [(2, 3, 11, 13, 5, 3, 2, 1), (1, 8, 7, 7, 16, 1, 1, 0), (2, 4, 12, 12, 6, 7, 2, 3)])
def test_vs_reference_conv_bn_relu(geom):
    N, cin, h, w, cout, k, s, p = geom
    x, wt, b = O.randn((N, cin, h, w), 1), O.randn((cout, cin, k, k), 2), O.randn((cout,), 3)
    y1 = O.conv2d(x, wt, b, s, p)
    y2 = O.conv2d(x, wt, b, s, p, backend="reference")
    assert np.array_equal(bits(y1), bits(y2))
    g, be, m, v = O.uniform((cout,), 4, .5, 1.5), O.randn((cout,), 5), O.randn((cout,), 6), O.uniform((cout,), 7, .5, 2)
    a = O.batchnorm2d_eval(y1, g, be, m, v)
    bb = O.batchnorm2d_eval(y2, g, be, m, v, backend="reference")
    assert all(np.array_equal(bits(u), bits(t)) for u, t in zip(a, bb))
    assert np.array_equal(bits(O.relu(a[0])), bits(O.relu(bb[0], backend="reference")))


@ref_built
@pytest.mark.parametrize("geom", [(2, 3, 11, 13, 5, 3, 2, 1), (1, 8, 7, 7, 16, 1, 1, 0), (2, 4, 12, 12, 6, 7, 2, 3),
                                  (3, 4, 8, 8, 4, 3, 1, 1)])
def test_vs_reference_training(geom):
    N, cin, h, w, cout, k, s, p = geom
    x, wt = O.randn((N, cin, h, w), 21), O.randn((cout, cin, k, k), 22)
    Ho, Wo = O.out_hw(h, w, k, k, s, p)
    g = O.randn((N, cout, Ho, Wo), 23)
    assert np.array_equal(bits(O.conv2d_backward_input(g, wt, h, w, s, p)),
                          bits(O.conv2d_backward_input(g, wt, h, w, s, p, backend="reference")))
    a = O.conv2d_backward_weight(x, g, k, k, s, p)
    b = O.conv2d_backward_weight(x, g, k, k, s, p, backend="reference")
    assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[1]), bits(b[1]))
    gam = O.uniform((cin,), 24, 0.5, 1.5)
    _, _, _, sm, si = O.batchnorm2d_train(x, gam, np.zeros(cin, np.float32), np.zeros(cin, np.float32),
                                          np.ones(cin, np.float32))
    gy = O.randn(x.shape, 25)
    r1 = O.batchnorm2d_backward(gy, x, sm, si, gam)
    r2 = O.batchnorm2d_backward(gy, x, sm, si, gam, backend="reference")
    assert all(np.array_equal(bits(u), bits(t)) for u, t in zip(r1, r2))
    y1, i1 = O.maxpool2d(x, 3, 2, 1)
    y2, i2 = O.maxpool2d(x, 3, 2, 1, backend="reference")
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(i1, i2)
    assert np.array_equal(bits(O.avgpool2d(x, 3, 2, 1)), bits(O.avgpool2d(x, 3, 2, 1, backend="reference")))
    assert np.array_equal(bits(O.adaptive_avgpool2d(x, 2, 3)), bits(O.adaptive_avgpool2d(x, 2, 3, backend="reference")))


# ----------------------------------------------- 4. float64 and closed forms
@pytest.mark.parametrize("M,K,N", [(33, 65, 17), (128, 784, 256), (7, 1000, 9)])
def test_matmul_vs_float64(M, K, N):
    A, B = O.randn((M, K), 7), O.randn((K, N), 8)
    C64, bound = O.gemm_f64(A, B)
    assert O.normalized_error(O.matmul(A, B), C64, bound) <= 1e-6
    assert O.normalized_error(O.matmul_transB(A, np.ascontiguousarray(B.T)), C64, bound) <= 1e-6
    assert O.normalized_error(O.matmul_transA(np.ascontiguousarray(A.T), B), C64, bound) <= 1e-6


def test_matmul_identity_and_transpose_rule():
    A = O.randn((9, 12), 1)
    assert np.array_equal(O.matmul(A, np.eye(12, dtype=np.float32)), A)
    B = O.randn((12, 5), 2)
    # (AB)^T = B^T A^T, exactly (same fma chains in the same k order)
    assert np.array_equal(O.matmul(A, B).T, O.matmul(np.ascontiguousarray(B.T), np.ascontiguousarray(A.T)))


def test_conv_vs_float64_and_direct_loop():
    x, w, b = O.randn((2, 3, 7, 6), 1), O.randn((4, 3, 3, 2), 2), O.randn((4,), 3)
    for s, p in [(1, 0), (2, 1), (3, 2)]:
        y = O.conv2d(x, w, b, s, p)
        y64, bound = O.conv_f64(x, w, b, s, p)
        assert O.normalized_error(y, y64, bound) <= 1e-6
    # the textbook 7-loop convolution on a tiny case (independent of im2col)
    y = O.conv2d(x, w, b, 2, 1)
    Ho, Wo = y.shape[2:]
    ref = np.zeros_like(y, dtype=np.float64)
    for n in range(2):
        for co in range(4):
            for oh in range(Ho):
                for ow in range(Wo):
                    acc = float(b[co])
                    for ci in range(3):
                        for kh in range(3):
                            for kw in range(2):
                                ih, iw = oh * 2 - 1 + kh, ow * 2 - 1 + kw
                                if 0 <= ih < 7 and 0 <= iw < 6:
                                    acc += float(x[n, ci, ih, iw]) * float(w[co, ci, kh, kw])
                    ref[n, co, oh, ow] = acc
    assert np.allclose(y, ref, atol=1e-5)


def test_bn_closed_form():
    x = O.randn((2, 3, 4, 4), 9)
    g, b, m, v = O.uniform((3,), 1, .5, 1.5), O.randn((3,), 2), O.randn((3,), 3), O.uniform((3,), 4, .5, 1.5)
    y, sm, si = O.batchnorm2d_eval(x, g, b, m, v)
    inv = 1.0 / np.sqrt(v.astype(np.float64) + 1e-5)
    expect = g[None, :, None, None] * (x - m[None, :, None, None]) * inv[None, :, None, None] + b[None, :, None, None]
    assert np.allclose(y, expect, rtol=1e-6, atol=1e-6)
    assert np.array_equal(sm, m)
    assert np.allclose(si, inv, rtol=1e-7)


def test_half_truncation_rule():
    """FP16Converter::floatToHalf truncates (fp16.ixx:92): differs from RNE only
    where the dropped 13 bits are >= half an ulp."""
    x = np.array([1.0, 65504.0, 1.0 + 2 ** -11 + 2 ** -12, -2.5, 0.0, 1e-40, 7e4, 2 ** -20], np.float32)
    t = O.float_to_half_trunc(x)
    assert t[0] == 0x3C00 and t[1] == 0x7BFF and t[3] == 0xC100 and t[4] == 0
    assert t[2] == 0x3C00                      # truncated; round-to-nearest gives 0x3C01
    assert x[2:3].astype(np.float16).view(np.uint16)[0] == 0x3C01
    assert t[5] == 0                           # fp32 subnormal flushed
    assert t[6] == 0x7C00                      # overflow -> inf
    assert t[7] == (x[7:8].astype(np.float16).view(np.uint16)[0])   # exact fp16 subnormal


# ------------------------------------------- training path: closed forms
@pytest.mark.parametrize("geom", [(2, 3, 9, 9, 4, 3, 1, 1), (2, 3, 9, 9, 4, 3, 2, 1), (1, 4, 8, 8, 6, 1, 2, 0),
                                  (1, 2, 12, 12, 3, 7, 2, 3)])
def test_conv_gradients_adjoint(geom):
    """<conv(x, w), g> = <x, dX(g)> = <w, dW(x, g)> (the gradients are the adjoints of
    the forward conv in x and in w), in float64 for the checker and within the
    K-scaled bar for the oracle; dB = sum of g."""
    N, C, H, W, Co, K, s, p = geom
    x, w = O.randn((N, C, H, W), 1), O.randn((Co, C, K, K), 2)
    Ho, Wo = O.out_hw(H, W, K, K, s, p)
    g = O.randn((N, Co, Ho, Wo), 3)
    y64, _ = O.conv_f64(x, w, None, s, p)
    (dX, dXb), (dW, dWb), (dB, dBb) = O.conv_backward_f64(x, w, g, s, p)
    lhs = float((y64 * g).sum())
    assert abs(lhs - float((np.asarray(x, np.float64) * dX).sum())) <= 1e-9 * (1 + abs(lhs))
    assert abs(lhs - float((np.asarray(w, np.float64) * dW).sum())) <= 1e-9 * (1 + abs(lhs))
    assert np.allclose(dB, np.asarray(g, np.float64).sum(axis=(0, 2, 3)))
    assert O.normalized_error(O.conv2d_backward_input(g, w, H, W, s, p), dX, dXb) <= O.TOL_FP32
    gw, gb = O.conv2d_backward_weight(x, g, K, K, s, p)
    assert O.normalized_error(gw, dW, dWb) <= O.TOL_FP32
    assert O.normalized_error(gb, dB, dBb) <= O.TOL_FP32


def test_bn_backward_numeric_gradient():
    """The float64 BN backward equals central differences of the float64 BN training
    forward (loss = sum(y * r)) in x, gamma and beta; the oracle meets it."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 3, 2))
    gamma, beta = rng.uniform(0.5, 1.5, 3), rng.standard_normal(3)
    r = rng.standard_normal(x.shape)

    def loss(xv, gv, bv):
        y, _, _, _ = O.bn_train_f64(xv, gv, bv)
        return float((y * r).sum())

    _, mean, _, inv = O.bn_train_f64(x, gamma, beta)
    dX, dG, dB, bound, absGX, absG = O.bn_backward_f64(r, x, mean, inv, gamma)
    h = 1e-6
    num = np.zeros_like(x)
    for i in np.ndindex(*x.shape):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        num[i] = (loss(xp, gamma, beta) - loss(xm, gamma, beta)) / (2 * h)
    assert np.max(np.abs(num - dX)) < 1e-6
    for c in range(3):
        e = np.eye(3)[c] * h
        assert abs((loss(x, gamma + e, beta) - loss(x, gamma - e, beta)) / (2 * h) - dG[c]) < 1e-6
        assert abs((loss(x, gamma, beta + e) - loss(x, gamma, beta - e)) / (2 * h) - dB[c]) < 1e-6
    x32 = x.astype(np.float32)
    _, _, _, sm, si = O.batchnorm2d_train(x32, gamma.astype(np.float32), beta.astype(np.float32),
                                          np.zeros(3, np.float32), np.ones(3, np.float32))
    gi, gg, gb = O.batchnorm2d_backward(r.astype(np.float32), x32, sm, si, gamma.astype(np.float32))
    dX2, dG2, dB2, bound2, absGX2, absG2 = O.bn_backward_f64(r, x32, sm, si, gamma)
    assert O.normalized_error(gi, dX2, bound2) <= O.TOL_FP32
    assert O.normalized_error(gg, dG2, absGX2) <= O.TOL_FP32
    assert O.normalized_error(gb, dB2, absG2) <= O.TOL_FP32


def test_pooling_closed_forms():
    """Pools against numpy sliding windows: max (first maximum's flat index), average
    with padding counted in the divisor, adaptive regions; backward = transpose."""
    x = O.randn((2, 3, 9, 10), 7)
    K, s, p = 3, 2, 1
    Ho, Wo = O.out_hw(9, 10, K, K, s, p)
    xp = np.full((2, 3, 9 + 2 * p, 10 + 2 * p), -np.inf, np.float64)
    xp[:, :, p:p + 9, p:p + 10] = x
    y, idx = O.maxpool2d(x, K, s, p)
    for oh in range(Ho):
        for ow in range(Wo):
            win = xp[:, :, oh * s:oh * s + K, ow * s:ow * s + K].reshape(2, 3, -1)
            assert np.array_equal(y[:, :, oh, ow], win.max(axis=2).astype(np.float32))
            a = win.argmax(axis=2)
            ih, iw = oh * s - p + a // K, ow * s - p + a % K
            flat = ((np.arange(2)[:, None] * 3 + np.arange(3)[None, :]) * 9 + ih) * 10 + iw
            assert np.array_equal(idx[:, :, oh, ow], flat)
    xz = np.zeros_like(xp)
    xz[:, :, p:p + 9, p:p + 10] = x
    ya = O.avgpool2d(x, K, s, p)
    for oh in range(Ho):
        for ow in range(Wo):
            ref = xz[:, :, oh * s:oh * s + K, ow * s:ow * s + K].sum(axis=(2, 3)) / 9.0
            assert np.allclose(ya[:, :, oh, ow], ref, rtol=1e-6, atol=1e-6)
    g = O.randn(ya.shape, 8)
    ga = O.avgpool2d_backward(g, 9, 10, K, s, p)
    assert np.isclose(float((ya.astype(np.float64) * g).sum()), float((x.astype(np.float64) * ga).sum()), rtol=1e-5)
    gm = O.maxpool2d_backward(g, idx, 9, 10)
    assert np.isclose(float((y.astype(np.float64) * g).sum()), float((x.astype(np.float64) * gm).sum()), rtol=1e-5)
    yad = O.adaptive_avgpool2d(x, 1, 1)
    assert np.allclose(yad[:, :, 0, 0], x.mean(axis=(2, 3)), rtol=1e-5, atol=1e-6)
    gad = O.randn(yad.shape, 9)
    assert np.allclose(O.adaptive_avgpool2d_backward(gad, 9, 10), np.broadcast_to(gad / 90.0, x.shape), rtol=1e-6)


def test_training_planted_mistakes():
    """A conv gradient with a shifted tap or a dropped image, or BN backward without
    the mean-gradient term, must fail the bar."""
    x, w = O.randn((2, 3, 9, 9), 11), O.randn((4, 3, 3, 3), 12)
    g = O.randn((2, 4, 5, 5), 13)
    (dX, dXb), (dW, dWb), _ = O.conv_backward_f64(x, w, g, 2, 1)
    gi = O.conv2d_backward_input(g, w, 9, 9, 2, 1)
    assert O.normalized_error(np.roll(gi, 1, axis=3), dX, dXb) > O.TOL_FP32
    gw, _ = O.conv2d_backward_weight(x[:1], g[:1], 3, 3, 2, 1)           # second image dropped
    assert O.normalized_error(gw, dW, dWb) > O.TOL_FP32
    xb, gy = O.randn((2, 3, 4, 4), 14), O.randn((2, 3, 4, 4), 15)
    gam = O.uniform((3,), 16, 0.5, 1.5)
    _, _, _, sm, si = O.batchnorm2d_train(xb, gam, np.zeros(3, np.float32), np.zeros(3, np.float32),
                                          np.ones(3, np.float32))
    dX, _, _, bound, _, _ = O.bn_backward_f64(gy, xb, sm, si, gam)
    naive = gam[None, :, None, None] * si[None, :, None, None] * gy              # ignores the batch statistics
    assert O.normalized_error(naive, dX, bound) > O.TOL_FP32


# ---------------------------------------- planted mistakes are caught (CPU)
def test_tolerance_catches_planted_mistakes():
    """A dropped k term, a transposed operand or an off-by-one row in a result
    built from the oracle must fail the K-scaled 1e-4 bar."""
    A, B = O.randn((64, 256), 1), O.randn((256, 48), 2)
    C64, bound = O.gemm_f64(A, B)
    good = O.matmul(A, B)
    assert O.normalized_error(good, C64, bound) <= O.TOL_FP32
    dropped = O.matmul(A[:, 1:], B[1:])                       # k = 0 term missing
    assert O.normalized_error(dropped, C64, bound) > O.TOL_FP32
    Bsq = O.randn((256, 256), 3)
    C64s, bounds = O.gemm_f64(A, Bsq)
    assert O.normalized_error(O.matmul(A, np.ascontiguousarray(Bsq.T)), C64s, bounds) > O.TOL_FP32
    shifted = np.roll(good, 1, axis=0)
    assert O.normalized_error(shifted, C64, bound) > O.TOL_FP32
    # conv: wrong padding offset
    x, w = O.randn((1, 3, 10, 10), 4), O.randn((5, 3, 3, 3), 5)
    y64, cb = O.conv_f64(x, w, None, 1, 1)
    wrong = np.roll(O.conv2d(x, w, None, 1, 1), 1, axis=3)
    assert O.normalized_error(wrong, y64, cb) > O.TOL_FP32


# ------------------------------------- softmax, attention, loss, bias gradient
def test_golden_softmax_attention_loss(gold):
    """Bit-exact against vectors the compiled reference wrote: softmax rows with ties, large
    magnitudes, -inf and NaN; the attention core composed from the reference's transpose2d,
    batchedMatmul and softmax; crossEntropy (a clamped zero probability, a row with two
    targets) and crossEntropySoftmaxBackward."""
    k = "softmax_6x13"
    assert np.array_equal(bits(O.softmax(gold[f"{k}.x"])), bits(gold[f"{k}.y"]))
    k = "attention_2x7x3x4"
    assert np.array_equal(bits(O.attention(gold[f"{k}.qkv"], 2, 7, 3, 4, 0.5)), bits(gold[f"{k}.out"]))
    k = "cross_entropy_5x10"
    loss = np.float32(O.cross_entropy(gold[f"{k}.p"], gold[f"{k}.t"]))
    assert loss.view(np.uint32) == np.float32(gold[f"{k}.loss"]).view(np.uint32)
    assert np.array_equal(bits(O.cross_entropy_softmax_backward(gold[f"{k}.p"], gold[f"{k}.t"])), bits(gold[f"{k}.grad"]))


@ref_built
def test_vs_reference_softmax_attention_loss():
    """Fresh seeded inputs: softmax (ties, magnitudes up to 1e4), the ViT attention core at
    197 tokens, crossEntropy and its gradient, all bit-exact against the compiled reference."""
    x = O.randn((64, 197), 81, 30.0)
    x[::3, 10:20] = 17.0
    x[5] *= 300.0
    assert np.array_equal(bits(O.softmax(x)), bits(O.softmax(x, backend="reference")))
    qkv = O.randn((197, 3 * 2 * 64), 82)
    assert np.array_equal(bits(O.attention(qkv, 1, 197, 2, 64, 0.125)),
                          bits(O.attention(qkv, 1, 197, 2, 64, 0.125, backend="reference")))
    p = O.softmax(O.randn((128, 10), 83, 2.0))
    t = np.eye(10, dtype=np.float32)[O.rng(84).integers(0, 10, 128)]
    assert np.float32(O.cross_entropy(p, t)) == np.float32(O.cross_entropy(p, t, backend="reference"))
    assert np.array_equal(bits(O.cross_entropy_softmax_backward(p, t)),
                          bits(O.cross_entropy_softmax_backward(p, t, backend="reference")))


def _softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_softmax_attention_vs_float64():
    """Softmax per element within 2^-24 * (2|x - max| + 4 + (n - 1)) relative of float64: the
    rounding of x - max (amplified by |x - max| through exp), one exp, one division, and the
    worst case of a sequential sum of n positive terms. The attention core within 1e-6 of the float64 result per context
    element, relative to sum_j P_ij |V_jd|. A softmax over the wrong axis and attention with
    unscaled Q must fail these bars."""
    x = O.randn((32, 197), 91, 5.0)
    p = O.softmax(x)
    p64 = _softmax64(x)
    budget = 2.0 ** -24 * (2.0 * np.abs(x - x.max(axis=1, keepdims=True)) + 4.0 + (x.shape[1] - 1))
    assert np.all(np.abs(p - p64) / p64 <= budget)
    assert np.allclose(p.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    wrong = O.softmax(np.ascontiguousarray(x.T)).T
    assert not np.all(np.abs(wrong[:, :32] - p64[:, :32]) / p64[:, :32] <= budget[:, :32])
    B_, S_, H_, D_ = 2, 50, 3, 64
    qkv = O.randn((B_ * S_, 3 * H_ * D_), 92)
    a = O.attention(qkv, B_, S_, H_, D_, 0.125)
    a64, bound = O.attention_f64(qkv, B_, S_, H_, D_, 0.125)
    assert O.normalized_error(a, a64, bound) <= 1e-6
    unscaled = O.attention(qkv, B_, S_, H_, D_, 1.0)
    assert O.normalized_error(unscaled, a64, bound) > 1e-2


def test_cross_entropy_and_bias_gradient_closed_forms():
    """crossEntropy equals -mean log(max(p, 1e-7)) over the one-hot entries (float64, 1e-6
    relative); dropping the clamp turns a zero probability into inf. The joint gradient is
    (p - t) / batch exactly as float32 arithmetic. The bias gradient equals numpy's sequential
    float32 cumulative sum over the rows (bit for bit), and an all-ones gradient gives N*HW."""
    p = O.softmax(O.randn((128, 10), 93, 2.0))
    lab = O.rng(94).integers(0, 10, 128)
    t = np.eye(10, dtype=np.float32)[lab]
    ref = -np.mean(np.log(np.maximum(p[np.arange(128), lab].astype(np.float64), 1e-7)))
    assert abs(O.cross_entropy(p, t) - ref) <= 1e-6 * abs(ref)
    p0 = p.copy()
    p0[0, lab[0]] = 0.0
    assert np.isfinite(O.cross_entropy(p0, t))
    with np.errstate(divide="ignore"):
        assert not np.isfinite(-np.mean(np.log(p0[np.arange(128), lab])))
    g = O.cross_entropy_softmax_backward(p, t)
    assert np.array_equal(bits(g), bits((p - t) * np.float32(1.0 / 128)))
    go = O.randn((300, 37), 95)
    seq = np.cumsum(go, axis=0, dtype=np.float32)[-1]
    assert np.array_equal(bits(O.add_bias_backward(go, 300, 37)), bits(seq))
    go3 = O.randn((4, 6, 25), 96)
    seq3 = np.cumsum(go3.transpose(1, 0, 2).reshape(6, -1), axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(bits(O.add_bias_backward(go3, 4, 6, 25)), bits(seq3))
    assert np.all(O.add_bias_backward(np.ones((4, 6, 25), np.float32), 4, 6, 25) == 100.0)
    assert not np.array_equal(bits(O.add_bias_backward(go[:-1], 299, 37)), bits(seq))   # a dropped row shows


@ref_built
def test_resnet18_train_step_oracle_equals_reference():
    """One image through the whole ResNet-18 training step (forward with batch statistics,
    backward to every weight) composed from oracle functions equals the same composition of
    the compiled reference's functions bit for bit."""
    from resnet_net import cpu_train_step, make_params
    P = make_params(seed=5, num_classes=10)
    img = O.randn((1, 3, 224, 224), 97)
    g = O.randn((1, 10), 98, 0.1)
    a = cpu_train_step(P, img, g)
    b = cpu_train_step(P, img, g, backend="reference")
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(bits(a[k]), bits(b[k])), k


def test_sum_and_head_maps_closed_forms():
    """CPUBackend::sum: exact on integer-valued data, ones sum to n below 2^24, and the float
    sequential order (2^24 + 1 + 1 ... stays 2^24, which a pairwise or float64 sum would not).
    The head split / merge (vit.ixx:196-232): exact permutations against numpy reshapes, Q
    scaled by one float multiply, merge(split) returning the Q, K and V thirds of the input."""
    assert O.sum_(np.ones(1000, np.float32)) == np.float32(1000.0)
    ints = O.rng(95).integers(-1000, 1000, 4099).astype(np.float32)
    assert O.sum_(ints) == np.float32(ints.astype(np.int64).sum())
    seq = np.array([2.0 ** 24] + [1.0] * 8, np.float32)
    assert O.sum_(seq) == np.float32(2.0 ** 24)                # each +1 rounds away in float
    assert np.float32(seq.astype(np.float64).sum()) == np.float32(2.0 ** 24 + 8)
    assert O.sum_(np.zeros(0, np.float32)) == np.float32(0.0)
    B_, S_, H_, D_ = 3, 5, 4, 6
    qkv = O.randn((B_ * S_, 3 * H_ * D_), 96)
    q, k, v = O.qkv_split_heads(qkv, B_, S_, H_, D_, 0.37)
    t = qkv.reshape(B_, S_, 3, H_, D_).transpose(2, 0, 3, 1, 4).reshape(3, B_ * H_, S_, D_)
    assert np.array_equal(bits(q), bits(t[0] * np.float32(0.37)))
    assert np.array_equal(bits(k), bits(t[1]))
    assert np.array_equal(bits(v), bits(t[2]))
    for i, part in enumerate((k, v)):
        merged = O.merge_heads(part, B_, S_, H_, D_)
        assert np.array_equal(bits(merged), bits(qkv[:, (i + 1) * H_ * D_:(i + 2) * H_ * D_]))
    swapped = O.merge_heads(np.ascontiguousarray(k.reshape(B_, H_, S_, D_).transpose(0, 2, 1, 3)).reshape(
        B_ * H_, S_, D_), B_, S_, H_, D_)
    assert not np.array_equal(bits(swapped), bits(qkv[:, H_ * D_:2 * H_ * D_]))


@ref_built
def test_vs_reference_sum():
    """CPUBackend::sum bit-exact against the compiled reference, on sizes around the AVX2
    width and a large array whose sequential rounding differs from float64."""
    R = O.ref_lib()
    if not hasattr(R, "refSum"):
        pytest.skip("compiled reference predates refSum: rebuild oracle/_ref")
    for n, seed in ((1, 1), (7, 2), (8, 3), (31, 4), (1000, 5), (1 << 20, 6)):
        x = O.randn((n,), 97 + seed, 3.0)
        assert O.sum_(x).view(np.uint32) == O.sum_(x, backend="reference").view(np.uint32), n
