"""Training half of the conv / BatchNorm path: conv2d input and weight
gradients, BatchNorm2d training statistics and its backward pass, against
float64 and against the oracle (CPUBackend restated: conv2dBackwardInput /
conv2dBackwardWeight cpu_backend.ixx:666-772, batchNorm2d training
:796-822, batchNorm2dBackward :847-890).

Tolerances (written here, all 1e-4 relative to an error budget):
  * conv gradients: the same contraction over absolute values — dX against
    col2im(|W|^T |gO|), dW against sum |gO| im2col(|x|)^T, dB against sum |gO|;
  * BN statistics: mean against mean|x|, variance against var + mean|x|^2,
    y against |gamma| invStd (|x| + |mean| + mean|x|) + |beta|;
  * BN backward: dX against |gamma| invStd / cnt (cnt |dy| + sum|dy| + |xhat| sum|dy xhat|),
    dGamma against sum |dy xhat|, dBeta against sum |dy|.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu
TOL = O.TOL_FP32

# (N, Cin, H, W, Cout, KH, KW, stride, pad): the input gradient runs one convolution per
# output phase (s*s of them; stride > kernel leaves phases without taps, zero-filled);
# the tap counts cover every gather mode (32-bit mask, 64-bit mask, coordinate compares).
GRAD_SHAPES = [
    (2, 16, 14, 14, 32, 3, 3, 1, 1),    # ResNet 3x3 s1
    (2, 16, 15, 15, 32, 3, 3, 2, 1),    # 3x3 s2, odd input
    (2, 32, 14, 14, 64, 1, 1, 2, 0),    # 1x1 s2 downsample
    (1, 3, 32, 32, 16, 7, 7, 2, 3),     # 7x7 s2 stem
    (2, 8, 11, 11, 8, 5, 5, 1, 1),      # 5x5 s1 pad 1 (flipped pad 3)
    (2, 8, 12, 10, 16, 3, 1, 1, 0),     # KH != KW
    (2, 8, 9, 9, 8, 1, 1, 1, 1),        # pad > K-1
    (2, 16, 8, 8, 24, 1, 1, 1, 0),      # 1x1 s1: x read as a plane, 4-pixel vectors
    (2, 16, 7, 7, 24, 1, 1, 1, 0),      # 1x1 s1, 49 pixels per image: scalar plane reads
    (3, 5, 7, 9, 6, 3, 3, 3, 2),        # stride 3, ragged
    (1, 3, 10, 12, 5, 4, 8, 1, 2),      # 32 taps: 64-bit tap mask
    (1, 2, 12, 12, 3, 7, 9, 1, 3),      # 63 taps: last 64-bit mask mode
    (1, 2, 10, 10, 3, 8, 8, 1, 3),      # 64 taps: coordinate compares
    (2, 2, 13, 13, 4, 9, 9, 2, 4),      # 81 taps, stride 2
    (1, 2, 9, 9, 2, 3, 3, 4, 0),        # stride > kernel: phases without taps
    (1, 2, 8, 8, 2, 2, 2, 2, 1),        # even kernel, stride 2, pad 1
]


def _ids(s):
    return "N{}C{}H{}W{}o{}k{}x{}s{}p{}".format(*s)


def _data(shape, seed):
    N, Cin, H, W, Cout, KH, KW, s, p = shape
    Ho, Wo = O.out_hw(H, W, KH, KW, s, p)
    x = O.randn((N, Cin, H, W), seed)
    w = O.randn((Cout, Cin, KH, KW), seed + 1, 0.2)
    g = O.randn((N, Cout, Ho, Wo), seed + 2)
    return x, w, g, Ho, Wo


@pytest.mark.parametrize("shape", GRAD_SHAPES, ids=_ids)
def test_conv_backward_input(hip, shape):
    N, Cin, H, W, Cout, KH, KW, s, p = shape
    x, w, g, Ho, Wo = _data(shape, 31 + sum(shape))
    dG, dW = to_dev(hip, g), to_dev(hip, w)
    dX = empty_dev(hip, (N, Cin, H, W))
    hip.HIPBackend.conv2dBackwardInput(dG, dW, dX, N, Cin, H, W, Cout, KH, KW, s, p)
    got = dX.numpy()
    (X64, Xb), _, _ = O.conv_backward_f64(x, w, g, s, p) if KH == KW else _f64_rect(x, w, g, s, p)
    assert O.normalized_error(got, X64, Xb) <= TOL
    ref = O.conv2d_backward_input(g, w, H, W, s, p)
    assert O.normalized_error(got, ref, Xb) <= TOL


@pytest.mark.parametrize("shape", GRAD_SHAPES, ids=_ids)
def test_conv_backward_weight(hip, shape):
    N, Cin, H, W, Cout, KH, KW, s, p = shape
    x, w, g, Ho, Wo = _data(shape, 57 + sum(shape))
    dx, dg = to_dev(hip, x), to_dev(hip, g)
    dW = empty_dev(hip, (Cout, Cin, KH, KW))
    dB = empty_dev(hip, (Cout,))
    hip.HIPBackend.conv2dBackwardWeight(dx, dg, dW, dB, N, Cin, H, W, Cout, KH, KW, s, p)
    _, (W64, Wb), (B64, Bb) = O.conv_backward_f64(x, w, g, s, p) if KH == KW else _f64_rect(x, w, g, s, p)
    gw, gb = dW.numpy(), dB.numpy()
    assert O.normalized_error(gw, W64, Wb) <= TOL
    assert O.normalized_error(gb, B64, Bb) <= TOL
    rw, rb = O.conv2d_backward_weight(x, g, KH, KW, s, p)
    assert O.normalized_error(gw, rw, Wb) <= TOL
    assert O.normalized_error(gb, rb, Bb) <= TOL
    # the bias pointer is optional
    dW2 = empty_dev(hip, (Cout, Cin, KH, KW))
    hip.HIPBackend.conv2dBackwardWeight(dx, dg, dW2, None, N, Cin, H, W, Cout, KH, KW, s, p)
    assert np.array_equal(dW2.numpy(), gw), "weight gradient must not depend on the bias request"


def _f64_rect(x, w, g, s, p):
    """float64 gradients for rectangular kernels (direct loops over taps)."""
    x64, w64, g64 = (np.asarray(a, np.float64) for a in (x, w, g))
    N, Cin, H, W = x64.shape
    Cout, _, KH, KW = w64.shape
    Ho, Wo = g64.shape[2:]
    xp = np.zeros((N, Cin, H + 2 * p, W + 2 * p))
    xp[:, :, p:p + H, p:p + W] = x64
    dXp, dXpb = np.zeros_like(xp), np.zeros_like(xp)
    dW, dWb = np.zeros_like(w64), np.zeros_like(w64)
    for kh in range(KH):
        for kw in range(KW):
            win = xp[:, :, kh:kh + s * (Ho - 1) + 1:s, kw:kw + s * (Wo - 1) + 1:s]   # N Cin Ho Wo
            dW[:, :, kh, kw] = np.einsum("nohw,nchw->oc", g64, win)
            dWb[:, :, kh, kw] = np.einsum("nohw,nchw->oc", np.abs(g64), np.abs(win))
            dXp[:, :, kh:kh + s * (Ho - 1) + 1:s, kw:kw + s * (Wo - 1) + 1:s] += np.einsum("oc,nohw->nchw", w64[:, :, kh, kw], g64)
            dXpb[:, :, kh:kh + s * (Ho - 1) + 1:s, kw:kw + s * (Wo - 1) + 1:s] += np.einsum("oc,nohw->nchw", np.abs(w64[:, :, kh, kw]), np.abs(g64))
    sl = (slice(None), slice(None), slice(p, p + H), slice(p, p + W))
    return (dXp[sl], dXpb[sl]), (dW, dWb), (g64.sum(axis=(0, 2, 3)), np.abs(g64).sum(axis=(0, 2, 3)))


def _wgrad_rows(x, g, rows, K, s, p):
    """float64 weight-gradient rows and their |.| budget: sum_n g[n, rows] im2col(x[n])^T."""
    cols, _, _ = O._im2col64(np.asarray(x, np.float64), K, K, s, p)     # N x Kc x HW
    g64 = np.asarray(g, np.float64).reshape(g.shape[0], g.shape[1], -1)[:, rows]
    ref = np.einsum("nop,nkp->ok", g64, cols, optimize=True)
    bound = np.einsum("nop,nkp->ok", np.abs(g64), np.abs(cols), optimize=True)
    return ref, bound


# ResNet shapes at batch 8 (long pixel axes: hundreds of pixel splits, summed in order)
WGRAD_LARGE = [
    (8, 3, 224, 224, 64, 7, 2, 3),      # stem, 49 taps, 100k pixels
    (8, 64, 56, 56, 64, 3, 1, 1),       # layer 1
    (8, 128, 28, 28, 256, 1, 2, 0),     # downsample 1x1 s2
    (8, 256, 14, 14, 256, 3, 1, 1),     # layer 3 (196 pixels per image: 4-pixel vectors)
    (8, 256, 56, 56, 64, 1, 1, 0),      # ResNet-50 bottleneck 1x1 reduce
]


@pytest.mark.parametrize("shape", WGRAD_LARGE, ids=lambda s: "N{}C{}H{}W{}o{}k{}s{}p{}".format(*s))
def test_conv_backward_weight_large(hip, shape):
    N, Cin, H, W, Cout, K, s, p = shape
    Ho, Wo = O.out_hw(H, W, K, K, s, p)
    x = O.randn((N, Cin, H, W), 61 + Cin)
    g = O.randn((N, Cout, Ho, Wo), 62 + Cout)
    dW = empty_dev(hip, (Cout, Cin, K, K))
    hip.HIPBackend.conv2dBackwardWeight(to_dev(hip, x), to_dev(hip, g), dW, None, N, Cin, H, W, Cout, K, K, s, p)
    got = dW.numpy().reshape(Cout, -1)
    rows = np.array([0, 1, Cout // 2 - 1, Cout - 1])
    ref, bound = _wgrad_rows(x, g, rows, K, s, p)
    assert O.normalized_error(got[rows], ref, bound) <= TOL
    assert np.all(np.isfinite(got))


def test_conv_backward_weight_batch_chunks(hip):
    """A 1x1 conv whose output gradient (289 MiB) exceeds one 256 MiB buffer view:
    the batch is walked in two chunks, the second adding onto the first."""
    N, Cin, H, W, Cout = 90, 64, 56, 56, 256
    x = O.randn((N, Cin, H, W), 73)
    g = O.randn((N, Cout, H, W), 74)
    dW = empty_dev(hip, (Cout, Cin, 1, 1))
    hip.HIPBackend.conv2dBackwardWeight(to_dev(hip, x), to_dev(hip, g), dW, None, N, Cin, H, W, Cout, 1, 1, 1, 0)
    got = dW.numpy().reshape(Cout, Cin)
    rows = np.array([0, 77, 255])
    x64 = np.asarray(x, np.float64).reshape(N, Cin, -1)
    g64 = np.asarray(g, np.float64).reshape(N, Cout, -1)[:, rows]
    ref = np.einsum("nop,nkp->ok", g64, x64, optimize=True)
    bound = np.einsum("nop,nkp->ok", np.abs(g64), np.abs(x64), optimize=True)
    assert O.normalized_error(got[rows], ref, bound) <= TOL


def test_conv_backward_weight_chunked(hip):
    """ResNet-18 layer-4 conv at batch 32 (49 pixels per image: no 4-pixel vectors)."""
    N, Cin, H, W, Cout, K, s, p = 32, 512, 7, 7, 512, 3, 1, 1
    x = O.randn((N, Cin, H, W), 71)
    g = O.randn((N, Cout, H, W), 72)
    dW = empty_dev(hip, (Cout, Cin, K, K))
    hip.HIPBackend.conv2dBackwardWeight(to_dev(hip, x), to_dev(hip, g), dW, None, N, Cin, H, W, Cout, K, K, s, p)
    got = dW.numpy().reshape(Cout, -1)
    rows = np.array([0, 1, 255, 511])
    ref, bound = _wgrad_rows(x, g, rows, K, s, p)
    assert O.normalized_error(got[rows], ref, bound) <= TOL


# planes of 49 and fewer pixels go several to a workgroup; 6400 pixels take
# several workgroups per plane
BN_SHAPES = [(4, 8, 7, 9), (8, 64, 28, 28), (32, 16, 7, 7), (1, 3, 1, 1), (2, 300, 5, 5), (2, 4, 80, 80)]


@pytest.mark.parametrize("shape", BN_SHAPES, ids=lambda s: "N{}C{}H{}W{}".format(*s))
def test_batchnorm_training(hip, shape):
    N, C, H, W = shape
    x = O.randn(shape, 81 + C) * 2.0 + 0.5
    gamma, beta = O.uniform((C,), 82, 0.5, 1.5), O.randn((C,), 83, 0.1)
    rm0, rv0 = O.randn((C,), 84, 0.1), O.uniform((C,), 85, 0.5, 1.5)
    dx, dy = to_dev(hip, x), empty_dev(hip, shape)
    drm, drv = to_dev(hip, rm0), to_dev(hip, rv0)
    dsm, dsi = empty_dev(hip, (C,)), empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2d(dx, dy, to_dev(hip, gamma), to_dev(hip, beta), drm, drv, dsm, dsi, N, C, H, W,
                               1e-5, 0.1, True)
    y, rm, rv, sm, si = dy.numpy(), drm.numpy(), drv.numpy(), dsm.numpy(), dsi.numpy()
    y64, mean64, var64, inv64 = O.bn_train_f64(x, gamma, beta)
    absmean = np.abs(np.asarray(x, np.float64)).mean(axis=(0, 2, 3))
    assert np.max(np.abs(sm - mean64) / absmean) <= TOL
    assert np.max(np.abs(1.0 / si.astype(np.float64) ** 2 - 1e-5 - var64) / (var64 + absmean ** 2)) <= TOL
    assert np.max(np.abs(rm - (0.9 * rm0 + 0.1 * mean64)) / (np.abs(rm0) + absmean)) <= TOL
    assert np.max(np.abs(rv - (0.9 * rv0 + 0.1 * var64)) / (rv0 + var64 + absmean ** 2)) <= TOL
    ybound = (np.abs(gamma)[None, :, None, None] * inv64[None, :, None, None] *
              (np.abs(np.asarray(x, np.float64)) + np.abs(mean64)[None, :, None, None] + absmean[None, :, None, None])
              + np.abs(beta)[None, :, None, None])
    assert O.normalized_error(y, y64, ybound) <= TOL
    # against the oracle (the reference's sequential sums)
    ry, rrm, rrv, rsm, rsi = O.batchnorm2d_train(x, gamma, beta, rm0, rv0)
    assert O.normalized_error(y, ry, ybound) <= TOL
    assert np.max(np.abs(sm - rsm) / absmean) <= TOL
    assert np.max(np.abs(si - rsi) / rsi) <= TOL
    # saved-statistics pointers are optional
    dy2, drm2, drv2 = empty_dev(hip, shape), to_dev(hip, rm0), to_dev(hip, rv0)
    hip.HIPBackend.batchNorm2d(dx, dy2, to_dev(hip, gamma), to_dev(hip, beta), drm2, drv2, None, None, N, C, H, W,
                               1e-5, 0.1, True)
    assert np.array_equal(dy2.numpy(), y) and np.array_equal(drm2.numpy(), rm) and np.array_equal(drv2.numpy(), rv)


@pytest.mark.parametrize("shape", BN_SHAPES, ids=lambda s: "N{}C{}H{}W{}".format(*s))
def test_batchnorm_backward(hip, shape):
    N, C, H, W = shape
    x = O.randn(shape, 91 + C)
    gy = O.randn(shape, 92 + C)
    gamma, beta = O.uniform((C,), 93, 0.5, 1.5), O.randn((C,), 94, 0.1)
    _, _, _, sm, si = O.batchnorm2d_train(x, gamma, beta, np.zeros(C, np.float32), np.ones(C, np.float32))
    dgi, dgg, dgb = empty_dev(hip, shape), empty_dev(hip, (C,)), empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2dBackward(to_dev(hip, gy), to_dev(hip, x), to_dev(hip, sm), to_dev(hip, si),
                                       to_dev(hip, gamma), dgi, dgg, dgb, N, C, H, W)
    gi, gg, gb = dgi.numpy(), dgg.numpy(), dgb.numpy()
    dX, dG, dB, bound, absGX, absG = O.bn_backward_f64(gy, x, sm, si, gamma)
    assert O.normalized_error(gi, dX, bound) <= TOL
    assert O.normalized_error(gg, dG, absGX) <= TOL
    assert O.normalized_error(gb, dB, absG) <= TOL
    ri, rg, rb = O.batchnorm2d_backward(gy, x, sm, si, gamma)
    assert O.normalized_error(gi, ri, bound) <= TOL
    assert O.normalized_error(gg, rg, absGX) <= TOL
    assert O.normalized_error(gb, rb, absG) <= TOL


# Fused training passes: each must equal the separate reference ops bit for bit.
FUSE_SHAPES = [(4, 8, 7, 9), (8, 64, 28, 28), (2, 300, 5, 5), (2, 4, 80, 80)]


@pytest.mark.parametrize("shape", FUSE_SHAPES, ids=lambda s: "N{}C{}H{}W{}".format(*s))
@pytest.mark.parametrize("res,act", [(False, 0), (False, 1), (True, 1)], ids=["bn", "bn_relu", "bn_add_relu"])
def test_batchnorm_train_act(hip, shape, res, act):
    N, C, H, W = shape
    x = O.randn(shape, 101 + C) * 1.5 + 0.25
    r = O.randn(shape, 102 + C) if res else None
    gamma, beta = O.uniform((C,), 103, 0.5, 1.5), O.randn((C,), 104, 0.1)
    rm0, rv0 = O.randn((C,), 105, 0.1), O.uniform((C,), 106, 0.5, 1.5)
    dx, dr = to_dev(hip, x), (to_dev(hip, r) if res else None)
    dgam, dbet = to_dev(hip, gamma), to_dev(hip, beta)
    # fused
    dy, drm, drv, dsm, dsi = empty_dev(hip, shape), to_dev(hip, rm0), to_dev(hip, rv0), empty_dev(hip, (C,)), \
        empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2dTrainAct(dx, dy, dgam, dbet, drm, drv, dsm, dsi, N, C, H, W, 1e-5, 0.1, dr, act)
    # separate reference ops
    ey, erm, erv, esm, esi = empty_dev(hip, shape), to_dev(hip, rm0), to_dev(hip, rv0), empty_dev(hip, (C,)), \
        empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2d(dx, ey, dgam, dbet, erm, erv, esm, esi, N, C, H, W, 1e-5, 0.1, True)
    n = N * C * H * W
    if res:
        hip.HIPBackend.add(ey, dr, ey, n)
    if act:
        hip.HIPBackend.relu(ey, ey, n)
    for a, b in ((dy, ey), (drm, erm), (drv, erv), (dsm, esm), (dsi, esi)):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    # and against the oracle chain (sums in the reference's order: within the BN bar)
    ry, _, _, _, _ = O.batchnorm2d_train(x, gamma, beta, rm0, rv0)
    if res:
        ry = O.add(ry, r)
    if act:
        ry = O.relu(ry)
    y64, mean64, var64, inv64 = O.bn_train_f64(x, gamma, beta)
    absmean = np.abs(np.asarray(x, np.float64)).mean(axis=(0, 2, 3))
    bound = (np.abs(gamma)[None, :, None, None] * inv64[None, :, None, None] *
             (np.abs(np.asarray(x, np.float64)) + np.abs(mean64)[None, :, None, None] + absmean[None, :, None, None])
             + np.abs(beta)[None, :, None, None] + (np.abs(r) if res else 0.0))
    assert O.normalized_error(dy.numpy(), ry, bound) <= TOL


@pytest.mark.parametrize("shape", FUSE_SHAPES, ids=lambda s: "N{}C{}H{}W{}".format(*s))
def test_batchnorm_backward_relu(hip, shape):
    N, C, H, W = shape
    x = O.randn(shape, 111 + C)
    gy = O.randn(shape, 112 + C)
    m = O.randn(shape, 113 + C)
    m.reshape(-1)[:4] = [np.nan, 0.0, -0.0, 1e-45]      # gate edge cases: only > 0 passes
    gamma = O.uniform((C,), 114, 0.5, 1.5)
    _, _, _, sm, si = O.batchnorm2d_train(x, gamma, np.zeros(C, np.float32), np.zeros(C, np.float32),
                                          np.ones(C, np.float32))
    dgy, dm, dx = to_dev(hip, gy), to_dev(hip, m), to_dev(hip, x)
    dsm, dsi, dgam = to_dev(hip, sm), to_dev(hip, si), to_dev(hip, gamma)
    fi, fg, fb = empty_dev(hip, shape), empty_dev(hip, (C,)), empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2dBackwardRelu(dgy, dm, dx, dsm, dsi, dgam, fi, fg, fb, N, C, H, W)
    t = empty_dev(hip, shape)
    hip.HIPBackend.reluBackward(dm, dgy, t, N * C * H * W)
    si_, sg_, sb_ = empty_dev(hip, shape), empty_dev(hip, (C,)), empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2dBackward(t, dx, dsm, dsi, dgam, si_, sg_, sb_, N, C, H, W)
    for a, b in ((fi, si_), (fg, sg_), (fb, sb_)):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    gated = O.relu_backward(m, gy)
    dX, dG, dB, bound, absGX, absG = O.bn_backward_f64(gated, x, sm, si, gamma)
    assert O.normalized_error(fi.numpy(), dX, bound) <= TOL
    assert O.normalized_error(fg.numpy(), dG, absGX) <= TOL
    assert O.normalized_error(fb.numpy(), dB, absG) <= TOL
    # gradient outputs optional
    hip.HIPBackend.batchNorm2dBackwardRelu(dgy, dm, dx, dsm, dsi, dgam, fi, None, None, N, C, H, W)
    assert np.array_equal(fi.numpy().view(np.uint32), si_.numpy().view(np.uint32))


@pytest.mark.parametrize("n", [1, 7, 4096, 1000003])
def test_add_relu_backward(hip, n):
    a, x, g = O.randn((n,), n), O.randn((n,), n + 1), O.randn((n,), n + 2)
    if n >= 4:
        x[:4] = [np.nan, 0.0, -0.0, 1e-45]
    do = empty_dev(hip, (n,))
    hip.HIPBackend.addReluBackward(to_dev(hip, a), to_dev(hip, x), to_dev(hip, g), do, n)
    ref = O.add(a, O.relu_backward(x, g))
    assert np.array_equal(do.numpy().view(np.uint32), ref.view(np.uint32))
