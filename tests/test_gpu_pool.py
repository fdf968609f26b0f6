"""Pooling, the residual sum and the residual-fused conv against the oracle.

Pooling forward and the gather-form backwards compute the reference's
expressions in the reference's summation order, so their bar is bit equality
(cpu_backend.ixx:897-1023, :1467-1510, :147-160). The reference-signature max
pool backward scatters with atomic adds: an input that wins several windows
gets their gradients in an unspecified order, so it is held to 1e-6 of the sum
of |contributions|. The residual-fused conv is held to the conv bar (1e-4 of
the float64 budget, plus |residual|).
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# (N, C, H, W, K, stride, pad): ResNet stem max pool, overlapping / non-overlapping, ragged, padded-only windows
POOL = [(2, 64, 112, 112, 3, 2, 1), (3, 5, 9, 10, 2, 2, 0), (2, 3, 7, 7, 3, 1, 1), (1, 2, 5, 6, 4, 3, 2),
        (1, 1, 3, 3, 2, 2, 2)]   # the last: a window wholly in the padding


def _pid(s):
    return "N{}C{}H{}W{}k{}s{}p{}".format(*s)


@pytest.mark.parametrize("g", POOL, ids=_pid)
def test_maxpool(hip, g):
    N, C, H, W, K, s, p = g
    x = O.randn((N, C, H, W), sum(g))
    x[0, 0, :2, :2] = 0.5                                   # ties: the first maximum wins
    y_ref, i_ref = O.maxpool2d(x, K, s, p)
    Ho, Wo = y_ref.shape[2:]
    dx, dy, di = to_dev(hip, x), empty_dev(hip, y_ref.shape), empty_dev(hip, y_ref.shape, np.int32)
    hip.HIPBackend.maxPool2d(dx, dy, di, N, C, H, W, K, K, s, p)
    assert np.array_equal(bits(dy.numpy()), bits(y_ref))
    assert np.array_equal(di.numpy(), i_ref)
    gO = O.randn(y_ref.shape, 7 + sum(g))
    gi_ref = O.maxpool2d_backward(gO, i_ref, H, W)
    dg, dgi = to_dev(hip, gO), empty_dev(hip, x.shape)
    hip.HIPBackend.maxPool2dBackwardEx(dg, di, dgi, N, C, H, W, K, K, s, p)
    assert np.array_equal(bits(dgi.numpy()), bits(gi_ref))
    dgi2 = to_dev(hip, np.full(x.shape, 9.0, np.float32))   # must be overwritten, not accumulated
    hip.HIPBackend.maxPool2dBackward(dg, di, dgi2, N, C, Ho, Wo, H, W)
    absum = O.maxpool2d_backward(np.abs(gO), i_ref, H, W).astype(np.float64)
    assert np.all(np.abs(dgi2.numpy() - gi_ref) <= 1e-6 * absum)
    # without indices the forward still runs
    hip.HIPBackend.maxPool2d(dx, dy, None, N, C, H, W, K, K, s, p)
    assert np.array_equal(bits(dy.numpy()), bits(y_ref))


# The stem pooling (3x3, stride 2, pad 1, even H and W) has its own kernels:
# a paired forward when W % 4 == 0 and a 2x2-block gather backward. Planes: a
# constant plane (every window ties: the first candidate in (kh, kw) order
# wins), a plane of large values at odd (row, col) (each the maximum of up to
# four windows, so the backward adds several gradients into one input), and
# random planes. W % 4 != 0 exercises the general forward with the fast backward.
@pytest.mark.parametrize("shape", [(2, 4, 8, 12), (1, 3, 6, 10), (2, 3, 16, 16), (1, 2, 2, 4)],
                         ids=lambda v: "N{}C{}H{}W{}".format(*v))
def test_maxpool_stem_paths(hip, shape):
    N, C, H, W = shape
    x = O.randn((N, C, H, W), 100 + H + W)
    x[0, 0] = 0.25
    if C > 1:
        x[0, 1] = -1.0
        x[0, 1, 1::2, 1::2] = 5.0 + np.arange((H // 2) * (W // 2), dtype=np.float32).reshape(H // 2, W // 2) % 3
    y_ref, i_ref = O.maxpool2d(x, 3, 2, 1)
    dx, dy, di = to_dev(hip, x), empty_dev(hip, y_ref.shape), empty_dev(hip, y_ref.shape, np.int32)
    hip.HIPBackend.maxPool2d(dx, dy, di, N, C, H, W, 3, 3, 2, 1)
    assert np.array_equal(bits(dy.numpy()), bits(y_ref))
    assert np.array_equal(di.numpy(), i_ref)
    gO = O.randn(y_ref.shape, 200 + H)
    gO[0, 0, 0, 0] = -0.0
    gi_ref = O.maxpool2d_backward(gO, i_ref, H, W)
    dg, dgi = to_dev(hip, gO), to_dev(hip, np.full(x.shape, 3.0, np.float32))
    hip.HIPBackend.maxPool2dBackwardEx(dg, di, dgi, N, C, H, W, 3, 3, 2, 1)
    assert np.array_equal(bits(dgi.numpy()), bits(gi_ref))


@pytest.mark.parametrize("g", POOL, ids=_pid)
def test_avgpool(hip, g):
    N, C, H, W, K, s, p = g
    x = O.randn((N, C, H, W), 3 + sum(g))
    y_ref = O.avgpool2d(x, K, s, p)
    Ho, Wo = y_ref.shape[2:]
    dx, dy = to_dev(hip, x), empty_dev(hip, y_ref.shape)
    hip.HIPBackend.avgPool2d(dx, dy, N, C, H, W, K, K, s, p)
    assert np.array_equal(bits(dy.numpy()), bits(y_ref))
    gO = O.randn(y_ref.shape, 5 + sum(g))
    dgi = to_dev(hip, np.full(x.shape, 9.0, np.float32))
    hip.HIPBackend.avgPool2dBackward(to_dev(hip, gO), dgi, N, C, H, W, Ho, Wo, K, K, s, p)
    assert np.array_equal(bits(dgi.numpy()), bits(O.avgpool2d_backward(gO, H, W, K, s, p)))


# global pooling (1 x 1 output) through the LDS-staged path: the network's 7 x 7 planes, a
# plane count that is not a multiple of 64 at the largest staged plane (16 x 16), and a
# plane one row past it (the general kernel)
@pytest.mark.parametrize("g", [(2, 512, 7, 7, 1, 1), (3, 37, 16, 16, 1, 1), (1, 5, 17, 16, 1, 1), (2, 3, 11, 11, 3, 4),
                               (1, 2, 2, 3, 3, 5), (2, 4, 9, 9, 9, 9)],
                         ids=lambda g: "N{}C{}H{}W{}o{}x{}".format(*g))
def test_adaptive_avgpool(hip, g):
    N, C, H, W, OH, OW = g
    x = O.randn((N, C, H, W), sum(g))
    y_ref = O.adaptive_avgpool2d(x, OH, OW)
    dy = empty_dev(hip, y_ref.shape)
    hip.HIPBackend.adaptiveAvgPool2d(to_dev(hip, x), dy, N, C, H, W, OH, OW)
    y = dy.numpy()
    nan = np.isnan(y_ref)                                    # empty regions (H < OH) divide 0 by 0
    assert np.array_equal(np.isnan(y), nan)
    assert np.array_equal(bits(y[~nan]), bits(y_ref[~nan]))
    gO = O.randn(y_ref.shape, 3 + sum(g))
    dgi = empty_dev(hip, x.shape)
    hip.HIPBackend.adaptiveAvgPool2dBackward(to_dev(hip, gO), dgi, N, C, H, W, OH, OW)
    assert np.array_equal(bits(dgi.numpy()), bits(O.adaptive_avgpool2d_backward(gO, H, W)))


@pytest.mark.parametrize("n", [1, 5, 4096, 1000003])
def test_add(hip, n):
    a, b = O.randn((n,), n), O.randn((n,), n + 1)
    dc = empty_dev(hip, (n,))
    hip.HIPBackend.add(to_dev(hip, a), to_dev(hip, b), dc, n)
    assert np.array_equal(bits(dc.numpy()), bits(O.add(a, b)))


# ResNet block tails: 3x3 s1 conv2 + shortcut, and a ragged odd geometry.
RES = [(2, 64, 56, 56, 64, 3, 1, 1), (2, 128, 28, 28, 128, 3, 1, 1), (2, 512, 7, 7, 512, 3, 1, 1),
       (3, 5, 9, 7, 6, 3, 2, 1)]


@pytest.mark.parametrize("g", RES, ids=lambda g: "N{}C{}H{}W{}o{}k{}s{}p{}".format(*g))
def test_conv_bn_add_relu(hip, g):
    N, Cin, H, W, Cout, K, s, p = g
    Ho, Wo = O.out_hw(H, W, K, K, s, p)
    x = O.randn((N, Cin, H, W), 11 + sum(g))
    w = O.uniform((Cout, Cin, K, K), 12, -np.sqrt(6.0 / (Cin * K * K)), np.sqrt(6.0 / (Cin * K * K)))
    gam, bet = O.uniform((Cout,), 13, 0.5, 1.5), O.randn((Cout,), 14, 0.1)
    mu, var = O.randn((Cout,), 15, 0.1), O.uniform((Cout,), 16, 0.5, 1.5)
    res = O.randn((N, Cout, Ho, Wo), 17)
    dout = empty_dev(hip, (N, Cout, Ho, Wo))
    hip.HIPBackend.conv2dBiasBnAddAct(to_dev(hip, x), to_dev(hip, w), None, to_dev(hip, gam), to_dev(hip, bet),
                                      to_dev(hip, mu), to_dev(hip, var), 1e-5, to_dev(hip, res), 1, dout, N, Cin, H, W,
                                      Cout, K, K, s, p)
    y64, bound = O.conv_f64(x, w, None, s, p, gam, bet, mu, var, 1e-5, act=0)
    y64 = np.maximum(y64 + res, 0.0)
    bound = bound + np.abs(res)
    got = dout.numpy()
    assert O.normalized_error(got, y64, bound) <= O.TOL_FP32
    # the reference chain conv2d -> batchNorm2d(eval) -> add -> relu
    z = O.conv_bn_act(x, w, None, gam, bet, mu, var, 1e-5, act=0, stride=s, pad=p)
    chain = O.relu(O.add(z, res))
    assert O.normalized_error(got, chain, bound) <= O.TOL_FP32


def test_conv_add_rejects_aliasing(hip):
    d = to_dev(hip, np.ones(64, np.float32))
    with pytest.raises(hip.OmHipError, match="alias"):
        hip.HIPBackend.conv2dBiasBnAddAct(d, d, None, None, None, None, None, 1e-5, d, 1, d, 1, 1, 8, 8, 1, 1, 1, 1, 0)
