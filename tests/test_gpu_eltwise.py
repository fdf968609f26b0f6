"""Bit-exact parity of the memory-bound HAL ops against the oracle.

relu / reluBackward / addBias / transpose2d / im2col / fills / copy and
batchNorm2d (inference) compute exactly the reference expressions
(cpu_backend.ixx:317-346, :433-446, :544-575, :781-842, :1535-1539), so the
bar is bitwise equality, NaN / signed-zero / infinity cases included.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


SPECIAL = np.array([np.nan, -np.nan, -0.0, 0.0, -1.0, 1.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38],
                   np.float32)


@pytest.mark.parametrize("n", [1, 7, 12, 1000, 4097, 1 << 20])
def test_relu_bitexact(hip, n):
    x = O.randn((n,), n)
    x[: min(n, SPECIAL.size)] = SPECIAL[: min(n, SPECIAL.size)]
    dx, dy = to_dev(hip, x), empty_dev(hip, (n,))
    hip.HIPBackend.relu(dx, dy, n)
    assert np.array_equal(bits(dy.numpy()), bits(O.relu(x)))
    assert np.array_equal(bits(O.relu(x)), bits(O.relu(x, backend="reference"))) if O.ref_lib() else True


def test_relu_unaligned_and_inplace(hip):
    n = 1001
    x = O.randn((n + 1,), 3)
    dx = to_dev(hip, x)
    dy = empty_dev(hip, (n + 1,))
    # offset by one float: exercises the scalar path
    hip.call("omHipReLU", dx.ptr + 4, dy.ptr + 4, n)
    assert np.array_equal(bits(dy.numpy()[1:]), bits(O.relu(x[1:])))
    hip.call("omHipReLU", dx.ptr, dx.ptr, n + 1)   # in place
    assert np.array_equal(bits(dx.numpy()), bits(O.relu(x)))


def test_relu_backward_bitexact(hip):
    n = 5003
    x = O.randn((n,), 5)
    x[:SPECIAL.size] = SPECIAL
    g = O.randn((n,), 6)
    dx, dg, dgi = to_dev(hip, x), to_dev(hip, g), empty_dev(hip, (n,))
    hip.HIPBackend.reluBackward(dx, dg, dgi, n)
    assert np.array_equal(bits(dgi.numpy()), bits(O.relu_backward(x, g)))


@pytest.mark.parametrize("b,c", [(128, 256), (128, 10), (3, 7), (1, 1)])
def test_add_bias_rows(hip, b, c):
    A = O.randn((b, c), b + c)
    bias = O.randn((c,), 7)
    dA, dB, dO = to_dev(hip, A), to_dev(hip, bias), empty_dev(hip, (b, c))
    hip.HIPBackend.addBias(dA, dB, dO, b, c)
    assert np.array_equal(bits(dO.numpy()), bits(O.add_bias(A, bias)))


def test_add_bias_nchw(hip):
    x = O.randn((2, 5, 3, 4), 8)
    bias = O.randn((5,), 9)
    dx, db, do = to_dev(hip, x), to_dev(hip, bias), empty_dev(hip, x.shape)
    hip.call("omHipAddBias", dx.ptr, db.ptr, do.ptr, 2, 5, 12)
    assert np.array_equal(do.numpy(), x + bias[None, :, None, None])


@pytest.mark.parametrize("r,c", [(1, 1), (3, 5), (64, 197), (197, 64), (1000, 33), (784, 256)])
def test_transpose_exact(hip, r, c):
    A = O.randn((r, c), r * c)
    dA, dB = to_dev(hip, A), empty_dev(hip, (c, r))
    hip.HIPBackend.transpose2d(dA, dB, r, c)
    assert np.array_equal(dB.numpy(), O.transpose2d(A))


@pytest.mark.parametrize("geom", [(2, 4, 8, 8), (32, 64, 56, 56), (1, 3, 1, 1), (3, 7, 5, 9)])
def test_batchnorm_eval_bitexact(hip, geom):
    N, C, H, W = geom
    x = O.randn(geom, sum(geom))
    g, b, m, v = O.uniform((C,), 1, 0.5, 1.5), O.randn((C,), 2, 0.1), O.randn((C,), 3, 0.1), O.uniform((C,), 4, 0.5, 1.5)
    y_ref, sm_ref, si_ref = O.batchnorm2d_eval(x, g, b, m, v)
    dx, dy = to_dev(hip, x), empty_dev(hip, geom)
    dg, db, dm, dv = (to_dev(hip, a) for a in (g, b, m, v))
    dsm, dsi = empty_dev(hip, (C,)), empty_dev(hip, (C,))
    hip.HIPBackend.batchNorm2d(dx, dy, dg, db, dm, dv, dsm, dsi, N, C, H, W, 1e-5, 0.1, False)
    assert np.array_equal(bits(dy.numpy()), bits(y_ref))
    assert np.array_equal(bits(dsm.numpy()), bits(sm_ref))
    assert np.array_equal(bits(dsi.numpy()), bits(si_ref))
    # running statistics are untouched in inference mode
    assert np.array_equal(dm.numpy(), m) and np.array_equal(dv.numpy(), v)


def test_batchnorm_null_pointer_rejected(hip):
    d = to_dev(hip, np.ones(4, np.float32))
    with pytest.raises(hip.OmHipError, match="null pointer"):
        hip.HIPBackend.batchNorm2d(d, d, None, d, d, d, d, d, 1, 1, 2, 2, 1e-5, 0.1, True)


@pytest.mark.parametrize("geom", [(3, 9, 9, 3, 3, 1, 1), (3, 9, 9, 3, 3, 2, 1), (2, 8, 8, 1, 1, 2, 0),
                                  (3, 32, 32, 7, 7, 2, 3), (4, 5, 7, 3, 2, 1, 0)])
def test_im2col_exact(hip, geom):
    Cin, H, W, KH, KW, s, p = geom
    x = O.randn((Cin, H, W), 77)
    Ho, Wo = (H + 2 * p - KH) // s + 1, (W + 2 * p - KW) // s + 1
    dx, dc = to_dev(hip, x), empty_dev(hip, (Cin * KH * KW, Ho * Wo))
    hip.HIPBackend.im2col(dx, Cin, H, W, KH, KW, p, p, s, s, dc)
    ref = np.empty((Cin * KH * KW, Ho * Wo), np.float32)
    O.lib().omrefIm2col(O._p(x), Cin, H, W, KH, KW, p, p, s, s, O._p(ref))
    assert np.array_equal(dc.numpy(), ref)


def test_fill_and_copy(hip):
    n = 12345
    d = empty_dev(hip, (n,))
    hip.HIPBackend.fillValue(d, n, 2.5)
    assert np.all(d.numpy() == 2.5)
    hip.HIPBackend.fillZeros(d, n)
    assert np.all(d.numpy() == 0)
    hip.HIPBackend.fillOnes(d, n - 1)
    h = d.numpy()
    assert np.all(h[:-1] == 1) and h[-1] == 0
    src = to_dev(hip, O.randn((n,), 1))
    hip.HIPBackend.copy(src, d, n)
    assert np.array_equal(d.numpy(), src.numpy())


def test_half_conversions(hip):
    x = np.concatenate([O.randn((10000,), 3) * 100, SPECIAL, np.array([65504, 65520, 1e-8, 6e-8, 2 ** -24], np.float32)])
    n = x.size
    dx, dh, dbf, dback = to_dev(hip, x), empty_dev(hip, (n,), np.uint16), empty_dev(hip, (n,), np.uint16), empty_dev(hip, (n,))
    hip.HIPBackend.convertToHalf(dx, dh, n)
    h = dh.numpy()
    expect = x.astype(np.float16).view(np.uint16)     # IEEE round-to-nearest-even
    nan = np.isnan(x)
    assert np.array_equal(h[~nan], expect[~nan])
    assert np.all(np.isnan(h[nan].view(np.float16)))
    hip.HIPBackend.convertToHalf(dx, dbf, n, bf16=True)
    assert np.array_equal(dbf.numpy()[~nan], O.bf16_bits(x)[~nan])
    hip.HIPBackend.convertFromHalf(dh, dback, n)
    assert np.array_equal(dback.numpy()[~nan], x.astype(np.float16).astype(np.float32)[~nan])
    hip.HIPBackend.convertFromHalf(dbf, dback, n, bf16=True)
    assert np.array_equal(dback.numpy()[~nan], O.bf16_round(x)[~nan])
