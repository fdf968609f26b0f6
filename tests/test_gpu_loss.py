"""Softmax, cross-entropy, their joint gradient and the bias gradient on the GPU.

Reference: CPUBackend::softmax / crossEntropy / crossEntropySoftmaxBackward
(cpu_backend.ixx:352-410) and AddBiasBackward (autograd.ixx:399-433), through
the oracle on the same inputs.

Bars:
  * softmax: per element |p - p_ref| <= 2^-24 * (8 + 2(n - 1)) * p_ref + 2^-126 — both
    sides compute the same x - max, so they differ by the exp implementations (an ulp
    each) and two fixed-order sums of n positive terms; below the normal range (2^-126)
    the difference is absolute; NaN where the oracle has NaN;
  * loss: 1e-6 relative (a sum of one log per row, in a different order);
  * joint gradient: bit for bit (one subtraction and one multiplication);
  * bias gradient: bit for bit when the rows are added in order (nHW = 1, up to
    4096 rows); otherwise |db - db64| <= 2^-24 * (L + 16) * sum|g|, L being the
    longest run added in order (a row part, or a thread's share of a plane);
  * the fused entry equals the three separate calls bit for bit.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _softmax_ok(p, x, ref):
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(p), nan)
    budget = 2.0 ** -24 * (8.0 + 2.0 * (x.shape[-1] - 1))
    ok = np.abs(p[~nan] - ref[~nan]) <= budget * ref[~nan] + 2.0 ** -126
    assert np.all(ok), float(np.max(np.abs(p[~nan] - ref[~nan]) / np.maximum(ref[~nan], 1e-38)))


@pytest.mark.parametrize("rows,cols", [(128, 10), (64, 197), (7, 1000), (3, 5000), (1, 1), (130, 63)])
def test_softmax(hip, rows, cols):
    x = O.randn((rows, cols), rows * 7 + cols, 6.0)
    if cols >= 20:
        x[0, 3:9] = 4.0                              # tied maxima
        x[-1] *= 50.0                                # most of the row underflows
    print(f"case softmax {rows}x{cols}", flush=True)
    dx, dy = to_dev(hip, x), empty_dev(hip, (rows, cols))
    hip.HIPBackend.softmax(dx, dy, rows, cols)
    _softmax_ok(dy.numpy(), x, O.softmax(x))


def test_softmax_special_values(hip):
    """A NaN first element propagates (the reference's scan keeps it as the maximum); a NaN
    elsewhere makes the row NaN through the sum; -inf gives 0; a row of equal values gives
    1/n exactly."""
    x = O.randn((5, 70), 3, 2.0)
    x[0, 0] = np.nan
    x[1, 33] = np.nan
    x[2, [1, 40, 69]] = -np.inf
    x[3] = 0.25
    x[4, 64] = 80.0                                   # the maximum sits in the second lane pass
    dx, dy = to_dev(hip, x), empty_dev(hip, x.shape)
    hip.HIPBackend.softmax(dx, dy, 5, 70)
    p, ref = dy.numpy(), O.softmax(x)
    _softmax_ok(p, x, ref)
    assert np.all(np.isnan(p[0])) and np.all(np.isnan(p[1]))
    assert np.all(p[2, [1, 40, 69]] == 0.0)
    assert np.array_equal(_bits(p[3]), _bits(np.full(70, np.float32(1.0) / np.float32(70.0))))


@pytest.mark.parametrize("rows,cols", [(128, 10), (33, 1000)])
def test_cross_entropy_and_gradient(hip, rows, cols):
    H = hip.HIPBackend
    p = O.softmax(O.randn((rows, cols), 5, 3.0))
    lab = O.rng(6).integers(0, cols, rows)
    t = np.eye(cols, dtype=np.float32)[lab]
    p[0, lab[0]] = 0.0                                # clamped to 1e-7
    t[1, (lab[1] + 1) % cols] = 0.9                   # a second target above 0.5
    dp, dt = to_dev(hip, p), to_dev(hip, t)
    dl, dg = empty_dev(hip, (1,)), empty_dev(hip, (rows, cols))
    H.crossEntropyForward(dp, dt, dl, rows, cols)
    H.crossEntropySoftmaxBackward(dp, dt, dg, rows, cols)
    loss, ref = float(dl.numpy()[0]), O.cross_entropy(p, t)
    assert abs(loss - ref) <= 1e-6 * abs(ref)
    assert np.array_equal(_bits(dg.numpy()), _bits(O.cross_entropy_softmax_backward(p, t)))


@pytest.mark.parametrize("rows,cols", [(128, 10), (200, 1000), (16, 7), (300, 200), (129, 64), (1, 65)])
def test_fused_softmax_cross_entropy(hip, rows, cols):
    """omHipSoftmaxCrossEntropy = softmax -> crossEntropy -> crossEntropySoftmaxBackward, bit for
    bit, with every combination of outputs requested."""
    H = hip.HIPBackend
    x = O.randn((rows, cols), 8, 4.0)
    t = np.eye(cols, dtype=np.float32)[O.rng(9).integers(0, cols, rows)]
    dx, dt = to_dev(hip, x), to_dev(hip, t)
    p1, l1, g1 = empty_dev(hip, (rows, cols)), empty_dev(hip, (1,)), empty_dev(hip, (rows, cols))
    H.softmax(dx, p1, rows, cols)
    H.crossEntropyForward(p1, dt, l1, rows, cols)
    H.crossEntropySoftmaxBackward(p1, dt, g1, rows, cols)
    want_p, want_l, want_g = p1.numpy(), l1.numpy(), g1.numpy()
    for with_p, with_g in [(True, True), (False, True), (True, False), (False, False)]:
        p2 = empty_dev(hip, (rows, cols)) if with_p else None
        g2 = empty_dev(hip, (rows, cols)) if with_g else None
        l2 = empty_dev(hip, (1,))
        H.softmaxCrossEntropy(dx, dt, p2, l2, g2, rows, cols)
        assert _bits(l2.numpy())[0] == _bits(want_l)[0], (with_p, with_g)
        if with_p:
            assert np.array_equal(_bits(p2.numpy()), _bits(want_p)), (with_p, with_g)
        if with_g:
            assert np.array_equal(_bits(g2.numpy()), _bits(want_g)), (with_p, with_g)


@pytest.mark.parametrize("N,C", [(128, 256), (128, 10), (4096, 37), (1, 5), (257, 3000)])
def test_bias_gradient_rows_in_order(hip, N, C):
    g = O.randn((N, C), N + C)
    dg, db = to_dev(hip, g), empty_dev(hip, (C,))
    hip.HIPBackend.addBiasBackward(dg, db, N, C, 1)
    assert np.array_equal(_bits(db.numpy()), _bits(O.add_bias_backward(g, N, C)))


@pytest.mark.parametrize("N,C,HW", [(12608, 768, 1), (5000, 17, 1), (32, 64, 3136), (3, 5, 7)])
def test_bias_gradient_parts(hip, N, C, HW):
    """Many rows (16 ordered parts) and conv-layout planes (a fixed tree per channel)."""
    g = O.randn((N, C, HW), 17)
    dg, db = to_dev(hip, g), empty_dev(hip, (C,))
    hip.HIPBackend.addBiasBackward(dg, db, N, C, HW)
    g64 = g.astype(np.float64)
    want = g64.sum(axis=(0, 2))
    absum = np.abs(g64).sum(axis=(0, 2))
    run = (N + 15) // 16 if HW == 1 else N * ((HW + 255) // 256)
    assert np.all(np.abs(db.numpy() - want) <= 2.0 ** -24 * (run + 16) * absum)


def test_bias_gradient_degenerate(hip):
    db = to_dev(hip, np.full(6, 3.0, np.float32))
    hip.HIPBackend.addBiasBackward(None, db, 0, 6, 1)
    assert np.all(db.numpy() == 0.0)
