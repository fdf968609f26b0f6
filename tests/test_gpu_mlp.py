"""MLP 784->256->128->10 forward + backward through the HAL (batch 128, fp32).

The reference step (train_main.cpp / Linear, linear.ixx:50-58; MatMulBackward,
autograd.ixx:226-290; tensorSoftmaxCrossEntropy tensor_ops.ixx:583-633 with
SoftmaxCrossEntropyBackward autograd.ixx:440-488; AddBiasBackward
autograd.ixx:399-433) is: y = x @ W + b, ReLU, ...; softmax, cross-entropy
against one-hot labels, joint gradient (p - t) / batch; backward dA = G x B^T,
dW = A^T x G, db = column sums of G, ReLU mask. On the GPU the transposes are
folded into the MatmulTransB / MatmulTransA entries. Each GPU op is checked in
situ against the oracle applied to the same (GPU-produced) inputs: GEMMs with
the K-scaled bound, softmax per element within 2^-24 * (8 + 2(n - 1))
relative plus 2^-126 absolute (one exp of identical arguments on both sides, two
fixed-order sums of n positive terms), the loss within 1e-6 relative, the joint gradient, ReLU
and the bias gradients (rows added in order) bit for bit.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu
TOL = O.TOL_FP32
LAYERS = [(784, 256), (256, 128), (128, 10)]
BATCH = 128


def _kaiming_uniform(fan_in, fan_out, seed):
    b = np.sqrt(6.0 / fan_in)
    return O.uniform((fan_in, fan_out), seed, -b, b)


def softmax_budget(x):
    """Per-element relative bar of the device softmax against the oracle's on the same rows."""
    return 2.0 ** -24 * (8.0 + 2.0 * (x.shape[-1] - 1))


def test_mlp_step(hip):
    H = hip.HIPBackend
    x = O.uniform((BATCH, 784), 1)
    labels = O.rng(2).integers(0, 10, BATCH)
    Ws = [_kaiming_uniform(i, o, 10 + k) for k, (i, o) in enumerate(LAYERS)]
    bs = [np.zeros(o, np.float32) for _, o in LAYERS]

    # ---------------- forward ----------------
    acts = [x]
    pre = []
    d_act = to_dev(hip, x)
    d_acts = [d_act]
    for k, (i, o) in enumerate(LAYERS):
        dW, db = to_dev(hip, Ws[k]), to_dev(hip, bs[k])
        dz = empty_dev(hip, (BATCH, o))
        H.matmul(d_acts[-1], dW, dz, BATCH, i, o)
        z_gpu = dz.numpy()
        z_ref = O.matmul(acts[-1], Ws[k])
        _, bound = O.gemm_f64(acts[-1], Ws[k])
        assert O.normalized_error(z_gpu, z_ref, bound) <= TOL
        H.addBias(dz, db, dz, BATCH, o)
        assert np.array_equal(dz.numpy(), O.add_bias(z_gpu, bs[k]))
        pre.append(dz.numpy())
        if k < len(LAYERS) - 1:
            da = empty_dev(hip, (BATCH, o))
            H.relu(dz, da, BATCH * o)
            assert np.array_equal(da.numpy(), O.relu(pre[-1]))
            d_acts.append(da)
            acts.append(da.numpy())
        else:
            logits = dz.numpy()

    # ---------------- loss ----------------
    T = np.eye(10, dtype=np.float32)[labels]
    d_logits, d_T = dz, to_dev(hip, T)
    d_p, d_loss, dG = empty_dev(hip, (BATCH, 10)), empty_dev(hip, (1,)), empty_dev(hip, (BATCH, 10))
    H.softmax(d_logits, d_p, BATCH, 10)
    H.crossEntropyForward(d_p, d_T, d_loss, BATCH, 10)
    H.crossEntropySoftmaxBackward(d_p, d_T, dG, BATCH, 10)
    p_gpu, p_ref = d_p.numpy(), O.softmax(logits)
    assert np.all(np.abs(p_gpu - p_ref) <= softmax_budget(logits) * p_ref + 2.0 ** -126)
    loss = float(d_loss.numpy()[0])
    assert abs(loss - O.cross_entropy(p_gpu, T)) <= 1e-6 * abs(loss)
    G = dG.numpy()
    assert np.array_equal(G.view(np.uint32), O.cross_entropy_softmax_backward(p_gpu, T).view(np.uint32))

    # ---------------- backward ----------------
    for k in reversed(range(len(LAYERS))):
        i, o = LAYERS[k]
        A = acts[k]
        dWg = empty_dev(hip, (i, o))
        H.matmulTransA(d_acts[k], dG, dWg, i, BATCH, o)          # dW = A^T G
        dA_ref, dW_ref = O.matmul_backward(G, A, Ws[k])
        _, bW = O.gemm_f64(A, G, transA=True)
        assert O.normalized_error(dWg.numpy(), dW_ref, bW) <= TOL
        dbg = empty_dev(hip, (o,))
        H.addBiasBackward(dG, dbg, BATCH, o, 1)                  # db = column sums of G
        assert np.array_equal(dbg.numpy().view(np.uint32), O.add_bias_backward(G, BATCH, o).view(np.uint32))
        if k == 0:
            break
        dAg = empty_dev(hip, (BATCH, i))
        H.matmulTransB(dG, to_dev(hip, Ws[k]), dAg, BATCH, o, i)  # dA = G W^T
        _, bA = O.gemm_f64(G, Ws[k], transB=True)
        assert O.normalized_error(dAg.numpy(), dA_ref, bA) <= TOL
        dGprev = empty_dev(hip, (BATCH, i))
        H.reluBackward(to_dev(hip, pre[k - 1]), dAg, dGprev, BATCH * i)
        assert np.array_equal(dGprev.numpy(), O.relu_backward(pre[k - 1], dAg.numpy()))
        G = dGprev.numpy()
        dG = dGprev


@pytest.mark.parametrize("M,K,N", [(128, 784, 256), (128, 128, 10), (37, 29, 53), (64, 4096, 96)])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("with_bias", [True, False])
def test_linear_bias_act(hip, M, K, N, act, with_bias):
    """The fused Linear entry equals the unfused HAL chain (matmul -> addBias ->
    ReLU) bit for bit, and the oracle chain under the K-scaled bound. 64 x 4096
    x 96 takes the split-K path (bias and ReLU applied by the finishing sum)."""
    H = hip.HIPBackend
    A = O.randn((M, K), 51)
    W = O.randn((K, N), 52, 0.05)
    b = O.randn((N,), 53, 0.5) if with_bias else None
    dA, dW = to_dev(hip, A), to_dev(hip, W)
    db = to_dev(hip, b) if with_bias else None
    fused, ref = empty_dev(hip, (M, N)), empty_dev(hip, (M, N))
    print(f"case linear M={M} K={K} N={N} act={act} bias={with_bias}", flush=True)
    H.linearBiasAct(dA, dW, db, fused, M, K, N, act)
    H.matmul(dA, dW, ref, M, K, N)
    if with_bias:
        H.addBias(ref, db, ref, M, N)
    if act:
        H.relu(ref, ref, M * N)
    got, want = fused.numpy(), ref.numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y = O.matmul(A, W)
    if with_bias:
        y = O.add_bias(y, b)
    if act:
        y = O.relu(y)
    C64, bound = O.gemm_f64(A, W)
    assert O.normalized_error(got, y, bound + (np.abs(b)[None, :] if with_bias else 0)) <= TOL


# (batch, in, out): the three MLP layers at batch 128, ragged sizes, sizes that are not
# whole 16-byte vectors (scalar loaders) and a batch above one K slice of 16 rows.
LINEAR_BACKWARD_SHAPES = [(128, 784, 256), (128, 256, 128), (128, 128, 10), (37, 50, 3), (64, 64, 64), (5, 130, 66),
                          (300, 96, 40)]


@pytest.mark.parametrize("nb,ni,no", LINEAR_BACKWARD_SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("gated", [False, True], ids=["plain", "relu_gate"])
def test_linear_backward(hip, nb, ni, no, gated):
    """omHipLinearBackward (dW = X^T G, db = column sums of G, dX = G W^T, gated by the layer
    below's ReLU output) against the separate entries it fuses, bit for bit (none of these
    products splits K), and against the oracle within the K-scaled bound."""
    H = hip.HIPBackend
    x = O.randn((nb, ni), nb + ni)
    x[x < 0] *= 0.0   # a ReLU output: the gate of the layer below (zeros where it was inactive)
    g = O.randn((nb, no), nb + no + 1)
    w = _kaiming_uniform(ni, no, ni + no)
    dx_, dg, dw = to_dev(hip, x), to_dev(hip, g), to_dev(hip, w)
    gW, gb, gX = empty_dev(hip, (ni, no)), empty_dev(hip, (no,)), empty_dev(hip, (nb, ni))
    H.linearBackward(dx_, dg, dw, dx_ if gated else None, gW, gb, gX, nb, ni, no)
    # the separate entries
    cW, cb, cX = empty_dev(hip, (ni, no)), empty_dev(hip, (no,)), empty_dev(hip, (nb, ni))
    H.matmulTransA(dx_, dg, cW, ni, nb, no)
    H.addBiasBackward(dg, cb, nb, no, 1)
    H.matmulTransB(dg, dw, cX, nb, no, ni)
    if gated:
        H.reluBackward(dx_, cX, cX, nb * ni)
    for got, want in ((gW, cW), (gb, cb), (gX, cX)):
        assert np.array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32))
    # the oracle
    refW, bW = O.gemm_f64(x, g, transA=True)
    assert O.normalized_error(gW.numpy(), refW, bW) <= TOL
    assert np.array_equal(gb.numpy(), O.add_bias_backward(g, nb, no))   # rows added in order from 0
    refX, bX = O.gemm_f64(g, w, transB=True)
    if gated:
        refX = np.where(x > 0, refX, 0.0)
    assert O.normalized_error(gX.numpy(), refX, bX) <= TOL


def test_linear_backward_optional_outputs(hip):
    """Null db / dX are skipped; the outputs that are asked for match the full call's."""
    H = hip.HIPBackend
    nb, ni, no = 96, 72, 40
    x, g, w = O.randn((nb, ni), 5), O.randn((nb, no), 6), O.randn((ni, no), 7)
    dx_, dg, dw = to_dev(hip, x), to_dev(hip, g), to_dev(hip, w)
    full = [empty_dev(hip, s) for s in ((ni, no), (no,), (nb, ni))]
    H.linearBackward(dx_, dg, dw, None, *full, nb, ni, no)
    only_w = empty_dev(hip, (ni, no))
    H.linearBackward(dx_, dg, None, None, only_w, None, None, nb, ni, no)
    assert np.array_equal(only_w.numpy(), full[0].numpy())


def test_linear_backward_degenerate(hip):
    """No rows: dW and db are zero. No output features: dX is zero (gated or not)."""
    H = hip.HIPBackend
    gW, gb = to_dev(hip, np.full((8, 4), 7.0, np.float32)), to_dev(hip, np.full((4,), 7.0, np.float32))
    x, g, w = to_dev(hip, O.randn((1, 8), 1)), to_dev(hip, O.randn((1, 4), 2)), to_dev(hip, O.randn((8, 4), 3))
    H.linearBackward(x, g, w, None, gW, gb, None, 0, 8, 4)
    assert not gW.numpy().any() and not gb.numpy().any()
    gX = to_dev(hip, np.full((3, 8), 7.0, np.float32))
    xs = to_dev(hip, np.abs(O.randn((3, 8), 4)))
    H.linearBackward(xs, g, w, xs, None, None, gX, 3, 8, 0)
    assert not gX.numpy().any()


# (batch, in, classes): the MLP's 128 x 128 x 10 head and ragged sizes in one workgroup;
# 512 and 1000 rows (a last block of 40), 300 x 70 (K % 4 != 0) and 64 x 200 x 64 (LDS
# for 32 rows only) in blocks of rows; and two heads the fused kernel does not take
# (100 classes; 4000 rows, whose gradient and terms exceed the last workgroup's LDS):
# the separate entries run those.
HEAD_STEP_SHAPES = [(128, 128, 10), (100, 70, 13), (33, 16, 1), (256, 128, 10), (512, 128, 10), (1000, 64, 10),
                    (300, 70, 13), (64, 200, 64), (512, 256, 10), (64, 32, 100), (4000, 16, 10)]


def _head_mode(nb, ni, nc):
    """Which kernel omHipLinearSoftmaxCrossEntropyStep runs for these sizes: "single" (the
    whole batch in one workgroup: at most 256 rows padded to 16), "rows" (a workgroup per
    block of 64, 32 or 16 rows, the whole batch's gradient and terms in the last one's LDS)
    or None (the separate entries). LDS budget 128 KiB, row strides 17 mod 64."""
    pad = lambda v: -(-v // 16) * 16
    s17 = lambda v: v + (17 - v % 64) % 64
    if nc > 64:
        return None
    kp, np_ = pad(ni), pad(nc)
    block = lambda r: 4 * (r * s17(kp) + kp * s17(np_) + r * s17(np_) + r * nc + r)
    if pad(nb) <= 256 and block(pad(nb)) <= 128 * 1024:
        return "single"
    if 4 * (nb * nc + nb) <= 128 * 1024 and any(block(r) <= 128 * 1024 for r in (64, 32, 16)):
        return "rows"
    return None


@pytest.mark.parametrize("nb,ni,nc", HEAD_STEP_SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("gated", [False, True], ids=["plain", "relu_gate"])
def test_linear_softmax_ce_step(hip, nb, ni, nc, gated):
    """omHipLinearSoftmaxCrossEntropyStep: logits and the three products against float64 (K-scaled
    bound); the logit gradient against the oracle's softmax of the step's own logits within the
    softmax bar above (times 1/batch, plus the roundings of p - t and of the product by
    1/batch); the loss against the oracle's
    cross-entropy of those probabilities within 1e-5 relative; the bias gradient bit for bit
    (rows added in order from 0). Heads the fused kernel does not take run the separate entries:
    there the loss and the logit gradient are also bit-identical to omHipSoftmaxCrossEntropy's.
    The second call (only the weight gradient asked for) reproduces the first's bit for bit,
    which also shows the first left its arrival counter at zero."""
    H = hip.HIPBackend
    x = O.randn((nb, ni), nb + ni)
    x[x < 0] *= 0.0   # a ReLU output: the gate of the layer below
    w = _kaiming_uniform(ni, nc, ni + nc)
    b = O.randn((nc,), nc, 0.1)
    T = np.eye(nc, dtype=np.float32)[O.rng(nb).integers(0, nc, nb)]
    dx_, dw, db, dT = to_dev(hip, x), to_dev(hip, w), to_dev(hip, b), to_dev(hip, T)
    z, loss, g = empty_dev(hip, (nb, nc)), empty_dev(hip, (1,)), empty_dev(hip, (nb, nc))
    gW, gb, gX = empty_dev(hip, (ni, nc)), empty_dev(hip, (nc,)), empty_dev(hip, (nb, ni))
    print(f"case head step {nb}x{ni}x{nc} gated {gated} mode {_head_mode(nb, ni, nc)}", flush=True)
    H.linearSoftmaxCrossEntropyStep(dx_, dw, db, dT, dx_ if gated else None, z, loss, g, gW, gb, gX, nb, ni, nc)
    zg, gg = z.numpy(), g.numpy()
    z64, bz = O.gemm_f64(x, w)
    assert O.normalized_error(zg, z64 + b, bz + np.abs(b)) <= TOL
    p_ref = O.softmax(zg)
    g_ref = O.cross_entropy_softmax_backward(p_ref, T)
    # the roundings of p - t and of the product by fl(1/batch) (inexact when batch is not a
    # power of two), on both sides: 3 * 2^-24 |p - t| / batch
    bar = (softmax_budget(zg) * p_ref + 3 * 2.0 ** -24 * np.abs(p_ref - T) + 2.0 ** -126) / nb * 1.0001
    assert np.all(np.abs(gg - g_ref) <= bar)
    lv = float(loss.numpy()[0])
    assert abs(lv - O.cross_entropy(p_ref, T)) <= 1e-5 * abs(lv)
    if _head_mode(nb, ni, nc) is None:   # the separate entries ran
        loss2, g2 = empty_dev(hip, (1,)), empty_dev(hip, (nb, nc))
        H.softmaxCrossEntropy(z, dT, None, loss2, g2, nb, nc)
        assert np.array_equal(loss.numpy().view(np.uint32), loss2.numpy().view(np.uint32))
        assert np.array_equal(gg.view(np.uint32), g2.numpy().view(np.uint32))
    refW, bW = O.gemm_f64(x, gg, transA=True)
    assert O.normalized_error(gW.numpy(), refW, bW) <= TOL
    assert np.array_equal(gb.numpy(), O.add_bias_backward(gg, nb, nc))
    refX, bX = O.gemm_f64(gg, w, transB=True)
    if gated:
        refX = np.where(x > 0, refX, 0.0)
    assert O.normalized_error(gX.numpy(), refX, bX) <= TOL
    # optional outputs: only the weight gradient asked for
    gW2 = empty_dev(hip, (ni, nc))
    H.linearSoftmaxCrossEntropyStep(dx_, dw, db, dT, None, None, None, None, gW2, None, None, nb, ni, nc)
    assert np.array_equal(gW2.numpy(), gW.numpy())


@pytest.mark.parametrize("nb,ni,nc", [(128, 128, 10), (300, 128, 13)], ids=lambda v: str(v))
def test_linear_softmax_ce_step_unaligned(hip, nb, ni, nc):
    """The head's scalar paths: the input, a separate gate (the ReLU output below, equal to
    the input) and the input gradient 4 bytes past 16-byte alignment take the element-wise
    copy, gate and store paths of the fused kernel (one workgroup at 128 rows, row blocks at
    300). Every output equals the aligned call's (the input as its own gate) bit for bit."""
    H = hip.HIPBackend
    x = O.randn((nb, ni), 77 + nb)
    x[x < 0] *= 0.0
    w = _kaiming_uniform(ni, nc, 5 + nc)
    b = O.randn((nc,), nc + 1, 0.1)
    T = np.eye(nc, dtype=np.float32)[O.rng(nb + 1).integers(0, nc, nb)]
    dx, dw, db, dT = to_dev(hip, x), to_dev(hip, w), to_dev(hip, b), to_dev(hip, T)
    outs = lambda: (empty_dev(hip, (nb, nc)), empty_dev(hip, (1,)), empty_dev(hip, (nb, nc)),
                    empty_dev(hip, (ni, nc)), empty_dev(hip, (nc,)))
    z1, l1, g1, w1, b1 = outs()
    gx1 = empty_dev(hip, (nb, ni))
    print(f"case head step aligned {nb}x{ni}x{nc}", flush=True)
    H.linearSoftmaxCrossEntropyStep(dx, dw, db, dT, dx, z1, l1, g1, w1, b1, gx1, nb, ni, nc)
    # the same operands one float into buffers one float longer
    pad = np.zeros((1,), np.float32)
    xs = to_dev(hip, np.concatenate([pad, x.ravel()]))
    gs = to_dev(hip, np.concatenate([pad, x.ravel()]))
    gxs = to_dev(hip, np.full((nb * ni + 1,), 7.0, np.float32))
    z2, l2, g2, w2, b2 = outs()
    print(f"case head step unaligned {nb}x{ni}x{nc}", flush=True)
    H.linearSoftmaxCrossEntropyStep(xs.ptr + 4, dw, db, dT, gs.ptr + 4, z2, l2, g2, w2, b2, gxs.ptr + 4, nb, ni, nc)
    same = lambda a, c: np.array_equal(a.view(np.uint32), c.view(np.uint32))
    for a, c in ((z1, z2), (l1, l2), (g1, g2), (w1, w2), (b1, b2)):
        assert same(a.numpy(), c.numpy())
    gxu = gxs.numpy()
    assert gxu[0] == 7.0   # nothing written before the view
    assert same(gx1.numpy().ravel(), gxu[1:])
