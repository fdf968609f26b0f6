"""MLP 784->256->128->10 forward + backward through the HAL (batch 128, fp32).

The reference step (train_main.cpp / Linear, linear.ixx:50-58; MatMulBackward,
autograd.ixx:226-290) is: y = x @ W + b, ReLU, ...; backward dA = G x B^T,
dW = A^T x G, ReLU mask. On the GPU the transposes are folded into the
MatmulTransB / MatmulTransA entries. Each GPU op is checked in situ against
the oracle applied to the same (GPU-produced) inputs with the K-scaled bound,
and the whole step against the oracle-only chain.
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


def _ce_grad(logits, labels):
    z = logits.astype(np.float64)
    z = z - z.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    p[np.arange(len(labels)), labels] -= 1.0
    return (p / len(labels)).astype(np.float32)


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

    # ---------------- backward ----------------
    G = _ce_grad(logits, labels)
    dG = to_dev(hip, G)
    for k in reversed(range(len(LAYERS))):
        i, o = LAYERS[k]
        A = acts[k]
        dWg = empty_dev(hip, (i, o))
        H.matmulTransA(d_acts[k], dG, dWg, i, BATCH, o)          # dW = A^T G
        dA_ref, dW_ref = O.matmul_backward(G, A, Ws[k])
        _, bW = O.gemm_f64(A, G, transA=True)
        assert O.normalized_error(dWg.numpy(), dW_ref, bW) <= TOL
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
