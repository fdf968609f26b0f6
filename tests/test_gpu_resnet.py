"""ResNet-18 end to end on libomhip against the reference chain on the CPU.

Inference: the fused network (conv + BN + ReLU epilogues, residual sums in the
second conv of each block, max pool, global average pool, FC) against the
unfused reference chain conv2d -> batchNorm2d(eval) -> relu / add / maxPool2d /
adaptiveAvgPool2d / matmul + addBias (oracle) on the same two images.
Training: one forward with batch statistics and the backward pass; every conv
weight gradient and the FC gradients against the same step on the CPU.

Bars (relative Frobenius error): logits <= 1e-4. The training step is
checked in two halves, because the reference is ill-conditioned across them:
a ReLU input within a few ulps of zero (or a max-pool near-tie) takes
different sides in two valid fp32 evaluations and reroutes a gradient, which
moves early-layer gradients by ~1e-2 for differences of 1e-5 in the forward.
So (1) every forward intermediate of the GPU step (conv outputs, BN outputs
and saved statistics, block sums) must be within 1e-4 of the CPU forward, and
(2) the GPU gradients must be within 1e-3 of the reference backward replayed
on the GPU's own forward state (same ReLU / max-pool decisions).
"""
import numpy as np
import pytest

import oracle as O
from conftest import to_dev
from resnet_net import GpuResNet18, conv_list, cpu_backward, cpu_forward, cpu_forward_train, make_params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def params():
    return make_params(seed=3)


def test_resnet18_inference(hip, params):
    img = O.randn((2, 3, 224, 224), 41)
    net = GpuResNet18(hip, params, 2)
    logits = net.forward(to_dev(hip, img)).numpy()
    ref = cpu_forward(params, img)
    err = O.frobenius_rel(logits, ref)
    print(f"[resnet18 inference] logits rel Frobenius error {err:.2e}")
    assert err <= 1e-4
    assert np.array_equal(np.argsort(logits, axis=1)[:, -5:], np.argsort(ref, axis=1)[:, -5:])


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "reference_ops"])
def test_resnet18_train_step(hip, params, fused):
    img = O.randn((2, 3, 224, 224), 42)
    g_logits = O.randn((2, 1000), 43, 0.01)
    net = GpuResNet18(hip, params, 2, train=True, fused=fused)
    net.forward_train(to_dev(hip, img))
    net.backward(to_dev(hip, g_logits))
    got = net.grads()
    fwd_gpu = net.forward_state(img)
    fwd_cpu = cpu_forward_train(params, img)
    worst_f = 0.0
    for k, g in fwd_gpu.items():
        if k in ("img", "pool.idx"):
            continue
        v = fwd_cpu[k]
        e = O.frobenius_rel(g.reshape(v.shape), v)
        worst_f = max(worst_f, e)
        assert e <= 1e-4, k
    ref = cpu_backward(params, fwd_gpu, g_logits)
    worst = 0.0
    for name in [n for n, *_ in conv_list()] + ["fc.w", "fc.b"]:
        e = O.frobenius_rel(got[name].reshape(ref[name].shape), ref[name])
        worst = max(worst, e)
        assert e <= 1e-3, name
    print(f"[resnet18 train step] worst forward-state error {worst_f:.2e}, worst weight-gradient error {worst:.2e}")
