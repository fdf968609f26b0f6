"""The reference's own network definitions on the HAL entries, in its op order.

ResNet18 as resnet.ixx:186-254 writes it (3x3 stride-1 stem, max pool only for
inputs taller than 32, BasicBlock conv1 -> bn1 -> relu -> conv2 -> bn2 -> + shortcut
-> relu), ResNet50 as resnet50.ixx:202-279 (3x3 stem, no max pool, Bottleneck
1x1 -> 3x3 -> 1x1 with the shortcut summed after bn3), and the Bottleneck blocks
of the benchmark's ResNet-50 stack at their real shapes. The GPU side fuses
each conv's BN and ReLU and the block's shortcut sum into the conv epilogue;
the CPU side is the reference's unfused chain through the oracle.

Bars (relative Frobenius error against the oracle chain): block outputs <= 1e-5,
logits <= 1e-4 (the network bar), and the same top-1 class per image.
"""
import numpy as np
import pytest

import oracle as O
import ref_nets as R
from conftest import to_dev

pytestmark = pytest.mark.gpu


def _block_params(cin, wd, ds, seed):
    P = {}
    P["b.conv1.w"] = R._kaiming((wd, cin, 1, 1), seed)
    R._bn(P, "b.bn1", wd, seed + 1)
    P["b.conv2.w"] = R._kaiming((wd, wd, 3, 3), seed + 2)
    R._bn(P, "b.bn2", wd, seed + 3)
    P["b.conv3.w"] = R._kaiming((4 * wd, wd, 1, 1), seed + 4)
    R._bn(P, "b.bn3", 4 * wd, seed + 5)
    if ds:
        P["b.ds.w"] = R._kaiming((4 * wd, cin, 1, 1), seed + 6)
        R._bn(P, "b.dsbn", 4 * wd, seed + 7)
    return P


# (name, Cin, H, width, stride, downsample): ResNet-50 stack blocks at 224x224
BLOCKS = [("l1.0", 64, 56, 64, 1, True), ("l2.0", 256, 56, 128, 2, True), ("l2.1", 512, 28, 128, 1, False),
          ("l3.1", 1024, 14, 256, 1, False), ("l4.0", 1024, 14, 512, 2, True), ("l4.2", 2048, 7, 512, 1, False)]


@pytest.mark.parametrize("blk", BLOCKS, ids=[b[0] for b in BLOCKS])
def test_bottleneck_block(hip, blk):
    name, cin, h, wd, s, ds = blk
    P = _block_params(cin, wd, ds, 300 + cin + wd)
    x = O.randn((2, cin, h, h), 400 + cin)
    print(f"case bottleneck {name} b2", flush=True)
    net = R.GpuNet(hip, P)
    y, ho, wo = net.bottleneck(to_dev(hip, x), 2, h, h, "b", cin, wd, s, ds)
    got = y.numpy()
    ref = R.cpu_bottleneck(P, x, "b", s, ds)
    assert got.shape == ref.shape == (2, 4 * wd, ho, wo)
    err = O.frobenius_rel(got, ref)
    print(f"[bottleneck {name}] rel Frobenius error {err:.2e}")
    assert err <= 1e-5


@pytest.mark.parametrize("case", [(4, 1, 28, 10), (2, 3, 64, 10), (2, 3, 32, 100)],
                         ids=["mnist28_nopool", "rgb64_maxpool", "rgb32_nopool"])
def test_reference_resnet18(hip, case):
    N, cin, hw, classes = case
    P = R.make_resnet18(cin, classes, seed=11)
    img = O.randn((N, cin, hw, hw), 12 + hw)
    print(f"case resnet18 (reference layout) {case}", flush=True)
    net = R.GpuNet(hip, P)
    logits = net.resnet18(to_dev(hip, img), N, cin, hw, hw, classes).numpy()
    ref = R.cpu_resnet18(P, img)
    err = O.frobenius_rel(logits, ref)
    print(f"[resnet18 reference layout {case}] logits rel Frobenius error {err:.2e}")
    assert err <= 1e-4
    assert np.array_equal(np.argmax(logits, axis=1), np.argmax(ref, axis=1))


def test_reference_resnet50(hip):
    N, cin, hw, classes = 2, 3, 32, 10
    P = R.make_resnet50(cin, classes, seed=21)
    img = O.randn((N, cin, hw, hw), 22)
    print("case resnet50 (reference layout) 2x3x32x32", flush=True)
    net = R.GpuNet(hip, P)
    logits = net.resnet50(to_dev(hip, img), N, cin, hw, hw, classes).numpy()
    ref = R.cpu_resnet50(P, img)
    err = O.frobenius_rel(logits, ref)
    print(f"[resnet50 reference layout] logits rel Frobenius error {err:.2e}")
    assert err <= 1e-4
    assert np.array_equal(np.argmax(logits, axis=1), np.argmax(ref, axis=1))
