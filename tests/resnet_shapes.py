"""Conv shape sets of the benchmark configurations (NCHW, fp32).

ResNet-18 at 224x224 (torchvision layout: 7x7 s2 stem, 3x3 basic blocks, 1x1 s2
downsample): 20 convs. ResNet-50 at 224x224 (bottleneck 1x1-3x3-1x1, stride on
the 3x3, 1x1 s2 downsample): 53 convs. Each entry is
(name, Cin, H, W, Cout, K, stride, pad); the per-layer GEMM is
M = Cout, N = batch*Ho*Wo, K = Cin*K*K.
"""
from __future__ import annotations


def resnet18_convs():
    L = [("stem", 3, 224, 224, 64, 7, 2, 3)]
    for i in range(4):
        L.append((f"l1.{i}", 64, 56, 56, 64, 3, 1, 1))
    for stage, (cin, cout, hw) in enumerate([(64, 128, 56), (128, 256, 28), (256, 512, 14)], start=2):
        o = hw // 2
        L.append((f"l{stage}.0.conv1", cin, hw, hw, cout, 3, 2, 1))
        L.append((f"l{stage}.0.conv2", cout, o, o, cout, 3, 1, 1))
        L.append((f"l{stage}.0.ds", cin, hw, hw, cout, 1, 2, 0))
        L.append((f"l{stage}.1.conv1", cout, o, o, cout, 3, 1, 1))
        L.append((f"l{stage}.1.conv2", cout, o, o, cout, 3, 1, 1))
    assert len(L) == 20
    return L


def resnet50_convs():
    L = [("stem", 3, 224, 224, 64, 7, 2, 3)]
    cin = 64
    hw = 56
    for stage, (width, blocks) in enumerate([(64, 3), (128, 4), (256, 6), (512, 3)], start=1):
        cout = width * 4
        for b in range(blocks):
            stride = 2 if (b == 0 and stage > 1) else 1
            o = hw // stride
            L.append((f"l{stage}.{b}.conv1", cin, hw, hw, width, 1, 1, 0))
            L.append((f"l{stage}.{b}.conv2", width, hw, hw, width, 3, stride, 1))
            L.append((f"l{stage}.{b}.conv3", width, o, o, cout, 1, 1, 0))
            if b == 0:
                L.append((f"l{stage}.{b}.ds", cin, hw, hw, cout, 1, stride, 0))
            cin = cout
            hw = o
    assert len(L) == 53
    return L


def out_hw(H, K, stride, pad):
    return (H + 2 * pad - K) // stride + 1


def conv_flops(shape, batch):
    _, cin, h, w, cout, k, s, p = shape
    ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
    return 2.0 * cout * batch * ho * wo * cin * k * k


def conv_bytes(shape, batch):
    """Compulsory HBM bytes: input + weight + output + 4 BN vectors (fp32)."""
    _, cin, h, w, cout, k, s, p = shape
    ho, wo = out_hw(h, k, s, p), out_hw(w, k, s, p)
    return 4.0 * (batch * cin * h * w + cout * cin * k * k + batch * cout * ho * wo) + 16.0 * cout
