"""The reference's own networks, in the reference's op order, on the HAL entries.

ResNet18 (resnet.ixx:186-254): a 3x3 stride-1 stem conv -> BN -> ReLU, the 3x3
stride-2 max pool only when the input is taller than 32 (:240-242), four stages
of two BasicBlocks (64, 128, 256, 512 channels; strides 1, 2, 2, 2), global
average pool, Linear(512, classes). BasicBlock (:55-79): conv1 -> bn1 -> relu ->
conv2 -> bn2 -> + shortcut (1x1 stride-s conv + BN when the shape changes, else
the input) -> relu.

ResNet50 (resnet50.ixx:202-279): a 3x3 stride-1 stem conv -> BN -> ReLU, no max
pool, stages of 3, 4, 6, 3 Bottlenecks (widths 64, 128, 256, 512, expansion 4;
stride 2 on the first block of stages 2-4), global average pool, Linear(2048,
classes). Bottleneck (:57-83): 1x1 conv1 -> bn1 -> relu -> 3x3 conv2 (stride) ->
bn2 -> relu -> 1x1 conv3 -> bn3 -> + shortcut -> relu.

BatchNorm runs in inference mode (running statistics), as Module::eval() sets
for EngineBridge::infer. On the GPU every conv carries its BN and ReLU in the
epilogue (omHipConv2dBiasBnAct) and the block's last conv also the shortcut
sum (omHipConv2dBiasBnAddAct); the CPU twin runs the reference's unfused chain
conv2d -> batchNorm2d(eval) -> relu / add through the oracle.
"""
from __future__ import annotations

import numpy as np

import oracle as O

EPS = 1e-5


def _kaiming(shape, seed):
    fan_in = int(np.prod(shape[1:]))
    b = np.sqrt(6.0 / fan_in)
    return O.uniform(shape, seed, -b, b)


def _bn(P, name, c, seed):
    P[name + ".gamma"] = O.uniform((c,), seed, 0.5, 1.5)
    P[name + ".beta"] = O.randn((c,), seed + 1, 0.1)
    P[name + ".mean"] = O.randn((c,), seed + 2, 0.1)
    P[name + ".var"] = O.uniform((c,), seed + 3, 0.5, 1.5)


def resnet18_blocks():
    """(prefix, cin, cout, stride, has_downsample) of the 8 BasicBlocks (resnet.ixx:213-229)."""
    out = []
    for li, (cin, cout, s) in enumerate([(64, 64, 1), (64, 128, 2), (128, 256, 2), (256, 512, 2)], start=1):
        for i in range(2):
            ci, si = (cin, s) if i == 0 else (cout, 1)
            out.append((f"layer{li}.{i}", ci, cout, si, si != 1 or ci != cout))
    return out


def resnet50_blocks():
    """(prefix, cin, width, stride, has_downsample) of the 16 Bottlenecks (resnet50.ixx:211-241)."""
    out = []
    cin = 64
    for li, (width, n, s) in enumerate([(64, 3, 1), (128, 4, 2), (256, 6, 2), (512, 3, 2)], start=1):
        for i in range(n):
            si = s if i == 0 else 1
            out.append((f"layer{li}.{i}", cin, width, si, si != 1 or cin != 4 * width))
            cin = 4 * width
    return out


def make_resnet18(in_ch: int, classes: int, seed: int) -> dict:
    P = {"conv1.w": _kaiming((64, in_ch, 3, 3), seed)}
    _bn(P, "bn1", 64, seed + 1)
    for k, (pre, ci, co, s, ds) in enumerate(resnet18_blocks()):
        sd = seed + 100 * (k + 1)
        P[pre + ".conv1.w"] = _kaiming((co, ci, 3, 3), sd)
        _bn(P, pre + ".bn1", co, sd + 10)
        P[pre + ".conv2.w"] = _kaiming((co, co, 3, 3), sd + 20)
        _bn(P, pre + ".bn2", co, sd + 30)
        if ds:
            P[pre + ".ds.w"] = _kaiming((co, ci, 1, 1), sd + 40)
            _bn(P, pre + ".dsbn", co, sd + 50)
    P["fc.w"] = O.randn((512, classes), seed + 7, np.sqrt(2.0 / 512))
    P["fc.b"] = O.randn((classes,), seed + 8, 0.1)
    return P


def make_resnet50(in_ch: int, classes: int, seed: int) -> dict:
    P = {"conv1.w": _kaiming((64, in_ch, 3, 3), seed)}
    _bn(P, "bn1", 64, seed + 1)
    for k, (pre, ci, wd, s, ds) in enumerate(resnet50_blocks()):
        sd = seed + 100 * (k + 1)
        P[pre + ".conv1.w"] = _kaiming((wd, ci, 1, 1), sd)
        _bn(P, pre + ".bn1", wd, sd + 10)
        P[pre + ".conv2.w"] = _kaiming((wd, wd, 3, 3), sd + 20)
        _bn(P, pre + ".bn2", wd, sd + 30)
        P[pre + ".conv3.w"] = _kaiming((4 * wd, wd, 1, 1), sd + 40)
        _bn(P, pre + ".bn3", 4 * wd, sd + 50)
        if ds:
            P[pre + ".ds.w"] = _kaiming((4 * wd, ci, 1, 1), sd + 60)
            _bn(P, pre + ".dsbn", 4 * wd, sd + 70)
    P["fc.w"] = O.randn((2048, classes), seed + 7, np.sqrt(2.0 / 2048))
    P["fc.b"] = O.randn((classes,), seed + 8, 0.1)
    return P


def _ohw(h, k, s, p):
    return (h + 2 * p - k) // s + 1


# ------------------------------------------------------------------ GPU (HAL)
class GpuNet:
    """Runs a reference-layout network on the HAL entries with device-resident parameters."""

    def __init__(self, om, P: dict):
        self.om, self.H = om, om.HIPBackend
        self.d = {k: om.DeviceBuffer.from_numpy(np.ascontiguousarray(v)) for k, v in P.items()}
        self.keep = []

    def conv(self, x, N, cin, h, w, wname, bname, cout, k, s, p, act, res=None):
        """conv (no bias) -> BN(eval) [-> + res] [-> ReLU] in one launch; returns (y, ho, wo)."""
        ho, wo = _ohw(h, k, s, p), _ohw(w, k, s, p)
        y = self.om.DeviceBuffer.empty((N, cout, ho, wo))
        self.keep.append(y)
        d = self.d
        bn = (d[bname + ".gamma"], d[bname + ".beta"], d[bname + ".mean"], d[bname + ".var"])
        if res is None:
            self.H.conv2dBiasBnAct(x, d[wname], None, *bn, EPS, act, y, N, cin, h, w, cout, k, k, s, p)
        else:
            self.H.conv2dBiasBnAddAct(x, d[wname], None, *bn, EPS, res, act, y, N, cin, h, w, cout, k, k, s, p)
        return y, ho, wo

    def head(self, x, N, c, h, w, classes):
        pooled = self.om.DeviceBuffer.empty((N, c))
        logits = self.om.DeviceBuffer.empty((N, classes))
        self.keep += [pooled, logits]
        self.H.adaptiveAvgPool2d(x, pooled, N, c, h, w, 1, 1)
        self.H.linearBiasAct(pooled, self.d["fc.w"], self.d["fc.b"], logits, N, c, classes, 0)
        return logits

    def basic_block(self, x, N, h, w, pre, ci, co, s, ds):
        a1, ho, wo = self.conv(x, N, ci, h, w, pre + ".conv1.w", pre + ".bn1", co, 3, s, 1, 1)
        sc = self.conv(x, N, ci, h, w, pre + ".ds.w", pre + ".dsbn", co, 1, s, 0, 0)[0] if ds else x
        y, _, _ = self.conv(a1, N, co, ho, wo, pre + ".conv2.w", pre + ".bn2", co, 3, 1, 1, 1, res=sc)
        return y, ho, wo

    def bottleneck(self, x, N, h, w, pre, ci, wd, s, ds):
        a1, _, _ = self.conv(x, N, ci, h, w, pre + ".conv1.w", pre + ".bn1", wd, 1, 1, 0, 1)
        a2, ho, wo = self.conv(a1, N, wd, h, w, pre + ".conv2.w", pre + ".bn2", wd, 3, s, 1, 1)
        sc = self.conv(x, N, ci, h, w, pre + ".ds.w", pre + ".dsbn", 4 * wd, 1, s, 0, 0)[0] if ds else x
        y, _, _ = self.conv(a2, N, wd, ho, wo, pre + ".conv3.w", pre + ".bn3", 4 * wd, 1, 1, 0, 1, res=sc)
        return y, ho, wo

    def resnet18(self, img, N, cin, h, w, classes):
        x, h2, w2 = self.conv(img, N, cin, h, w, "conv1.w", "bn1", 64, 3, 1, 1, 1)
        if h > 32:
            hp, wp = _ohw(h2, 3, 2, 1), _ohw(w2, 3, 2, 1)
            pooled = self.om.DeviceBuffer.empty((N, 64, hp, wp))
            self.keep.append(pooled)
            self.H.maxPool2d(x, pooled, None, N, 64, h2, w2, 3, 3, 2, 1)
            x, h2, w2 = pooled, hp, wp
        for pre, ci, co, s, ds in resnet18_blocks():
            x, h2, w2 = self.basic_block(x, N, h2, w2, pre, ci, co, s, ds)
        return self.head(x, N, 512, h2, w2, classes)

    def resnet50(self, img, N, cin, h, w, classes):
        x, h2, w2 = self.conv(img, N, cin, h, w, "conv1.w", "bn1", 64, 3, 1, 1, 1)
        for pre, ci, wd, s, ds in resnet50_blocks():
            x, h2, w2 = self.bottleneck(x, N, h2, w2, pre, ci, wd, s, ds)
        return self.head(x, N, 2048, h2, w2, classes)


# ------------------------------------------------------------ CPU (oracle)
def _cbr(P, x, wname, bname, s, p, act):
    z = O.conv2d(x, P[wname], None, s, p)
    y, _, _ = O.batchnorm2d_eval(z, P[bname + ".gamma"], P[bname + ".beta"], P[bname + ".mean"],
                                 P[bname + ".var"], EPS)
    return O.relu(y) if act else y


def cpu_basic_block(P, x, pre, s, ds):
    a1 = _cbr(P, x, pre + ".conv1.w", pre + ".bn1", s, 1, True)
    y2 = _cbr(P, a1, pre + ".conv2.w", pre + ".bn2", 1, 1, False)
    sc = _cbr(P, x, pre + ".ds.w", pre + ".dsbn", s, 0, False) if ds else x
    return O.relu(O.add(y2, sc))


def cpu_bottleneck(P, x, pre, s, ds):
    a1 = _cbr(P, x, pre + ".conv1.w", pre + ".bn1", 1, 0, True)
    a2 = _cbr(P, a1, pre + ".conv2.w", pre + ".bn2", s, 1, True)
    y3 = _cbr(P, a2, pre + ".conv3.w", pre + ".bn3", 1, 0, False)
    sc = _cbr(P, x, pre + ".ds.w", pre + ".dsbn", s, 0, False) if ds else x
    return O.relu(O.add(y3, sc))


def _cpu_head(P, x):
    pooled = O.adaptive_avgpool2d(x, 1, 1).reshape(x.shape[0], -1)
    return O.add_bias(O.matmul(pooled, P["fc.w"]), P["fc.b"])


def cpu_resnet18(P, img):
    x = _cbr(P, img, "conv1.w", "bn1", 1, 1, True)
    if img.shape[2] > 32:
        x, _ = O.maxpool2d(x, 3, 2, 1)
    for pre, _, _, s, ds in resnet18_blocks():
        x = cpu_basic_block(P, x, pre, s, ds)
    return _cpu_head(P, x)


def cpu_resnet50(P, img):
    x = _cbr(P, img, "conv1.w", "bn1", 1, 1, True)
    for pre, _, _, s, ds in resnet50_blocks():
        x = cpu_bottleneck(P, x, pre, s, ds)
    return _cpu_head(P, x)
