"""ResNet-18 (torchvision layout, 224x224, 1000 classes) composed from the HAL
entries: the network the reference builds in src/engine/om.engine.resnet.ixx
(BasicBlock :55-79, ResNet18::forward :235-254), here with the torchvision
7x7 s2 stem + 3x3 s2 max pool.

GpuResNet18 runs it on libomhip:
  * forward()        — inference: every conv carries its BN (running stats) and
                       ReLU in the epilogue; the second conv of a block also adds
                       the shortcut (conv2dBiasBnAddAct);
  * forward_train()  — training forward: conv2d, batchNorm2d with batch
                       statistics, relu, add (BN cannot fold into the conv: its
                       statistics need the whole conv output);
  * backward(g)      — gradients of every conv weight, BN gamma/beta and the FC
                       layer for an upstream gradient g at the logits.
cpu_forward / cpu_forward_train / cpu_backward / cpu_train_step compose the
same network from the oracle (or the compiled reference CPUBackend): the
reference chain and the CPU baseline.
"""
from __future__ import annotations

import numpy as np

from omnimatchdeeplearningtool_amd import synthetic as S

STAGES = [("l1", 64, 64, 1), ("l2", 64, 128, 2), ("l3", 128, 256, 2), ("l4", 256, 512, 2)]
EPS = 1e-5
MOMENTUM = 0.1


def blocks():
    """(prefix, cin, cout, stride, has_downsample, input H) of the 8 BasicBlocks at 224x224."""
    hw = 56
    out = []
    for name, cin, cout, stride in STAGES:
        for b in range(2):
            ci = cin if b == 0 else cout
            s = stride if b == 0 else 1
            out.append((f"{name}.{b}", ci, cout, s, b == 0 and (s != 1 or ci != cout), hw))
            hw = (hw + 2 - 3) // s + 1
    return out


def make_params(seed: int = 0, num_classes: int = 1000) -> dict:
    """Kaiming-uniform conv / FC weights; BN gamma U[0.5,1.5], beta, mean N(0,0.1), var U[0.5,1.5]."""
    P = {}
    k = [seed * 1000]

    def nxt():
        k[0] += 1
        return k[0]

    def conv(name, cout, cin, ks):
        b = np.sqrt(6.0 / (cin * ks * ks))
        P[name + ".w"] = S.uniform((cout, cin, ks, ks), nxt(), -b, b)

    def bn(name, c):
        P[name + ".gamma"] = S.uniform((c,), nxt(), 0.5, 1.5)
        P[name + ".beta"] = S.randn((c,), nxt(), 0.1)
        P[name + ".mean"] = S.randn((c,), nxt(), 0.1)
        P[name + ".var"] = S.uniform((c,), nxt(), 0.5, 1.5)

    conv("stem", 64, 3, 7)
    bn("stem", 64)
    for pre, ci, co, s, ds, _ in blocks():
        conv(pre + ".conv1", co, ci, 3)
        bn(pre + ".conv1", co)
        conv(pre + ".conv2", co, co, 3)
        bn(pre + ".conv2", co)
        if ds:
            conv(pre + ".ds", co, ci, 1)
            bn(pre + ".ds", co)
    b = np.sqrt(6.0 / 512)
    P["fc.w"] = S.uniform((512, num_classes), nxt(), -b, b)     # Linear weight [in, out] (linear.ixx:50-58)
    P["fc.b"] = S.uniform((num_classes,), nxt(), -0.01, 0.01)
    return P


def conv_list():
    """(param name, Cin, H, Cout, K, stride, pad) of the 20 convs in network order."""
    L = [("stem", 3, 224, 64, 7, 2, 3)]
    for pre, ci, co, s, ds, hw in blocks():
        o = (hw + 2 - 3) // s + 1
        L.append((pre + ".conv1", ci, hw, co, 3, s, 1))
        L.append((pre + ".conv2", co, o, co, 3, 1, 1))
        if ds:
            L.append((pre + ".ds", ci, hw, co, 1, s, 0))
    return L


def pack_params(P: dict) -> np.ndarray:
    """The flat parameter array of omHipResNet18Create: per conv in network order its
    weight, BN gamma, beta, running mean and running var; then fc weight and bias."""
    parts = []
    for name, *_ in conv_list():
        parts += [P[name + ".w"].ravel(), P[name + ".gamma"], P[name + ".beta"], P[name + ".mean"],
                  P[name + ".var"]]
    parts += [P["fc.w"].ravel(), P["fc.b"]]
    return np.ascontiguousarray(np.concatenate(parts), np.float32)


def forward_flops(batch: int) -> float:
    """Conv + FC multiply-adds x 2 of one inference forward."""
    f = 0.0
    for _, ci, h, co, k, s, p in conv_list():
        o = (h + 2 * p - k) // s + 1
        f += 2.0 * batch * co * o * o * ci * k * k
    return f + 2.0 * batch * 512 * 1000


class GpuResNet18:
    def __init__(self, om, P: dict, batch: int, train: bool = False, fused: bool = True):
        self.om, self.H, self.B = om, om.HIPBackend, batch
        self.train = train
        self.fused = fused   # training step on the fused BN / ReLU / add entries
        self.d = {k: om.DeviceBuffer.from_numpy(np.ascontiguousarray(v)) for k, v in P.items()}
        self.nc = P["fc.w"].shape[1]
        self.buf = {}

    def _b(self, key, shape, dtype=np.float32):
        b = self.buf.get(key)
        if b is None:
            b = self.om.DeviceBuffer.empty(tuple(shape), dtype)
            self.buf[key] = b
        return b

    # ---------------------------------------------------------------- inference
    def _conv_fused(self, x, name, cin, h, cout, k, s, p, act, out_key, res=None):
        H, d, B = self.H, self.d, self.B
        o = (h + 2 * p - k) // s + 1
        y = self._b(out_key, (B, cout, o, o))
        args = (x, d[name + ".w"], None, d[name + ".gamma"], d[name + ".beta"], d[name + ".mean"], d[name + ".var"],
                EPS)
        if res is None:
            H.conv2dBiasBnAct(*args, act, y, B, cin, h, h, cout, k, k, s, p)
        else:
            H.conv2dBiasBnAddAct(*args, res, act, y, B, cin, h, h, cout, k, k, s, p)
        return y, o

    def forward(self, img):
        H, B = self.H, self.B
        a0, _ = self._conv_fused(img, "stem", 3, 224, 64, 7, 2, 3, 1, "stem.a")
        x = self._b("pool", (B, 64, 56, 56))
        H.maxPool2d(a0, x, None, B, 64, 112, 112, 3, 3, 2, 1)
        c = 64
        for pre, ci, co, s, ds, hw in blocks():
            a1, o = self._conv_fused(x, pre + ".conv1", ci, hw, co, 3, s, 1, 1, pre + ".a1")
            sc = self._conv_fused(x, pre + ".ds", ci, hw, co, 1, s, 0, 0, pre + ".sc")[0] if ds else x
            x, _ = self._conv_fused(a1, pre + ".conv2", co, o, co, 3, 1, 1, 1, pre + ".out", res=sc)
            c = co
        return self._head(x, c)

    def _head(self, x, c):
        H, B, d = self.H, self.B, self.d
        pooled = self._b("pooled", (B, c))
        H.adaptiveAvgPool2d(x, pooled, B, c, 7, 7, 1, 1)
        logits = self._b("logits", (B, self.nc))
        H.matmul(pooled, d["fc.w"], logits, B, c, self.nc)
        H.addBias(logits, d["fc.b"], logits, B, self.nc)
        return logits

    # ---------------------------------------------------------------- training
    def _conv_bn_train(self, x, name, cin, h, cout, k, s, p, key, out_key=None, act=0, res=None):
        """z = conv(x); y = BN_train(z) (saved stats); returns (y, o). With out_key the
        BN pass also adds res and applies the activation (the fused entry)."""
        H, d, B = self.H, self.d, self.B
        o = (h + 2 * p - k) // s + 1
        z = self._b(key + ".z", (B, cout, o, o))
        H.conv2d(x, d[name + ".w"], None, z, B, cin, h, h, cout, k, k, s, p)
        y = self._b(out_key or key + ".y", (B, cout, o, o))
        sm, si = self._b(key + ".sm", (cout,)), self._b(key + ".si", (cout,))
        if out_key is None:
            H.batchNorm2d(z, y, d[name + ".gamma"], d[name + ".beta"], d[name + ".mean"], d[name + ".var"], sm, si,
                          B, cout, o, o, EPS, MOMENTUM, True)
        else:
            H.batchNorm2dTrainAct(z, y, d[name + ".gamma"], d[name + ".beta"], d[name + ".mean"], d[name + ".var"],
                                  sm, si, B, cout, o, o, EPS, MOMENTUM, res, act)
        return y, o

    def _relu(self, x, key, n):
        a = self._b(key, (n,))
        self.H.relu(x, a, n)
        return a

    def forward_train(self, img):
        if self.fused:
            return self._forward_train_fused(img)
        H, B = self.H, self.B
        self.img = img
        y0, _ = self._conv_bn_train(img, "stem", 3, 224, 64, 7, 2, 3, "stem")
        a0 = self._relu(y0, "stem.a", B * 64 * 112 * 112)
        x = self._b("pool", (B, 64, 56, 56))
        idx = self._b("pool.idx", (B, 64, 56, 56), np.int32)
        H.maxPool2d(a0, x, idx, B, 64, 112, 112, 3, 3, 2, 1)
        self.block_in = []
        c = 64
        for pre, ci, co, s, ds, hw in blocks():
            self.block_in.append(x)
            y1, o = self._conv_bn_train(x, pre + ".conv1", ci, hw, co, 3, s, 1, pre + ".c1")
            a1 = self._relu(y1, pre + ".a1", B * co * o * o)
            y2, _ = self._conv_bn_train(a1, pre + ".conv2", co, o, co, 3, 1, 1, pre + ".c2")
            sc = self._conv_bn_train(x, pre + ".ds", ci, hw, co, 1, s, 0, pre + ".ds")[0] if ds else x
            ssum = self._b(pre + ".sum", (B, co, o, o))
            H.add(y2, sc, ssum, B * co * o * o)
            x = self._relu(ssum, pre + ".out", B * co * o * o)
            c = co
        self.last = x
        return self._head(x, c)

    def _forward_train_fused(self, img):
        """The training forward on the fused entries: BN statistics, residual add and
        ReLU in one pass per conv; the pre-activation tensors are never written."""
        H, B = self.H, self.B
        self.img = img
        a0, _ = self._conv_bn_train(img, "stem", 3, 224, 64, 7, 2, 3, "stem", out_key="stem.a", act=1)
        x = self._b("pool", (B, 64, 56, 56))
        idx = self._b("pool.idx", (B, 64, 56, 56), np.int32)
        H.maxPool2d(a0, x, idx, B, 64, 112, 112, 3, 3, 2, 1)
        self.block_in = []
        c = 64
        for pre, ci, co, s, ds, hw in blocks():
            self.block_in.append(x)
            a1, o = self._conv_bn_train(x, pre + ".conv1", ci, hw, co, 3, s, 1, pre + ".c1", out_key=pre + ".a1",
                                        act=1)
            sc = self._conv_bn_train(x, pre + ".ds", ci, hw, co, 1, s, 0, pre + ".ds")[0] if ds else x
            x, _ = self._conv_bn_train(a1, pre + ".conv2", co, o, co, 3, 1, 1, pre + ".c2", out_key=pre + ".out",
                                       act=1, res=sc)
            c = co
        self.last = x
        return self._head(x, c)

    def _bn_conv_backward(self, g_y, name, x_in, cin, h, cout, k, s, p, key, need_dx=True, mask=None):
        """Backward through y = BN(conv(x_in)): returns dx (or None); weight / BN grads stored.
        With mask the incoming gradient is first gated by mask > 0 (a ReLU's backward)."""
        H, d, B = self.H, self.d, self.B
        o = (h + 2 * p - k) // s + 1
        g_z = self._b(key + ".gz", (B, cout, o, o))
        if mask is None:
            H.batchNorm2dBackward(g_y, self.buf[key + ".z"], self.buf[key + ".sm"], self.buf[key + ".si"],
                                  d[name + ".gamma"], g_z, self._b(key + ".ggamma", (cout,)),
                                  self._b(key + ".gbeta", (cout,)), B, cout, o, o)
        else:
            H.batchNorm2dBackwardRelu(g_y, mask, self.buf[key + ".z"], self.buf[key + ".sm"], self.buf[key + ".si"],
                                      d[name + ".gamma"], g_z, self._b(key + ".ggamma", (cout,)),
                                      self._b(key + ".gbeta", (cout,)), B, cout, o, o)
        H.conv2dBackwardWeight(x_in, g_z, self._b(key + ".gw", (cout, cin, k, k)), None, B, cin, h, h, cout, k, k,
                               s, p)
        if not need_dx:
            return None
        g_x = self._b(key + ".gx", (B, cin, h, h))
        H.conv2dBackwardInput(g_z, d[name + ".w"], g_x, B, cin, h, h, cout, k, k, s, p)
        return g_x

    def backward(self, g_logits):
        H, B, d, nc = self.H, self.B, self.d, self.nc
        pooled = self.buf["pooled"]
        # FC: dW = pooled^T g, db = 1^T g, dpooled = g W^T
        H.matmulTransA(pooled, g_logits, self._b("fc.gw", (512, nc)), 512, B, nc)
        ones = self._b("ones", (1, B))
        H.fillValue(ones, B, 1.0)
        H.matmul(ones, g_logits, self._b("fc.gb", (1, nc)), 1, B, nc)
        g_p = self._b("g.pooled", (B, 512))
        H.matmulTransB(g_logits, d["fc.w"], g_p, B, nc, 512)
        g = self._b("g.last", (B, 512, 7, 7))
        H.adaptiveAvgPool2dBackward(g_p, g, B, 512, 7, 7, 1, 1)
        if self.fused:
            return self._backward_blocks_fused(g)
        bl = blocks()
        for bi in range(len(bl) - 1, -1, -1):
            pre, ci, co, s, ds, hw = bl[bi]
            o = (hw + 2 - 3) // s + 1
            n = B * co * o * o
            g_s = self._b(pre + ".gs", (B, co, o, o))
            H.reluBackward(self.buf[pre + ".sum"], g, g_s, n)
            g_a1 = self._bn_conv_backward(g_s, pre + ".conv2", self.buf[pre + ".a1"], co, o, co, 3, 1, 1, pre + ".c2")
            g_y1 = self._b(pre + ".gy1", (B, co, o, o))
            H.reluBackward(self.buf[pre + ".c1.y"], g_a1, g_y1, n)
            x_in = self.block_in[bi]
            g_x = self._bn_conv_backward(g_y1, pre + ".conv1", x_in, ci, hw, co, 3, s, 1, pre + ".c1")
            g_in = self._b(pre + ".gin", (B, ci, hw, hw))
            if ds:
                g_xd = self._bn_conv_backward(g_s, pre + ".ds", x_in, ci, hw, co, 1, s, 0, pre + ".ds")
                H.add(g_x, g_xd, g_in, B * ci * hw * hw)
            else:
                H.add(g_x, g_s, g_in, B * ci * hw * hw)
            g = g_in
        g_a0 = self._b("g.a0", (B, 64, 112, 112))
        H.maxPool2dBackwardEx(g, self.buf["pool.idx"], g_a0, B, 64, 112, 112, 3, 3, 2, 1)
        g_y0 = self._b("g.y0", (B, 64, 112, 112))
        H.reluBackward(self.buf["stem.y"], g_a0, g_y0, B * 64 * 112 * 112)
        self._bn_conv_backward(g_y0, "stem", self.img, 3, 224, 64, 7, 2, 3, "stem", need_dx=False)

    def _backward_blocks_fused(self, g):
        """Block backward on the fused entries. A ReLU's backward gates by its input > 0,
        which is its output > 0: the saved post-activation tensors serve as the masks."""
        H, B = self.H, self.B
        bl = blocks()
        for bi in range(len(bl) - 1, -1, -1):
            pre, ci, co, s, ds, hw = bl[bi]
            out = self.buf[pre + ".out"]
            g_a1 = self._bn_conv_backward(g, pre + ".conv2", self.buf[pre + ".a1"], co, (hw + 2 - 3) // s + 1, co,
                                          3, 1, 1, pre + ".c2", mask=out)
            x_in = self.block_in[bi]
            g_x = self._bn_conv_backward(g_a1, pre + ".conv1", x_in, ci, hw, co, 3, s, 1, pre + ".c1",
                                         mask=self.buf[pre + ".a1"])
            g_in = self._b(pre + ".gin", (B, ci, hw, hw))
            if ds:
                g_xd = self._bn_conv_backward(g, pre + ".ds", x_in, ci, hw, co, 1, s, 0, pre + ".ds", mask=out)
                H.add(g_x, g_xd, g_in, B * ci * hw * hw)
            else:
                H.addReluBackward(g_x, out, g, g_in, B * ci * hw * hw)
            g = g_in
        g_a0 = self._b("g.a0", (B, 64, 112, 112))
        H.maxPool2dBackwardEx(g, self.buf["pool.idx"], g_a0, B, 64, 112, 112, 3, 3, 2, 1)
        self._bn_conv_backward(g_a0, "stem", self.img, 3, 224, 64, 7, 2, 3, "stem", need_dx=False,
                               mask=self.buf["stem.a"])

    def forward_state(self, img: np.ndarray) -> dict:
        """Host copies of the training forward's intermediates (keys as cpu_forward_train)."""
        B = self.B
        f = {"img": img, "pool": self.buf["pool"].numpy(), "pool.idx": self.buf["pool.idx"].numpy(),
             "pooled": self.buf["pooled"].numpy()}
        fused = self.fused

        def conv_keys(key, shape, with_y):
            f[key + ".z"] = self.buf[key + ".z"].numpy().reshape(shape)
            if with_y:
                f[key + ".y"] = self.buf[key + ".y"].numpy().reshape(shape)
            f[key + ".sm"] = self.buf[key + ".sm"].numpy()
            f[key + ".si"] = self.buf[key + ".si"].numpy()
        conv_keys("stem", (B, 64, 112, 112), not fused)
        if fused:
            f["stem.a"] = self.buf["stem.a"].numpy().reshape(B, 64, 112, 112)
        for pre, ci, co, s, ds, hw in blocks():
            o = (hw + 2 - 3) // s + 1
            shp = (B, co, o, o)
            conv_keys(pre + ".c1", shp, not fused)
            conv_keys(pre + ".c2", shp, not fused)
            if ds:
                conv_keys(pre + ".ds", shp, True)
            for k in (".a1", ".out") if fused else (".a1", ".sum", ".out"):
                f[pre + k] = self.buf[pre + k].numpy().reshape(shp)
        return f

    def grads(self) -> dict:
        """Host copies of the weight gradients (conv name -> dW, plus fc.w / fc.b)."""
        out = {"fc.w": self.buf["fc.gw"].numpy(), "fc.b": self.buf["fc.gb"].numpy().reshape(-1)}
        for name, *_ in conv_list():
            key = name.replace(".conv1", ".c1").replace(".conv2", ".c2")
            out[name] = self.buf[key + ".gw"].numpy()
        return out


# ---------------------------------------------------------------- CPU chains
def cpu_forward(P: dict, img: np.ndarray, backend: str = "oracle") -> np.ndarray:
    """The reference's unfused inference chain: conv2d -> batchNorm2d(eval) -> relu,
    add, maxPool2d, adaptiveAvgPool2d, matmul + addBias."""
    import oracle as O
    def cbr(x, name, s, p, act=True):
        z = O.conv2d(x, P[name + ".w"], None, s, p, backend=backend)
        y, _, _ = O.batchnorm2d_eval(z, P[name + ".gamma"], P[name + ".beta"], P[name + ".mean"], P[name + ".var"],
                                     EPS, backend=backend)
        return O.relu(y, backend=backend) if act else y

    x = cbr(img, "stem", 2, 3)
    x, _ = O.maxpool2d(x, 3, 2, 1, backend=backend)
    for pre, ci, co, s, ds, hw in blocks():
        a1 = cbr(x, pre + ".conv1", s, 1)
        y2 = cbr(a1, pre + ".conv2", 1, 1, act=False)
        sc = cbr(x, pre + ".ds", s, 0, act=False) if ds else x
        x = O.relu(O.add(y2, sc, backend=backend), backend=backend)
    pooled = O.adaptive_avgpool2d(x, 1, 1, backend=backend).reshape(x.shape[0], -1)
    logits = O.matmul(pooled, P["fc.w"], backend=backend)
    return O.add_bias(logits, P["fc.b"], backend=backend)


def cpu_forward_train(P: dict, img: np.ndarray, backend: str = "oracle") -> dict:
    """Training forward with the reference's CPU functions. Returns every
    intermediate the backward needs (keys as GpuResNet18.forward_state)."""
    import oracle as O
    Pm = {k: v.copy() for k, v in P.items()}   # running stats are updated in place
    f = {"img": img}

    def conv_bn(x, name, s, p, key):
        z = O.conv2d(x, Pm[name + ".w"], None, s, p, backend=backend)
        y, rm, rv, sm, si = O.batchnorm2d_train(z, Pm[name + ".gamma"], Pm[name + ".beta"], Pm[name + ".mean"],
                                                Pm[name + ".var"], EPS, MOMENTUM, backend=backend)
        Pm[name + ".mean"], Pm[name + ".var"] = rm, rv
        f[key + ".z"], f[key + ".y"], f[key + ".sm"], f[key + ".si"] = z, y, sm, si
        return y

    y0 = conv_bn(img, "stem", 2, 3, "stem")
    f["stem.a"] = a0 = O.relu(y0, backend=backend)
    x, f["pool.idx"] = O.maxpool2d(a0, 3, 2, 1, backend=backend)
    f["pool"] = x
    for pre, ci, co, s, ds, hw in blocks():
        y1 = conv_bn(x, pre + ".conv1", s, 1, pre + ".c1")
        f[pre + ".a1"] = a1 = O.relu(y1, backend=backend)
        y2 = conv_bn(a1, pre + ".conv2", 1, 1, pre + ".c2")
        sc = conv_bn(x, pre + ".ds", s, 0, pre + ".ds") if ds else x
        f[pre + ".sum"] = ssum = O.add(y2, sc, backend=backend)
        f[pre + ".out"] = x = O.relu(ssum, backend=backend)
    f["pooled"] = O.adaptive_avgpool2d(x, 1, 1, backend=backend).reshape(x.shape[0], -1)
    return f


def cpu_forward_local(P: dict, f: dict, backend: str = "oracle") -> dict:
    """Each op of the training forward recomputed on the CPU from the GPU's own input to
    that op (f = GpuResNet18.forward_state of a fused step): conv2d, batchNorm2d (training
    statistics), relu, add, maxPool2d and adaptiveAvgPool2d, one layer at a time. Checks
    each kernel without the drift a deep chain accumulates from rounding differences."""
    import oracle as O
    out = {}

    def conv_bn(x, name, s, p, key):
        out[key + ".z"] = O.conv2d(x, P[name + ".w"], None, s, p, backend=backend)
        y, _, _, sm, si = O.batchnorm2d_train(f[key + ".z"], P[name + ".gamma"], P[name + ".beta"],
                                              P[name + ".mean"].copy(), P[name + ".var"].copy(), EPS, MOMENTUM,
                                              backend=backend)
        out[key + ".sm"], out[key + ".si"] = sm, si
        return y

    out["stem.a"] = O.relu(conv_bn(f["img"], "stem", 2, 3, "stem"), backend=backend)
    out["pool"], _ = O.maxpool2d(f["stem.a"], 3, 2, 1, backend=backend)
    x = f["pool"]
    for pre, ci, co, s, ds, hw in blocks():
        out[pre + ".a1"] = O.relu(conv_bn(x, pre + ".conv1", s, 1, pre + ".c1"), backend=backend)
        y2 = conv_bn(f[pre + ".a1"], pre + ".conv2", 1, 1, pre + ".c2")
        if ds:
            out[pre + ".ds.y"] = conv_bn(x, pre + ".ds", s, 0, pre + ".ds")
            sc = f[pre + ".ds.y"]
        else:
            sc = x
        out[pre + ".out"] = O.relu(O.add(y2, sc, backend=backend), backend=backend)
        x = f[pre + ".out"]
    out["pooled"] = O.adaptive_avgpool2d(x, 1, 1, backend=backend).reshape(x.shape[0], -1)
    return out


def _block_inputs(f: dict) -> list:
    ins, x = [], f["pool"]
    for pre, *_ in blocks():
        ins.append(x)
        x = f[pre + ".out"]
    return ins


def cpu_backward(P: dict, f: dict, g_logits: np.ndarray, backend: str = "oracle") -> dict:
    """Backward of the training step from the forward state f (from
    cpu_forward_train, or GpuResNet18.forward_state to replay the GPU's own
    forward decisions); returns the weight gradients (as GpuResNet18.grads)."""
    import oracle as O
    B = g_logits.shape[0]
    pooled = np.ascontiguousarray(f["pooled"].reshape(B, -1))
    grads = {"fc.w": O.matmul(np.ascontiguousarray(pooled.T), g_logits, backend=backend),
             "fc.b": O.matmul(np.ones((1, B), np.float32), g_logits, backend=backend).reshape(-1)}
    g_p = O.matmul(g_logits, np.ascontiguousarray(P["fc.w"].T), backend=backend)
    g = O.adaptive_avgpool2d_backward(g_p.reshape(B, 512, 1, 1), 7, 7, backend=backend)
    ins = _block_inputs(f)

    def bn_conv_bwd(g_y, name, key, x_in, s, p, need_dx=True):
        g_z, _, _ = O.batchnorm2d_backward(g_y, f[key + ".z"], f[key + ".sm"], f[key + ".si"], P[name + ".gamma"],
                                           backend=backend)
        w = P[name + ".w"]
        grads[name], _ = O.conv2d_backward_weight(x_in, g_z, w.shape[2], w.shape[3], s, p, bias=False,
                                                  backend=backend)
        if need_dx:
            return O.conv2d_backward_input(g_z, w, x_in.shape[2], x_in.shape[3], s, p, backend=backend)
        return None

    def relu_in(pre_key, post_key):
        # reluBackward gates by input > 0, i.e. output > 0: either tensor serves
        return f[pre_key] if pre_key in f else f[post_key]

    bl = blocks()
    for bi in range(len(bl) - 1, -1, -1):
        pre, ci, co, s, ds, hw = bl[bi]
        g_s = O.relu_backward(relu_in(pre + ".sum", pre + ".out"), g, backend=backend)
        g_a1 = bn_conv_bwd(g_s, pre + ".conv2", pre + ".c2", f[pre + ".a1"], 1, 1)
        g_y1 = O.relu_backward(relu_in(pre + ".c1.y", pre + ".a1"), g_a1, backend=backend)
        g_x = bn_conv_bwd(g_y1, pre + ".conv1", pre + ".c1", ins[bi], s, 1)
        g = O.add(g_x, bn_conv_bwd(g_s, pre + ".ds", pre + ".ds", ins[bi], s, 0) if ds else g_s, backend=backend)
    g_a0 = O.maxpool2d_backward(g, f["pool.idx"], 112, 112, backend=backend)
    g_y0 = O.relu_backward(relu_in("stem.y", "stem.a"), g_a0, backend=backend)
    bn_conv_bwd(g_y0, "stem", "stem", f["img"], 2, 3, need_dx=False)
    return grads


def cpu_train_step(P: dict, img: np.ndarray, g_logits: np.ndarray, backend: str = "oracle") -> dict:
    """Training forward (batch statistics) and backward with the reference's CPU functions."""
    return cpu_backward(P, cpu_forward_train(P, img, backend), g_logits, backend)
