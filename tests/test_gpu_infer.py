"""Device-resident plumbing and batch inference (the EngineBridge::inferBatch
path, EngineBridge.cpp:3525-3772): page-locked host memory, the transfer
stream and its ordering events, graph capture / replay, and the ResNet-18
classification pipeline.

Bars: copies, fills and replays are exact. The pipeline's probabilities are
held to 2e-6 (relative) against the softmax of the GPU network's own logits
(float32 in numpy, sequential sum as the reference loop; the host exp may
differ from numpy's by an ulp), its logits to the 1e-4 network bar against the
CPU chain; classes must agree wherever the top two probabilities differ by
more than that tolerance.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev
from resnet_net import GpuResNet18, cpu_forward, make_params, pack_params

pytestmark = pytest.mark.gpu

IMNET_MEAN = np.array([0.485, 0.456, 0.406], np.float32)
IMNET_INV = (np.float32(1.0) / np.array([0.229, 0.224, 0.225], np.float32)).astype(np.float32)


def test_pinned_async_roundtrip(hip):
    om = hip
    n = (1 << 20) + 3
    src = O.randn((n,), 5)
    ctypes = __import__("ctypes")
    hp = ctypes.c_void_p()
    om.call("omHipMallocHost", ctypes.byref(hp), n * 4)
    try:
        pinned = np.ctypeslib.as_array((ctypes.c_float * n).from_address(hp.value))
        pinned[:] = src
        d = empty_dev(om, (n,))
        out = empty_dev(om, (n,))
        om.call("omHipAsyncCopyH2D", d.ptr, hp.value, n * 4)
        om.call("omHipComputeWaitTransfer")            # the ReLU runs after the upload
        om.HIPBackend.relu(d, out, n)
        om.call("omHipTransferWaitCompute")            # the download runs after the ReLU
        om.call("omHipAsyncCopyD2H", hp.value, out.ptr, n * 4)
        om.call("omHipSyncTransferStream")
        assert np.array_equal(pinned.view(np.uint32), O.relu(src).view(np.uint32))
    finally:
        om.call("omHipFreeHost", hp.value)


@pytest.mark.parametrize("off,n", [(0, 1), (3, 5), (1, 4096 + 7), (0, (1 << 20) + 13)])
def test_memset_bytes(hip, off, n):
    buf = empty_dev(hip, ((n + off + 64) // 4 + 1,))
    hip.HIPBackend.fillValue(buf, buf.shape[0], -1.0)   # 0xbf800000 everywhere
    hip.call("omHipMemset", buf.ptr + off, 0x5a, n)
    got = buf.numpy().view(np.uint8)
    ref = np.frombuffer(np.full(buf.shape[0], -1.0, np.float32).tobytes(), np.uint8).copy()
    ref[off:off + n] = 0x5a
    assert np.array_equal(got, ref)


def test_graph_replay(hip):
    """Capture conv+BN+ReLU (remainder work split and split-K layers), a residual conv and a
    memset; replay three times with new inputs and eager work in between; every replay must
    equal the eager result bit for bit."""
    H = hip.HIPBackend
    N, C, Hh = 12, 64, 56
    w = O.uniform((C, C, 3, 3), 1, -0.06, 0.06)
    w4 = O.uniform((512, 256, 3, 3), 2, -0.02, 0.02)
    bn = [O.uniform((C,), 3, 0.5, 1.5), O.randn((C,), 4, 0.1), O.randn((C,), 5, 0.1), O.uniform((C,), 6, 0.5, 1.5)]
    bn4 = [O.uniform((512,), 7, 0.5, 1.5), O.randn((512,), 8, 0.1), O.randn((512,), 9, 0.1),
           O.uniform((512,), 10, 0.5, 1.5)]
    dw, dw4 = to_dev(hip, w), to_dev(hip, w4)
    dbn, dbn4 = [to_dev(hip, a) for a in bn], [to_dev(hip, a) for a in bn4]
    x = empty_dev(hip, (N, C, Hh, Hh))
    x4 = empty_dev(hip, (2, 256, 14, 14))
    y = empty_dev(hip, (N, C, Hh, Hh))
    z = empty_dev(hip, (N, C, Hh, Hh))
    y4 = empty_dev(hip, (2, 512, 7, 7))
    pad = empty_dev(hip, (1000,))

    def seq():
        H.conv2dBiasBnAct(x, dw, None, *dbn, 1e-5, 1, y, N, C, Hh, Hh, C, 3, 3, 1, 1)
        H.conv2dBiasBnAddAct(y, dw, None, *dbn, 1e-5, x, 1, z, N, C, Hh, Hh, C, 3, 3, 1, 1)
        H.conv2dBiasBnAct(x4, dw4, None, *dbn4, 1e-5, 1, y4, 2, 256, 14, 14, 512, 3, 3, 2, 1)
        hip.call("omHipMemset", pad.ptr, 0, 4000)

    def eager(seed):
        x.upload(O.randn((N, C, Hh, Hh), seed))
        x4.upload(O.randn((2, 256, 14, 14), seed + 1))
        seq()
        return z.numpy().copy(), y4.numpy().copy()

    ref0 = eager(100)                       # warm-up: tables, workspaces, pool blocks exist
    graph = hip.Graph(seq)
    for r in range(3):
        e_z, e_y4 = eager(200 + r)          # eager result on this replay's inputs
        pad.upload(np.ones(1000, np.float32))
        x.upload(O.randn((N, C, Hh, Hh), 200 + r))
        x4.upload(O.randn((2, 256, 14, 14), 201 + r))
        H.fillValue(z, N * C * Hh * Hh, 7.0)   # the replay must overwrite
        graph.launch()
        hip.synchronize()
        assert np.array_equal(z.numpy().view(np.uint32), e_z.view(np.uint32)), r
        assert np.array_equal(y4.numpy().view(np.uint32), e_y4.view(np.uint32)), r
        assert not np.any(pad.numpy()), r
    assert not np.array_equal(ref0[0], e_z)


def _softmax_ref(logits):
    """EngineBridge.cpp:3740-3756 in float32: exp(l - max), sequential sum, / max(sum, 1e-8)."""
    l = logits.astype(np.float32)
    e = np.exp(l - l.max(axis=1, keepdims=True)).astype(np.float32)
    s = np.cumsum(e, axis=1, dtype=np.float32)[:, -1:]
    return (e / np.maximum(s, np.float32(1e-8))).astype(np.float32)


@pytest.fixture(scope="module")
def net_params():
    return make_params(seed=3)


def test_resnet18_infer_batch(hip, net_params):
    P = net_params
    net = hip.ResNet18Infer(pack_params(P), 1000, 32)
    n_img = 37
    imgs = O.uniform((n_img, 3, 224, 224), 77, 0.0, 1.0)
    normed = ((imgs - IMNET_MEAN[None, :, None, None]) * IMNET_INV[None, :, None, None]).astype(np.float32)
    # logits of the resident forward on host-normalised images = the HAL-composed network
    gnet = GpuResNet18(hip, P, 5)
    d_in = to_dev(hip, normed[:5])
    d_log = empty_dev(hip, (5, 1000))
    net.forward(d_in, d_log, 5)
    ref_log = gnet.forward(d_in).numpy().reshape(5, 1000)
    assert np.array_equal(d_log.numpy().view(np.uint32), ref_log.view(np.uint32))
    # pipeline: 16-image batches (3 batches, the last ragged), ImageNet normalisation on device
    cls, conf, probs = net.infer_batch(imgs, batch_size=16)
    logits = np.concatenate([_forward_logits(hip, net, normed[i:i + 16]) for i in range(0, n_img, 16)])
    pref = _softmax_ref(logits)
    assert np.max(np.abs(probs - pref) / np.maximum(pref, 1e-30)) <= 2e-6
    assert np.array_equal(conf, probs.max(axis=1))
    top2 = np.sort(pref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 4e-6 * top2[:, 1]
    assert np.array_equal(cls[clear], pref.argmax(axis=1)[clear])
    # against the reference CPU chain (two images)
    cpu = cpu_forward(P, normed[:2])
    assert O.frobenius_rel(logits[:2], cpu) <= 1e-4
    # other batch sizes give the same answers: the work split (and so the summation order)
    # depends on the batch, so logits move within the network bar and probabilities by
    # about |logit change| in absolute terms
    for bs in (32, 5, 1):
        c2, f2, p2 = net.infer_batch(imgs, batch_size=bs)
        lb = np.concatenate([_forward_logits(hip, net, normed[i:i + bs]) for i in range(0, n_img, bs)])
        assert O.frobenius_rel(lb, logits) <= 1e-5, bs
        assert np.max(np.abs(p2 - _softmax_ref(lb))) <= 1e-6, bs
        assert np.max(np.abs(p2 - probs)) <= 1e-3, bs
        assert np.array_equal(c2[clear], cls[clear]), bs
    # confidence threshold: below it the class is -1 (EngineBridge.cpp:3760-3762)
    thr = float(np.median(conf))
    c3, f3, _ = net.infer_batch(imgs, batch_size=16, conf_threshold=thr, with_probs=False)
    assert np.array_equal(f3, conf)
    assert np.array_equal(c3 == -1, conf < np.float32(thr))


def _forward_logits(hip, net, normed):
    b = normed.shape[0]
    d_in, d_log = to_dev(hip, normed), empty_dev(hip, (b, 1000))
    net.forward(d_in, d_log, b)
    return d_log.numpy().reshape(b, 1000)


def test_resnet18_infer_rejects_bad_input(hip, net_params):
    net = hip.ResNet18Infer(pack_params(net_params), 1000, 4)
    with pytest.raises(hip.OmHipError, match="3x224x224"):
        net.infer_batch(np.zeros((1, 3, 112, 112), np.float32))
    with pytest.raises(hip.OmHipError, match="parameter floats"):
        hip.ResNet18Infer(pack_params(net_params)[:-1], 1000, 4)
