"""conv2d parity: implicit-GEMM MFMA conv (+ fused bias/BN/ReLU) against the
oracle's reference chain conv2d -> batchNorm2d(eval) -> relu.

Tolerance (K-scaled): |out_hip - out_ref| <= 1e-4 * budget, where budget is
the float64 conv of |x| and |w| (plus |bias|), scaled by |gamma| * invStd after
BN — the conv analogue of sum_k |a_ik||b_kj|. Every ResNet-18 conv shape (the
benchmark's 20 layers) runs at batch 2 against the oracle and at batch 32 on
images {0, 1, 30, 31} (tiles straddle image boundaries differently there);
every distinct ResNet-50 geometry runs at batch 2, the benchmark's batch-64
plans on sampled images; odd geometries and the explicit im2col path follow.
"""
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev
from resnet_shapes import out_hw, resnet18_convs, resnet50_convs

pytestmark = pytest.mark.gpu
TOL = O.TOL_FP32


def _params(cout, seed):
    gamma = O.uniform((cout,), seed + 1, 0.5, 1.5)
    beta = O.randn((cout,), seed + 2, 0.1)
    mean = O.randn((cout,), seed + 3, 0.1)
    var = O.uniform((cout,), seed + 4, 0.5, 1.5)
    return gamma, beta, mean, var


def _kaiming_uniform(shape, seed):
    fan_in = int(np.prod(shape[1:]))
    bound = np.sqrt(6.0 / fan_in)
    return O.uniform(shape, seed, -bound, bound)


def _run_conv(hip, x, w, bias, bn, act, stride, pad, entry="omHipConv2dBiasBnAct"):
    N, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    Ho, Wo = out_hw(H, KH, stride, pad), out_hw(W, KW, stride, pad)
    dx, dw = to_dev(hip, x), to_dev(hip, w)
    db = to_dev(hip, bias) if bias is not None else None
    dout = empty_dev(hip, (N, Cout, Ho, Wo))
    if entry == "omHipConv2dBiasBnAct":
        dbn = [to_dev(hip, a) for a in bn] if bn is not None else [None] * 4
        hip.call(entry, dx.ptr, dw.ptr, db.ptr if db else None, *[d.ptr if d else None for d in dbn],
                 1e-5, act, dout.ptr, N, Cin, H, W, Cout, KH, KW, stride, pad)
    else:
        hip.call(entry, dx.ptr, dw.ptr, db.ptr if db else None, dout.ptr, N, Cin, H, W, Cout, KH, KW, stride, pad)
    return dout.numpy()


def _check(out, x, w, bias, bn, act, stride, pad):
    ref = O.conv_bn_act(x, w, bias, *(bn if bn is not None else (None,) * 4), eps=1e-5, act=act,
                        stride=stride, pad=pad)
    kw = dict(zip(("gamma", "beta", "mean", "var"), bn)) if bn is not None else {}
    o64, bound = O.conv_f64(x, w, bias, stride, pad, act=act, **kw)
    e_ref = O.normalized_error(out, ref, bound)
    e_64 = O.normalized_error(out, o64, bound)
    assert e_ref <= TOL, f"vs oracle {e_ref:.3e}"
    assert e_64 <= TOL, f"vs float64 {e_64:.3e}"
    return e_ref


R18 = resnet18_convs()


@pytest.mark.parametrize("shape", R18, ids=[s[0] for s in R18])
def test_resnet18_layer_fused_b2(hip, shape):
    name, cin, h, w, cout, k, s, p = shape
    seed = zlib.crc32(name.encode()) % 10000
    x = O.randn((2, cin, h, w), seed)
    wt = _kaiming_uniform((cout, cin, k, k), seed + 10)
    bn = _params(cout, seed + 20)
    print(f"case r18 {name} b2", flush=True)
    out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    _check(out, x, wt, None, bn, 1, s, p)


@pytest.mark.parametrize("shape", R18, ids=[s[0] for s in R18])
def test_resnet18_layer_fused_b32_sampled(hip, shape):
    name, cin, h, w, cout, k, s, p = shape
    seed = zlib.crc32(name.encode()) % 10000 + 7
    x = O.randn((32, cin, h, w), seed)
    wt = _kaiming_uniform((cout, cin, k, k), seed + 10)
    bn = _params(cout, seed + 20)
    print(f"case r18 {name} b32", flush=True)
    out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    idx = [0, 1, 30, 31]
    _check(out[idx], np.ascontiguousarray(x[idx]), wt, None, bn, 1, s, p)


# Tile counts of 2-12 per CU that are not a multiple of the CU count: the tiles
# past the last whole round run as K pieces summed by a second kernel (tile
# edges exact, and ragged in Cout and pixels).
BALANCE = [(12, 64, 56, 56, 64, 3, 1, 1), (9, 16, 45, 45, 100, 3, 1, 1)]


@pytest.mark.parametrize("geom", BALANCE, ids=lambda g: "N{}C{}H{}W{}o{}k{}s{}p{}".format(*g))
@pytest.mark.parametrize("variant", ["bias", "bn_relu"])
def test_balanced_work_split(hip, geom, variant):
    N, cin, h, w, cout, k, s, p = geom
    x = O.randn((N, cin, h, w), 900 + cout)
    wt = _kaiming_uniform((cout, cin, k, k), 901)
    bias = O.randn((cout,), 902) if variant == "bias" else None
    bn = _params(cout, 903) if variant == "bn_relu" else None
    print(f"case balance {geom} {variant}", flush=True)
    if variant == "bias":
        out = _run_conv(hip, x, wt, bias, None, 0, s, p, entry="omHipConv2d")
    else:
        out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    _check(out, x, wt, bias, bn, 1 if bn is not None else 0, s, p)


# Few tiles and a long K: the K range is split, the partial sums are added by
# a second kernel four pixels at a time (Nq = 49 and 75 leave ragged quads;
# 392 takes the aligned 16-byte path).
SPLITK = [(1, 256, 7, 7, 100, 3, 1, 1), (3, 128, 9, 9, 70, 3, 2, 1), (2, 256, 14, 14, 64, 3, 1, 1)]


@pytest.mark.parametrize("geom", SPLITK, ids=lambda g: "N{}C{}H{}W{}o{}k{}s{}p{}".format(*g))
@pytest.mark.parametrize("variant", ["bias", "bn_relu"])
def test_split_k_finish(hip, geom, variant):
    N, cin, h, w, cout, k, s, p = geom
    x = O.randn((N, cin, h, w), 700 + cout)
    wt = _kaiming_uniform((cout, cin, k, k), 701)
    bias = O.randn((cout,), 702) if variant == "bias" else None
    bn = _params(cout, 703) if variant == "bn_relu" else None
    print(f"case splitk {geom} {variant}", flush=True)
    if variant == "bias":
        out = _run_conv(hip, x, wt, bias, None, 0, s, p, entry="omHipConv2d")
    else:
        out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    _check(out, x, wt, bias, bn, 1 if bn is not None else 0, s, p)


def _distinct(convs):
    """First layer of each distinct geometry (Cin, H, W, Cout, K, stride, pad)."""
    seen, out = set(), []
    for c in convs:
        if c[1:] not in seen:
            seen.add(c[1:])
            out.append(c)
    return out


R50 = _distinct(resnet50_convs())     # 23 geometries cover all 53 ResNet-50 convs


@pytest.mark.parametrize("shape", R50, ids=[s[0] for s in R50])
def test_resnet50_layer_fused_b2(hip, shape):
    name, cin, h, w, cout, k, s, p = shape
    seed = zlib.crc32(("r50" + name).encode()) % 10000
    x = O.randn((2, cin, h, w), seed)
    wt = _kaiming_uniform((cout, cin, k, k), seed + 10)
    bn = _params(cout, seed + 20)
    print(f"case r50 {name} b2", flush=True)
    out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    _check(out, x, wt, None, bn, 1, s, p)


R50_B64 = [c for c in resnet50_convs() if c[0] in ("stem", "l1.1.conv1", "l2.1.conv2", "l3.1.conv1", "l4.1.conv1",
                                                     "l4.0.ds", "l3.0.conv2", "l4.1.conv3")]


@pytest.mark.parametrize("shape", R50_B64, ids=[s[0] for s in R50_B64])
def test_resnet50_layer_fused_b64_sampled(hip, shape):
    """The benchmark's batch-64 launch plan (tile counts, split-K factors, remainder pieces and
    batch chunks) on images {0, 1, 33, 62, 63}."""
    name, cin, h, w, cout, k, s, p = shape
    seed = zlib.crc32(("r50b64" + name).encode()) % 10000
    x = O.randn((64, cin, h, w), seed)
    wt = _kaiming_uniform((cout, cin, k, k), seed + 10)
    bn = _params(cout, seed + 20)
    print(f"case r50 {name} b64", flush=True)
    out = _run_conv(hip, x, wt, None, bn, 1, s, p)
    idx = [0, 1, 33, 62, 63]
    _check(out[idx], np.ascontiguousarray(x[idx]), wt, None, bn, 1, s, p)


ODD = [
    # N, Cin, H, W, Cout, K, stride, pad
    (1, 1, 8, 8, 4, 3, 1, 1), (1, 1, 8, 8, 4, 3, 1, 0), (2, 3, 9, 9, 4, 3, 2, 1),
    (3, 5, 13, 11, 7, 3, 1, 1), (2, 7, 17, 19, 100, 5, 2, 2), (1, 16, 7, 7, 300, 1, 1, 0),
    (4, 3, 31, 29, 33, 7, 3, 3), (2, 64, 10, 10, 65, 3, 1, 1), (1, 2, 5, 5, 3, 5, 1, 0),
    # large kernels: 36 taps (64-bit tap mask), 81 taps (coordinate compares), both with K % 16 != 0
    (1, 2, 9, 9, 3, 6, 2, 2), (1, 1, 12, 12, 3, 9, 1, 4),
]


@pytest.mark.parametrize("geom", ODD)
@pytest.mark.parametrize("variant", ["plain", "bias", "bias_bn", "bn_relu", "bias_bn_relu"])
def test_odd_geometry(hip, geom, variant):
    N, cin, h, w, cout, k, s, p = geom
    seed = 100 + sum(geom)
    x = O.randn((N, cin, h, w), seed)
    wt = O.randn((cout, cin, k, k), seed + 1, 0.3)
    bias = O.randn((cout,), seed + 2) if "bias" in variant else None
    bn = _params(cout, seed + 3) if "bn" in variant else None
    act = 1 if "relu" in variant else 0
    if variant in ("plain", "bias"):
        out = _run_conv(hip, x, wt, bias, None, 0, s, p, entry="omHipConv2d")
    else:
        out = _run_conv(hip, x, wt, bias, bn, act, s, p)
    _check(out, x, wt, bias, bn, act, s, p)


# The implicit-GEMM loop keeps two K slices in flight; these reductions cover 1 to 5 whole
# slices of 16 (1x1 kernels over 16 ... 80 channels, the unmasked gather) and 2 to 5 slices
# with a partial last one (3x3 over 2 ... 8 channels).
SLICES = [(2, c, 12, 10, 24, 1, 1, 0) for c in (16, 32, 48, 64, 80)] + \
         [(2, c, 12, 10, 24, 3, 1, 1) for c in (2, 4, 6, 8)]


@pytest.mark.parametrize("geom", SLICES, ids=lambda g: "C{}k{}".format(g[1], g[5]))
def test_slice_counts(hip, geom):
    N, cin, h, w, cout, k, s, p = geom
    seed = 300 + cin + k
    x = O.randn((N, cin, h, w), seed)
    wt = O.randn((cout, cin, k, k), seed + 1, 0.3)
    bias = O.randn((cout,), seed + 2)
    bn = _params(cout, seed + 3)
    out = _run_conv(hip, x, wt, bias, bn, 1, s, p)
    _check(out, x, wt, bias, bn, 1, s, p)


# The RGB stem geometry (3 channels, 7x7, stride 2, pad 3, W % 4 == 0, W <= 224) runs on its own kernel:
# up to 7 consecutive output rows of one image per block, 64 channels per block (ragged Cout 40 and 100
# leave partial channel blocks), rows above / below the image and both side pads zero, Wo < 112 leaves
# partial pixel subtiles. On 256 CUs 8 x 101 output rows run 4 rows per block with a 1-row last block
# per image (the batch-32 ResNet stem, 7 rows per block, is in the b32 layer tests). W = 228 and
# W = 30 fall back to the general kernel.
STEM = [(2, 3, 224, 224, 64), (3, 3, 33, 64, 40), (1, 3, 17, 220, 100), (2, 3, 224, 4, 130), (1, 3, 7, 8, 64),
        (8, 3, 202, 96, 64), (1, 3, 20, 228, 64), (1, 3, 15, 30, 16)]


@pytest.mark.parametrize("geom", STEM, ids=lambda g: "N{}C{}H{}W{}o{}".format(*g))
@pytest.mark.parametrize("variant", ["plain", "bias", "bias_bn", "bn_relu", "bias_bn_relu"])
def test_stem_geometry(hip, geom, variant):
    N, cin, h, w, cout = geom
    seed = 300 + sum(geom)
    x = O.randn((N, cin, h, w), seed)
    wt = _kaiming_uniform((cout, cin, 7, 7), seed + 1)
    bias = O.randn((cout,), seed + 2) if "bias" in variant else None
    bn = _params(cout, seed + 3) if "bn" in variant else None
    act = 1 if "relu" in variant else 0
    print(f"case stem {geom} {variant}", flush=True)
    if variant in ("plain", "bias"):
        out = _run_conv(hip, x, wt, bias, None, 0, 2, 3, entry="omHipConv2d")
    else:
        out = _run_conv(hip, x, wt, bias, bn, act, 2, 3)
    _check(out, x, wt, bias, bn, act, 2, 3)


@pytest.mark.parametrize("geom", STEM[:3], ids=lambda g: "N{}C{}H{}W{}o{}".format(*g))
def test_stem_residual(hip, geom):
    """The stem kernel's residual epilogue: relu(BN(conv) + res) against float64 and the reference chain."""
    N, cin, h, w, cout = geom
    Ho, Wo = out_hw(h, 7, 2, 3), out_hw(w, 7, 2, 3)
    x = O.randn((N, cin, h, w), 41 + h)
    wt = _kaiming_uniform((cout, cin, 7, 7), 42)
    gam, bet, mu, var = _params(cout, 43)
    res = O.randn((N, cout, Ho, Wo), 44)
    dout = empty_dev(hip, (N, cout, Ho, Wo))
    print(f"case stem residual {geom}", flush=True)
    hip.HIPBackend.conv2dBiasBnAddAct(to_dev(hip, x), to_dev(hip, wt), None, to_dev(hip, gam), to_dev(hip, bet),
                                      to_dev(hip, mu), to_dev(hip, var), 1e-5, to_dev(hip, res), 1, dout, N, cin, h,
                                      w, cout, 7, 7, 2, 3)
    y64, bound = O.conv_f64(x, wt, None, 2, 3, gam, bet, mu, var, 1e-5, act=0)
    y64 = np.maximum(y64 + res, 0.0)
    bound = bound + np.abs(res)
    got = dout.numpy()
    assert O.normalized_error(got, y64, bound) <= TOL
    chain = O.relu(O.add(O.conv_bn_act(x, wt, None, gam, bet, mu, var, 1e-5, act=0, stride=2, pad=3), res))
    assert O.normalized_error(got, chain, bound) <= TOL


@pytest.mark.parametrize("geom", [(2, 3, 9, 9, 4, 3, 2, 1), (2, 64, 56, 56, 64, 3, 1, 1), (2, 3, 224, 224, 64, 7, 2, 3),
                                  (2, 256, 14, 14, 512, 1, 2, 0)])
def test_im2col_path(hip, geom):
    """omHipConv2dIm2col: explicit im2col + shared-weight batched GEMM + bias."""
    N, cin, h, w, cout, k, s, p = geom
    x = O.randn((N, cin, h, w), 500)
    wt = _kaiming_uniform((cout, cin, k, k), 501)
    bias = O.randn((cout,), 502)
    out = _run_conv(hip, x, wt, bias, None, 0, s, p, entry="omHipConv2dIm2col")
    _check(out, x, wt, bias, None, 0, s, p)


def test_conv_all_ones_interior(hip):
    """tests/test_conv.cpp:21-49 shapes; all-ones input -> interior = sum of weights."""
    x = np.ones((1, 1, 8, 8), np.float32)
    wt = O.randn((4, 1, 3, 3), 9)
    out = _run_conv(hip, x, wt, None, None, 0, 1, 1, entry="omHipConv2d")
    assert out.shape == (1, 4, 8, 8)
    s = wt.astype(np.float64).reshape(4, -1).sum(axis=1)
    for c in range(4):
        np.testing.assert_allclose(out[0, c, 1:7, 1:7], s[c], rtol=0, atol=1e-6)
    out0 = _run_conv(hip, x, wt, None, None, 0, 1, 0, entry="omHipConv2d")
    assert out0.shape == (1, 4, 6, 6)


def test_conv_invalid_arguments(hip):
    x = to_dev(hip, np.ones((1, 1, 4, 4), np.float32))
    w = to_dev(hip, np.ones((1, 1, 5, 5), np.float32))
    y = empty_dev(hip, (16,))
    with pytest.raises(hip.OmHipError):
        hip.call("omHipConv2d", x.ptr, w.ptr, None, y.ptr, 1, 1, 4, 4, 1, 5, 5, 1, 0)   # kernel > input
    with pytest.raises(hip.OmHipError):
        hip.call("omHipConv2d", x.ptr, w.ptr, None, y.ptr, 1, 1, 4, 4, 1, 3, 3, 0, 0)   # stride 0
    g = to_dev(hip, np.ones(1, np.float32))
    with pytest.raises(hip.OmHipError):   # partial BN parameters
        hip.call("omHipConv2dBiasBnAct", x.ptr, w.ptr, None, g.ptr, None, None, None, 1e-5, 1, y.ptr,
                 1, 1, 4, 4, 1, 3, 3, 1, 1)
