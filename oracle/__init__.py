"""The oracle: CPU restatement of the reference CPUBackend hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker (or the timed CPU baseline). The product library ``libomhip.so`` never
links, loads or calls anything here.

Contents
--------
``liboracle.so`` (``omref.cpp``)
    C++ restatement of ``CPUBackend::matmul / batchedMatmul / transpose2d /
    im2col / conv2d / batchNorm2d / relu / reluBackward / addBias`` and the
    ``MatMulBackward`` composition (reference files
    ``src/hal/om.hal.cpu_backend.ixx``, ``src/hal/om.hal.simd.ixx``,
    ``src/engine/om.engine.autograd.ixx``; line numbers at each function).
    Bit-identical to the reference CPUBackend compiled with clang.
``_ref/libomref_reference.so`` (optional, built by ``oracle/Makefile`` from the
    reference sources where they lie) — the reference CPUBackend itself.
float64 checkers (this file)
    ``gemm_f64`` / ``conv_f64`` return the float64 result together with the
    error budget ``sum_k |a_ik| |b_kj|`` used by the K-scaled tolerance
    ``|C - C64| <= tol * sum_k |a_ik||b_kj|`` (tol 1e-4 for fp32 inputs,
    1e-2 for fp16/bf16 inputs against fp32 CPUBackend).

Pinning (see tests/test_oracle_*.py): the restatement is checked bit-exactly
against the reference's own known-answer tests
(test_tensor_ops.cpp:55-82, test_phase5.cpp:206-222, test_nn.cpp:34-48),
against golden vectors written by the compiled reference (tests/golden/),
against ``_ref`` on fresh seeded inputs when it is built, and against float64
brute force plus closed forms (identity, transpose identity, linearity,
all-ones conv interior = sum of weights, BN closed form).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB: Optional[ctypes.CDLL] = None
_REF: Optional[ctypes.CDLL] = None
_REF_TRIED = False

_f = ctypes.POINTER(ctypes.c_float)
_u16 = ctypes.POINTER(ctypes.c_uint16)
_ip = ctypes.POINTER(ctypes.c_int)
_i = ctypes.c_int
_sz = ctypes.c_size_t


def lib_path() -> str:
    return os.path.join(_HERE, "liboracle.so")


def ref_path() -> str:
    return os.path.join(_HERE, "_ref", "libomref_reference.so")


def lib() -> ctypes.CDLL:
    """The restatement (liboracle.so). Raises if it was not built."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not os.path.exists(p):
            raise RuntimeError(f"oracle library missing: {p} (run `make -C oracle`)")
        L = ctypes.CDLL(p)
        sig = {
            "omrefMatmul": [_f, _f, _f, _i, _i, _i],
            "omrefMatmulTransB": [_f, _f, _f, _i, _i, _i],
            "omrefMatmulTransA": [_f, _f, _f, _i, _i, _i],
            "omrefBatchedMatmul": [_f, _f, _f, _i, _i, _i, _i],
            "omrefBatchedMatmulTransB": [_f, _f, _f, _i, _i, _i, _i],
            "omrefTranspose2d": [_f, _f, _i, _i],
            "omrefMatmulBackward": [_f, _f, _f, _f, _f, _i, _i, _i],
            "omrefIm2col": [_f, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f],
            "omrefConv2d": [_f, _f, _f, _f] + [_i] * 9,
            "omrefBatchNorm2d": [_f, _f, _f, _f, _f, _f, _f, _f, _i, _i, _i, _i,
                                 ctypes.c_float, ctypes.c_float, _i],
            "omrefRelu": [_f, _f, _sz],
            "omrefReluBackward": [_f, _f, _f, _sz],
            "omrefAddBias": [_f, _f, _f, _i, _i],
            "omrefConvBnRelu": [_f, _f, _f, _f, _f, _f, _f, ctypes.c_float, _i, _f] + [_i] * 9,
            "omrefFloatToHalfTruncN": [_f, _u16, _sz],
            "omrefFillValue": [_f, _sz, ctypes.c_float],
            "omrefCol2im": [_f, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f],
            "omrefConv2dBackwardInput": [_f, _f, _f] + [_i] * 9,
            "omrefConv2dBackwardWeight": [_f, _f, _f, _f] + [_i] * 9,
            "omrefBatchNorm2dBackward": [_f] * 8 + [_i] * 4,
            "omrefMaxPool2d": [_f, _f, _ip] + [_i] * 8,
            "omrefMaxPool2dBackward": [_f, _ip, _f] + [_i] * 6,
            "omrefAvgPool2d": [_f, _f] + [_i] * 8,
            "omrefAvgPool2dBackward": [_f, _f] + [_i] * 10,
            "omrefAdaptiveAvgPool2d": [_f, _f] + [_i] * 6,
            "omrefAdaptiveAvgPool2dBackward": [_f, _f] + [_i] * 6,
            "omrefAdd": [_f, _f, _f, _sz],
            "omrefSoftmax": [_f, _f, _i, _i],
            "omrefAttention": [_f, _f, _i, _i, _i, _i, ctypes.c_float],
            "omrefQkvSplitHeads": [_f, _f, _f, _f, _i, _i, _i, _i, ctypes.c_float],
            "omrefMergeHeads": [_f, _f, _i, _i, _i, _i],
            "omrefCrossEntropySoftmaxBackward": [_f, _f, _f, _i, _i],
            "omrefAddBiasBackward": [_f, _f, _i, _i, _i],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.omrefCrossEntropy.argtypes = [_f, _f, _i, _i]
        L.omrefCrossEntropy.restype = ctypes.c_float
        L.omrefSum.argtypes = [_f, _sz]
        L.omrefSum.restype = ctypes.c_float
        L.omrefHasAvx2.restype = ctypes.c_int
        L.omrefMaxThreads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def ref_lib() -> Optional[ctypes.CDLL]:
    """The compiled reference CPUBackend, or None when it was not built."""
    global _REF, _REF_TRIED
    if not _REF_TRIED:
        _REF_TRIED = True
        p = ref_path()
        if os.path.exists(p):
            R = ctypes.CDLL(p)
            sig = {
                "refMatmul": [_f, _f, _f, _i, _i, _i],
                "refBatchedMatmul": [_f, _f, _f, _i, _i, _i, _i],
                "refTranspose2d": [_f, _f, _i, _i],
                "refIm2col": [_f, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f],
                "refConv2d": [_f, _f, _f, _f] + [_i] * 9,
                "refBatchNorm2d": [_f, _f, _f, _f, _f, _f, _f, _f, _i, _i, _i, _i,
                                   ctypes.c_float, ctypes.c_float, _i],
                "refRelu": [_f, _f, _sz],
                "refReluBackward": [_f, _f, _f, _sz],
                "refAddBias": [_f, _f, _f, _i, _i],
                "refConv2dBackwardInput": [_f, _f, _f] + [_i] * 9,
                "refConv2dBackwardWeight": [_f, _f, _f, _f] + [_i] * 9,
                "refBatchNorm2dBackward": [_f] * 8 + [_i] * 4,
                "refMaxPool2d": [_f, _f, _ip] + [_i] * 8,
                "refMaxPool2dBackward": [_f, _ip, _f] + [_i] * 6,
                "refAvgPool2d": [_f, _f] + [_i] * 8,
                "refAvgPool2dBackward": [_f, _f] + [_i] * 10,
                "refAdaptiveAvgPool2d": [_f, _f] + [_i] * 6,
                "refAdaptiveAvgPool2dBackward": [_f, _f] + [_i] * 6,
                "refAdd": [_f, _f, _f, _sz],
                "refSoftmax": [_f, _f, _i, _i],
                "refCrossEntropySoftmaxBackward": [_f, _f, _f, _i, _i],
            }
            for name, args in sig.items():
                fn = getattr(R, name)
                fn.argtypes = args
                fn.restype = None
            R.refCrossEntropy.argtypes = [_f, _f, _i, _i]
            R.refCrossEntropy.restype = ctypes.c_float
            if hasattr(R, "refSum"):
                R.refSum.argtypes = [_f, _sz]
                R.refSum.restype = ctypes.c_float
            _REF = R
    return _REF


def _p(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle takes C-contiguous float32"
    return a.ctypes.data_as(_f)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------
# restatement wrappers (numpy in, numpy out)
# ---------------------------------------------------------------------------

def matmul(A, B, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::matmul (cpu_backend.ixx:239-286): C[M,N] = A[M,K] B[K,N]."""
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), np.float32)
    if backend == "reference":
        ref_lib().refMatmul(_p(A), _p(B), _p(C), M, K, N)
    else:
        lib().omrefMatmul(_p(A), _p(B), _p(C), M, K, N)
    return C


def matmul_transB(A, Bnk) -> np.ndarray:
    """transpose2d(B) + matmul: A[M,K] x B[N,K]^T (autograd.ixx:261-273)."""
    A, Bnk = _f32(A), _f32(Bnk)
    M, K = A.shape
    N = Bnk.shape[0]
    C = np.empty((M, N), np.float32)
    lib().omrefMatmulTransB(_p(A), _p(Bnk), _p(C), M, K, N)
    return C


def matmul_transA(Akm, B) -> np.ndarray:
    """transpose2d(A) + matmul: A[K,M]^T x B[K,N] (autograd.ixx:276-286)."""
    Akm, B = _f32(Akm), _f32(B)
    K, M = Akm.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().omrefMatmulTransA(_p(Akm), _p(B), _p(C), M, K, N)
    return C


def batched_matmul(A, B, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::batchedMatmul (cpu_backend.ixx:1520-1532)."""
    A, B = _f32(A), _f32(B)
    b, M, K = A.shape
    N = B.shape[2]
    C = np.empty((b, M, N), np.float32)
    if backend == "reference":
        ref_lib().refBatchedMatmul(_p(A), _p(B), _p(C), b, M, K, N)
    else:
        lib().omrefBatchedMatmul(_p(A), _p(B), _p(C), b, M, K, N)
    return C


def batched_matmul_transB(A, Bnk) -> np.ndarray:
    A, Bnk = _f32(A), _f32(Bnk)
    b, M, K = A.shape
    N = Bnk.shape[1]
    C = np.empty((b, M, N), np.float32)
    lib().omrefBatchedMatmulTransB(_p(A), _p(Bnk), _p(C), b, M, K, N)
    return C


def transpose2d(A, backend: str = "oracle") -> np.ndarray:
    A = _f32(A)
    r, c = A.shape
    out = np.empty((c, r), np.float32)
    (ref_lib().refTranspose2d if backend == "reference" else lib().omrefTranspose2d)(_p(A), _p(out), r, c)
    return out


def matmul_backward(G, A, B) -> Tuple[np.ndarray, np.ndarray]:
    """MatMulBackward::backward (autograd.ixx:226-290): (dA, dB)."""
    G, A, B = _f32(G), _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    dA = np.empty((M, K), np.float32)
    dB = np.empty((K, N), np.float32)
    lib().omrefMatmulBackward(_p(G), _p(A), _p(B), _p(dA), _p(dB), M, K, N)
    return dA, dB


def out_hw(H, W, KH, KW, stride, pad):
    return (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1


def im2col(x, KH, KW, pad, stride, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::im2col (cpu_backend.ixx:544-575) of one image x[Cin,H,W]."""
    x = _f32(x)
    Cin, H, W = x.shape
    Ho, Wo = out_hw(H, W, KH, KW, stride, pad)
    col = np.empty((Cin * KH * KW, Ho * Wo), np.float32)
    fn = ref_lib().refIm2col if backend == "reference" else lib().omrefIm2col
    fn(_p(x), Cin, H, W, KH, KW, pad, pad, stride, stride, _p(col))
    return col


def conv2d(x, w, bias=None, stride=1, pad=0, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::conv2d (cpu_backend.ixx:619-658), NCHW."""
    x, w = _f32(x), _f32(w)
    N, Cin, H, W = x.shape
    Cout, Cin2, KH, KW = w.shape
    assert Cin == Cin2
    Ho, Wo = out_hw(H, W, KH, KW, stride, pad)
    out = np.empty((N, Cout, Ho, Wo), np.float32)
    b = _f32(bias) if bias is not None else None
    fn = ref_lib().refConv2d if backend == "reference" else lib().omrefConv2d
    fn(_p(x), _p(w), _p(b), _p(out), N, Cin, H, W, Cout, KH, KW, stride, pad)
    return out


def batchnorm2d_eval(x, gamma, beta, mean, var, eps=1e-5, backend: str = "oracle"):
    """CPUBackend::batchNorm2d with bTraining=false (cpu_backend.ixx:781-842).

    Returns (y, savedMean, savedInvStd)."""
    x = _f32(x)
    N, C, H, W = x.shape
    y = np.empty_like(x)
    rm, rv = _f32(mean).copy(), _f32(var).copy()
    sm = np.empty(C, np.float32)
    si = np.empty(C, np.float32)
    fn = ref_lib().refBatchNorm2d if backend == "reference" else lib().omrefBatchNorm2d
    fn(_p(x), _p(y), _p(_f32(gamma)), _p(_f32(beta)), _p(rm), _p(rv), _p(sm), _p(si), N, C, H, W,
       ctypes.c_float(eps), ctypes.c_float(0.1), 0)
    return y, sm, si


def batchnorm2d_train(x, gamma, beta, run_mean, run_var, eps=1e-5, momentum=0.1, backend: str = "oracle"):
    """Training branch (cpu_backend.ixx:796-822): returns (y, runMean', runVar', savedMean, savedInvStd)."""
    x = _f32(x)
    N, C, H, W = x.shape
    y = np.empty_like(x)
    rm, rv = _f32(run_mean).copy(), _f32(run_var).copy()
    sm = np.empty(C, np.float32)
    si = np.empty(C, np.float32)
    fn = ref_lib().refBatchNorm2d if backend == "reference" else lib().omrefBatchNorm2d
    fn(_p(x), _p(y), _p(_f32(gamma)), _p(_f32(beta)), _p(rm), _p(rv), _p(sm), _p(si), N, C, H, W,
       ctypes.c_float(eps), ctypes.c_float(momentum), 1)
    return y, rm, rv, sm, si


def relu(x, backend: str = "oracle") -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    (ref_lib().refRelu if backend == "reference" else lib().omrefRelu)(_p(x), _p(y), x.size)
    return y


def relu_backward(x, g, backend: str = "oracle") -> np.ndarray:
    x, g = _f32(x), _f32(g)
    gi = np.empty_like(x)
    (ref_lib().refReluBackward if backend == "reference" else lib().omrefReluBackward)(_p(x), _p(g), _p(gi), x.size)
    return gi


def add_bias(A, bias, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::addBias (cpu_backend.ixx:433-440): out[b,j] = A[b,j] + bias[j]."""
    A, bias = _f32(A), _f32(bias)
    b, c = A.shape
    out = np.empty_like(A)
    (ref_lib().refAddBias if backend == "reference" else lib().omrefAddBias)(_p(A), _p(bias), _p(out), b, c)
    return out


def conv_bn_act(x, w, bias, gamma, beta, mean, var, eps=1e-5, act=1, stride=1, pad=0) -> np.ndarray:
    """conv2d -> batchNorm2d(eval) -> relu: the unfused reference chain."""
    x, w = _f32(x), _f32(w)
    N, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    Ho, Wo = out_hw(H, W, KH, KW, stride, pad)
    out = np.empty((N, Cout, Ho, Wo), np.float32)
    b = _f32(bias) if bias is not None else None
    g = _f32(gamma) if gamma is not None else None
    bt = _f32(beta) if beta is not None else None
    m = _f32(mean) if mean is not None else None
    v = _f32(var) if var is not None else None
    lib().omrefConvBnRelu(_p(x), _p(w), _p(b), _p(g), _p(bt), _p(m), _p(v), ctypes.c_float(eps), act, _p(out),
                          N, Cin, H, W, Cout, KH, KW, stride, pad)
    return out


def _fn(name: str, backend: str):
    return getattr(ref_lib(), "ref" + name) if backend == "reference" else getattr(lib(), "omref" + name)


def conv2d_backward_input(gO, w, H, W, stride=1, pad=0, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::conv2dBackwardInput (cpu_backend.ixx:666-705): col2im(W^T gO) per image."""
    gO, w = _f32(gO), _f32(w)
    N, Cout, Ho, Wo = gO.shape
    Cout2, Cin, KH, KW = w.shape
    assert Cout == Cout2 and out_hw(H, W, KH, KW, stride, pad) == (Ho, Wo)
    gI = np.empty((N, Cin, H, W), np.float32)
    _fn("Conv2dBackwardInput", backend)(_p(gO), _p(w), _p(gI), N, Cin, H, W, Cout, KH, KW, stride, pad)
    return gI


def conv2d_backward_weight(x, gO, KH, KW, stride=1, pad=0, bias=True, backend: str = "oracle"):
    """CPUBackend::conv2dBackwardWeight (cpu_backend.ixx:710-772): (gradWeight, gradBias or None)."""
    x, gO = _f32(x), _f32(gO)
    N, Cin, H, W = x.shape
    N2, Cout, Ho, Wo = gO.shape
    assert N == N2 and out_hw(H, W, KH, KW, stride, pad) == (Ho, Wo)
    gW = np.empty((Cout, Cin, KH, KW), np.float32)
    gB = np.empty(Cout, np.float32) if bias else None
    _fn("Conv2dBackwardWeight", backend)(_p(x), _p(gO), _p(gW), _p(gB), N, Cin, H, W, Cout, KH, KW, stride, pad)
    return gW, gB


def batchnorm2d_backward(gO, x, mean, inv_std, gamma, backend: str = "oracle"):
    """CPUBackend::batchNorm2dBackward (cpu_backend.ixx:847-890): (gradInput, gradGamma, gradBeta)."""
    gO, x = _f32(gO), _f32(x)
    N, C, H, W = x.shape
    gI = np.empty_like(x)
    gG = np.empty(C, np.float32)
    gB = np.empty(C, np.float32)
    _fn("BatchNorm2dBackward", backend)(_p(gO), _p(x), _p(_f32(mean)), _p(_f32(inv_std)), _p(_f32(gamma)), _p(gI),
                                        _p(gG), _p(gB), N, C, H, W)
    return gI, gG, gB


def _ipt(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_ip)


def maxpool2d(x, K, stride, pad, backend: str = "oracle"):
    """CPUBackend::maxPool2d (cpu_backend.ixx:897-934): (output, flat input index per output)."""
    x = _f32(x)
    N, C, H, W = x.shape
    Ho, Wo = out_hw(H, W, K, K, stride, pad)
    y = np.empty((N, C, Ho, Wo), np.float32)
    idx = np.empty((N, C, Ho, Wo), np.int32)
    _fn("MaxPool2d", backend)(_p(x), _p(y), _ipt(idx), N, C, H, W, K, K, stride, pad)
    return y, idx


def maxpool2d_backward(gO, idx, H, W, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::maxPool2dBackward (cpu_backend.ixx:937-955)."""
    gO = _f32(gO)
    idx = np.ascontiguousarray(idx, np.int32)
    N, C, Ho, Wo = gO.shape
    gI = np.empty((N, C, H, W), np.float32)
    _fn("MaxPool2dBackward", backend)(_p(gO), _ipt(idx), _p(gI), N, C, Ho, Wo, H, W)
    return gI


def avgpool2d(x, K, stride, pad, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::avgPool2d (cpu_backend.ixx:958-990): padding counts in the divisor."""
    x = _f32(x)
    N, C, H, W = x.shape
    Ho, Wo = out_hw(H, W, K, K, stride, pad)
    y = np.empty((N, C, Ho, Wo), np.float32)
    _fn("AvgPool2d", backend)(_p(x), _p(y), N, C, H, W, K, K, stride, pad)
    return y


def avgpool2d_backward(gO, H, W, K, stride, pad, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::avgPool2dBackward (cpu_backend.ixx:994-1023)."""
    gO = _f32(gO)
    N, C, Ho, Wo = gO.shape
    gI = np.empty((N, C, H, W), np.float32)
    _fn("AvgPool2dBackward", backend)(_p(gO), _p(gI), N, C, H, W, Ho, Wo, K, K, stride, pad)
    return gI


def adaptive_avgpool2d(x, OH, OW, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::adaptiveAvgPool2d (cpu_backend.ixx:1467-1488)."""
    x = _f32(x)
    N, C, H, W = x.shape
    y = np.empty((N, C, OH, OW), np.float32)
    _fn("AdaptiveAvgPool2d", backend)(_p(x), _p(y), N, C, H, W, OH, OW)
    return y


def adaptive_avgpool2d_backward(gO, H, W, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::adaptiveAvgPool2dBackward (cpu_backend.ixx:1491-1510)."""
    gO = _f32(gO)
    N, C, OH, OW = gO.shape
    gI = np.empty((N, C, H, W), np.float32)
    _fn("AdaptiveAvgPool2dBackward", backend)(_p(gO), _p(gI), N, C, H, W, OH, OW)
    return gI


def add(a, b, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::add (cpu_backend.ixx:147-160)."""
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    _fn("Add", backend)(_p(a), _p(b), _p(out), a.size)
    return out


def softmax(x, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::softmax over the last axis (cpu_backend.ixx:352-370)."""
    x = _f32(x)
    out = np.empty_like(x)
    _fn("Softmax", backend)(_p(x), _p(out), x.size // x.shape[-1], x.shape[-1])
    return out


def cross_entropy(pred, target, backend: str = "oracle") -> float:
    """CPUBackend::crossEntropy (cpu_backend.ixx:375-388): -sum log(max(p, 1e-7)) over the
    elements whose target exceeds 0.5, divided by the batch (float32)."""
    pred, target = _f32(pred), _f32(target)
    rows, cols = pred.size // pred.shape[-1], pred.shape[-1]
    if backend == "reference":
        R = ref_lib()
        if R is None:
            raise RuntimeError("the compiled reference (oracle/_ref) is not built")
        return float(np.float32(R.refCrossEntropy(_p(pred), _p(target), rows, cols)))
    return float(np.float32(lib().omrefCrossEntropy(_p(pred), _p(target), rows, cols)))


def cross_entropy_softmax_backward(s, target, backend: str = "oracle") -> np.ndarray:
    """CPUBackend::crossEntropySoftmaxBackward (cpu_backend.ixx:393-410): (s - t) * (1 / batch)."""
    s, target = _f32(s), _f32(target)
    out = np.empty_like(s)
    _fn("CrossEntropySoftmaxBackward", backend)(_p(s), _p(target), _p(out), s.size // s.shape[-1], s.shape[-1])
    return out


def add_bias_backward(g, N, C, HW=1) -> np.ndarray:
    """AddBiasBackward's bias gradient (autograd.ixx:428-433): per channel, the zeroed
    gradient adds every (n, hw) element in order."""
    g = _f32(g)
    out = np.empty(C, np.float32)
    lib().omrefAddBiasBackward(_p(g), _p(out), N, C, HW)
    return out


def attention(qkv, B, S, H, D, scale, backend: str = "oracle") -> np.ndarray:
    """MultiHeadAttention's core after the QKV projection (vit.ixx:193-236):
    qkv [B*S, 3*H*D] -> merged-head context [B*S, H*D]. With backend="reference"
    the matmuls, transposes and softmax are the compiled reference's own."""
    qkv = _f32(qkv)
    if backend != "reference":
        out = np.empty((B * S, H * D), np.float32)
        lib().omrefAttention(_p(qkv), _p(out), B, S, H, D, ctypes.c_float(scale))
        return out
    t = qkv.reshape(B, S, 3, H, D)
    Q = np.ascontiguousarray((t[:, :, 0] * np.float32(scale)).transpose(0, 2, 1, 3)).reshape(B * H, S, D)
    K = np.ascontiguousarray(t[:, :, 1].transpose(0, 2, 1, 3)).reshape(B * H, S, D)
    V = np.ascontiguousarray(t[:, :, 2].transpose(0, 2, 1, 3)).reshape(B * H, S, D)
    kT = np.stack([transpose2d(K[i], backend="reference") for i in range(B * H)])
    sc = batched_matmul(Q, kT, backend="reference")
    P = softmax(sc, backend="reference")
    ctx = batched_matmul(P, V, backend="reference")
    return np.ascontiguousarray(ctx.reshape(B, H, S, D).transpose(0, 2, 1, 3)).reshape(B * S, H * D)


def sum_(x, backend: str = "oracle") -> np.float32:
    """CPUBackend::sum (cpu_backend.ixx:290-294): a float accumulator over the elements in order."""
    x = _f32(x).reshape(-1)
    if backend == "reference":
        R = ref_lib()
        if R is None or not hasattr(R, "refSum"):
            raise RuntimeError("the compiled reference (oracle/_ref) is not built")
        return np.float32(R.refSum(_p(x), x.size))
    return np.float32(lib().omrefSum(_p(x), x.size))


def qkv_split_heads(qkv, B, S, H, D, scale):
    """MultiHeadAttention::forward's split (vit.ixx:196-212): Q*scale, K, V as [B*H, S, D]."""
    qkv = _f32(qkv)
    q, k, v = (np.empty((B * H, S, D), np.float32) for _ in range(3))
    lib().omrefQkvSplitHeads(_p(qkv), _p(q), _p(k), _p(v), B, S, H, D, ctypes.c_float(scale))
    return q, k, v


def merge_heads(x, B, S, H, D):
    """MultiHeadAttention::forward's merge (vit.ixx:220-232): [B*H, S, D] -> [B*S, H*D]."""
    x = _f32(x)
    out = np.empty((B * S, H * D), np.float32)
    lib().omrefMergeHeads(_p(x), _p(out), B, S, H, D)
    return out


def attention_f64(qkv, B, S, H, D, scale):
    """float64 attention from the given (rounded) inputs, and the error budget
    sum_j P_ij |V_jd| of each context element."""
    t = np.asarray(qkv, np.float64).reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)   # 3 B H S D
    Q, K, V = t[0], t[1], t[2]
    s = scale * np.matmul(Q, np.swapaxes(K, -1, -2))
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    P = e / e.sum(axis=-1, keepdims=True)
    ctx = np.matmul(P, V)
    bound = np.matmul(P, np.abs(V))
    f = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(B * S, H * D)
    return f(ctx), f(bound)


def float_to_half_trunc(x) -> np.ndarray:
    """FP16Converter::floatToHalf (fp16.ixx:36-100): truncating fp32 -> fp16 bits."""
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().omrefFloatToHalfTruncN(_p(x), out.ctypes.data_as(_u16), x.size)
    return out


# ---------------------------------------------------------------------------
# float64 checkers and the K-scaled tolerance
# ---------------------------------------------------------------------------

def gemm_f64(A, B, transA=False, transB=False) -> Tuple[np.ndarray, np.ndarray]:
    """float64 C = op(A) op(B) and the error budget |op(A)| |op(B)|."""
    A64 = np.asarray(A, np.float64)
    B64 = np.asarray(B, np.float64)
    if transA:
        A64 = np.swapaxes(A64, -1, -2)
    if transB:
        B64 = np.swapaxes(B64, -1, -2)
    return A64 @ B64, np.abs(A64) @ np.abs(B64)


def _im2col64(x64, KH, KW, stride, pad):
    N, C, H, W = x64.shape
    Ho, Wo = out_hw(H, W, KH, KW, stride, pad)
    xp = np.zeros((N, C, H + 2 * pad, W + 2 * pad), np.float64)
    xp[:, :, pad:pad + H, pad:pad + W] = x64
    cols = np.empty((N, C, KH, KW, Ho, Wo), np.float64)
    for kh in range(KH):
        for kw in range(KW):
            cols[:, :, kh, kw] = xp[:, :, kh:kh + stride * (Ho - 1) + 1:stride, kw:kw + stride * (Wo - 1) + 1:stride]
    return cols.reshape(N, C * KH * KW, Ho * Wo), Ho, Wo


def conv_f64(x, w, bias=None, stride=1, pad=0, gamma=None, beta=None, mean=None, var=None, eps=1e-5, act=0):
    """float64 direct convolution (+ bias, BN eval, ReLU) and its error budget.

    The budget is conv(|x|,|w|) scaled by |gamma|*invStd when BN is applied;
    ReLU does not enlarge it (|relu(a)-relu(b)| <= |a-b|)."""
    x64 = np.asarray(x, np.float64)
    w64 = np.asarray(w, np.float64)
    N = x64.shape[0]
    Cout, Cin, KH, KW = w64.shape
    cols, Ho, Wo = _im2col64(x64, KH, KW, stride, pad)
    wm = w64.reshape(Cout, -1)
    out = np.matmul(wm[None], cols).reshape(N, Cout, Ho, Wo)
    bound = np.matmul(np.abs(wm)[None], np.abs(cols)).reshape(N, Cout, Ho, Wo)
    if bias is not None:
        b = np.asarray(bias, np.float64)[None, :, None, None]
        out = out + b
        bound = bound + np.abs(b)
    if gamma is not None:
        g = np.asarray(gamma, np.float64)[None, :, None, None]
        bt = np.asarray(beta, np.float64)[None, :, None, None]
        m = np.asarray(mean, np.float64)[None, :, None, None]
        inv = 1.0 / np.sqrt(np.asarray(var, np.float64) + eps)[None, :, None, None]
        out = g * (out - m) * inv + bt
        bound = (bound + np.abs(m)) * np.abs(g) * inv + np.abs(bt)
    if act == 1:
        out = np.maximum(out, 0.0)
    return out, bound


def conv_backward_f64(x, w, gO, stride=1, pad=0):
    """float64 gradients of out = conv(x, w) for upstream gO, and their error budgets.

    dX = W^T gO scattered back (col2im), dW = gO im2col(x)^T, dB = sum gO; the
    budgets are the same contractions over absolute values."""
    x64 = np.asarray(x, np.float64)
    w64 = np.asarray(w, np.float64)
    g64 = np.asarray(gO, np.float64)
    N, Cin, H, W = x64.shape
    Cout, _, KH, KW = w64.shape
    cols, Ho, Wo = _im2col64(x64, KH, KW, stride, pad)
    wm = w64.reshape(Cout, -1)
    gm = g64.reshape(N, Cout, Ho * Wo)
    dW = np.einsum("nop,nkp->ok", gm, cols).reshape(w64.shape)
    dWb = np.einsum("nop,nkp->ok", np.abs(gm), np.abs(cols)).reshape(w64.shape)
    dB = gm.sum(axis=(0, 2))
    dBb = np.abs(gm).sum(axis=(0, 2))
    dcol = np.matmul(wm.T[None], gm)
    dcolb = np.matmul(np.abs(wm).T[None], np.abs(gm))
    dX = _col2im64(dcol, N, Cin, H, W, KH, KW, stride, pad)
    dXb = _col2im64(dcolb, N, Cin, H, W, KH, KW, stride, pad)
    return (dX, dXb), (dW, dWb), (dB, dBb)


def _col2im64(cols, N, C, H, W, KH, KW, stride, pad):
    Ho, Wo = out_hw(H, W, KH, KW, stride, pad)
    cols = cols.reshape(N, C, KH, KW, Ho, Wo)
    xp = np.zeros((N, C, H + 2 * pad, W + 2 * pad), np.float64)
    for kh in range(KH):
        for kw in range(KW):
            xp[:, :, kh:kh + stride * (Ho - 1) + 1:stride, kw:kw + stride * (Wo - 1) + 1:stride] += cols[:, :, kh, kw]
    return xp[:, :, pad:pad + H, pad:pad + W]


def bn_train_f64(x, gamma, beta, eps=1e-5):
    """float64 BN training forward: (y, batch mean, biased var, invStd)."""
    x64 = np.asarray(x, np.float64)
    mean = x64.mean(axis=(0, 2, 3))
    var = ((x64 - mean[None, :, None, None]) ** 2).mean(axis=(0, 2, 3))
    inv = 1.0 / np.sqrt(var + eps)
    y = np.asarray(gamma, np.float64)[None, :, None, None] * (x64 - mean[None, :, None, None]) * inv[None, :, None, None] \
        + np.asarray(beta, np.float64)[None, :, None, None]
    return y, mean, var, inv


def bn_backward_f64(gO, x, mean, inv_std, gamma):
    """float64 BN backward with the given statistics: (dX, dGamma, dBeta) and dX's error budget."""
    g64 = np.asarray(gO, np.float64)
    x64 = np.asarray(x, np.float64)
    m = np.asarray(mean, np.float64)[None, :, None, None]
    inv = np.asarray(inv_std, np.float64)[None, :, None, None]
    gam = np.asarray(gamma, np.float64)[None, :, None, None]
    cnt = x64.shape[0] * x64.shape[2] * x64.shape[3]
    xh = (x64 - m) * inv
    dG = (g64 * xh).sum(axis=(0, 2, 3))
    dB = g64.sum(axis=(0, 2, 3))
    dX = gam * inv / cnt * (cnt * g64 - dB[None, :, None, None] - xh * dG[None, :, None, None])
    absG = np.abs(g64).sum(axis=(0, 2, 3))
    absGX = (np.abs(g64) * np.abs(xh)).sum(axis=(0, 2, 3))
    bound = np.abs(gam) * inv / cnt * (cnt * np.abs(g64) + absG[None, :, None, None] + np.abs(xh) * absGX[None, :, None, None])
    return dX, dG, dB, bound, absGX, absG


def normalized_error(C, C64, bound) -> float:
    """max |C - C64| / max(bound, tiny): the K-scaled error measure."""
    C = np.asarray(C, np.float64)
    d = np.abs(C - C64)
    den = np.maximum(bound, np.finfo(np.float64).tiny)
    return float(np.max(d / den)) if d.size else 0.0


def frobenius_rel(C, Cref) -> float:
    C = np.asarray(C, np.float64)
    R = np.asarray(Cref, np.float64)
    n = np.linalg.norm(R)
    return float(np.linalg.norm(C - R) / n) if n > 0 else float(np.linalg.norm(C))


# Tolerances: fp32 inputs 1e-4; fp16/bf16 inputs with fp32 accumulate 1e-2.
TOL_FP32 = 1e-4
TOL_HALF = 1e-2


# ---------------------------------------------------------------------------
# seeded data
# ---------------------------------------------------------------------------

def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def randn(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def uniform(shape, seed: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    return rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 -> fp32 with round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), r)
    return (r.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)
