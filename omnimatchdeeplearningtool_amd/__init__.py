"""omnimatchdeeplearningtool_amd — MI355X (gfx950) compute backend for the
OmniMatch HAL matmul / conv2d hot path.

The product is ``libomhip.so`` (C ABI declared in ``include/omhip.h``) and the
C++23 ``om::HIPBackend`` in ``include/omhip_backend.hpp``. This Python module
is the host-side mirror used by tests and the bench:

* :func:`lib` loads ``libomhip.so`` (ctypes, signatures from the header) and
  raises if it is missing — there is no CPU fallback;
* :class:`DeviceBuffer` owns device memory from the library's caching pool;
* :class:`HIPBackend` exposes the HAL with the reference ``CPUBackend`` method
  names and argument order (src/hal/om.hal.cpu_backend.ixx), taking device
  pointers; a failing call raises ``RuntimeError`` with the library's message
  instead of being swallowed as ``CUDABackend`` does (om.hal.cuda_backend.ixx:283-983).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

__all__ = ["lib", "lib_path", "DeviceBuffer", "HIPBackend", "OmHipError", "init", "synchronize", "set_stream", "release_stream"]

_PKG = os.path.dirname(os.path.abspath(__file__))
_LIB: Optional[ctypes.CDLL] = None


class OmHipError(RuntimeError):
    pass


def lib_path() -> str:
    return os.path.join(_PKG, "libomhip.so")


_vp = ctypes.c_void_p
_i = ctypes.c_int
_ll = ctypes.c_longlong
_sz = ctypes.c_size_t
_fl = ctypes.c_float

# name -> argtypes (all return int)
_SIGS = {
    "omHipInit": [_i],
    "omHipGetDeviceCount": [],
    "omHipGetDeviceName": [_i, ctypes.c_char_p, _i],
    "omHipGetMemInfo": [_i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)],
    "omHipGetComputeCapability": [_i, ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "omHipSynchronize": [],
    "omHipSyncComputeStream": [],
    "omHipCleanup": [],
    "omHipForceReset": [],
    "omHipSum": [_vp, _vp, _i],
    "omHipMean": [_vp, _vp, _i],
    "omHipQkvSplitHeads": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _fl],
    "omHipMergeHeads": [_vp, _vp, _i, _i, _i, _i],
    "omHipAttention": [_vp, _vp, _i, _i, _i, _i, _fl],
    "omHipGetStream": [ctypes.POINTER(_vp)],
    "omHipSoftmax": [_vp, _vp, _i, _i],
    "omHipCrossEntropy": [_vp, _vp, _vp, _i, _i],
    "omHipSoftmaxCrossEntropyBackward": [_vp, _vp, _vp, _i, _i],
    "omHipSoftmaxCrossEntropy": [_vp, _vp, _vp, _vp, _vp, _i, _i],
    "omHipAddBiasBackward": [_vp, _vp, _i, _i, _i],
    "omHipSetStream": [_vp],
    "omHipReleaseStream": [_vp],
    "omHipMalloc": [ctypes.POINTER(_vp), _sz],
    "omHipFree": [_vp],
    "omHipCopyH2D": [_vp, _vp, _sz],
    "omHipCopyD2H": [_vp, _vp, _sz],
    "omHipCopyD2D": [_vp, _vp, _sz],
    "omHipMemset": [_vp, _i, _sz],
    "omHipPoolStats": [ctypes.POINTER(_sz), ctypes.POINTER(_sz)],
    "omHipMallocHost": [ctypes.POINTER(_vp), _sz],
    "omHipFreeHost": [_vp],
    "omHipAsyncCopyH2D": [_vp, _vp, _sz],
    "omHipAsyncCopyD2H": [_vp, _vp, _sz],
    "omHipSyncTransferStream": [],
    "omHipComputeWaitTransfer": [],
    "omHipTransferWaitCompute": [],
    "omHipGraphBeginCapture": [],
    "omHipGraphEndCapture": [ctypes.POINTER(_vp)],
    "omHipGraphLaunch": [_vp],
    "omHipGraphDestroy": [_vp],
    "omHipResNet18Create": [_vp, _ll, _i, _i, ctypes.POINTER(_vp)],
    "omHipResNet18Destroy": [_vp],
    "omHipResNet18Forward": [_vp, _vp, _vp, _i],
    "omHipResNet18InferBatch": [_vp, _vp, _i, _i, _i, _i, _i, _i, _fl, _vp, _vp, _vp],
    "omHipPoolTrim": [],
    "omHipFillZeros": [_vp, _i],
    "omHipFillOnes": [_vp, _i],
    "omHipFillValue": [_vp, _i, _fl],
    "omHipCopy": [_vp, _vp, _i],
    "omHipReLU": [_vp, _vp, _i],
    "omHipReLUBackward": [_vp, _vp, _vp, _i],
    "omHipAddBias": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmul": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmulTransB": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmulTransA": [_vp, _vp, _vp, _i, _i, _i],
    "omHipLinearBiasAct": [_vp, _vp, _vp, _vp, _i, _i, _i, _i],
    "omHipLinearBackward": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "omHipLinearSoftmaxCrossEntropyStep": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "omHipBatchedMatmul": [_vp, _vp, _vp, _i, _i, _i, _i],
    "omHipBatchedMatmulTransB": [_vp, _vp, _vp, _i, _i, _i, _i],
    "omHipGemmStridedBatched": [_i, _i, _i, _i, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll],
    "omHipGemmStridedBatchedNoAlloc": [_i, _i, _i, _i, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll],
    "omHipTranspose": [_vp, _vp, _i, _i],
    "omHipConv2d": [_vp, _vp, _vp, _vp] + [_i] * 9,
    "omHipConv2dIm2col": [_vp, _vp, _vp, _vp] + [_i] * 9,
    "omHipConv2dBiasBnAct": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _fl, _i, _vp] + [_i] * 9,
    "omHipIm2col": [_vp] + [_i] * 9 + [_vp],
    "omHipBatchNorm2d": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _fl, _fl, _i],
    "omHipConv2dBackwardInput": [_vp, _vp, _vp] + [_i] * 9,
    "omHipConv2dBackwardWeight": [_vp, _vp, _vp, _vp] + [_i] * 9,
    "omHipBatchNorm2dBackward": [_vp] * 8 + [_i] * 4 + [_fl],
    "omHipMaxPool2d": [_vp, _vp, _vp] + [_i] * 10,
    "omHipMaxPool2dBackward": [_vp, _vp, _vp] + [_i] * 6,
    "omHipMaxPool2dBackwardEx": [_vp, _vp, _vp] + [_i] * 10,
    "omHipAvgPool2d": [_vp, _vp] + [_i] * 10,
    "omHipAvgPool2dBackward": [_vp, _vp] + [_i] * 10,
    "omHipAdaptiveAvgPool2d": [_vp, _vp] + [_i] * 6,
    "omHipAdaptiveAvgPool2dBackward": [_vp, _vp] + [_i] * 6,
    "omHipAdd": [_vp, _vp, _vp, _i],
    "omHipAddReluBackward": [_vp, _vp, _vp, _vp, _i],
    "omHipBatchNorm2dTrainAct": [_vp] * 8 + [_i] * 4 + [_fl, _fl, _vp, _i],
    "omHipBatchNorm2dBackwardRelu": [_vp] * 9 + [_i] * 4 + [_fl],
    "omHipConv2dBiasBnAddAct": [_vp] * 7 + [_fl, _vp, _i, _vp] + [_i] * 9,
    "omHipAttentionHalf": [_i, _vp, _vp, _i, _i, _i, _i, _i, _fl],
    "omHipLinearHalf": [_i, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i],
    "omHipMultiHeadAttentionHalf": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i],
    "omHipConvertF32ToF16": [_vp, _vp, _i],
    "omHipConvertF32ToBF16": [_vp, _vp, _i],
    "omHipConvertF16ToF32": [_vp, _vp, _i],
    "omHipConvertBF16ToF32": [_vp, _vp, _i],
    "omHipMatmulF16": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmulBF16": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmulTransBF16": [_vp, _vp, _vp, _i, _i, _i],
    "omHipMatmulTransBBF16": [_vp, _vp, _vp, _i, _i, _i],
    "omHipGemmStridedBatchedHalf": [_i, _i, _i, _i, _i, _i, _i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll],
}


def lib() -> ctypes.CDLL:
    """Loads libomhip.so; raises OmHipError when it has not been built."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not os.path.exists(p):
            raise OmHipError(f"libomhip.so not built at {p}: run `python -m omnimatchdeeplearningtool_amd.build`")
        L = ctypes.CDLL(p)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.omHipGetLastError.argtypes = []
        L.omHipGetLastError.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().omHipGetLastError().decode(errors="replace")
        raise OmHipError(f"{what} failed: {msg}")


def call(name: str, *args) -> None:
    """Calls a C ABI entry and raises OmHipError on a nonzero status."""
    _check(getattr(lib(), name)(*args), name)


def init(device: int = 0) -> None:
    call("omHipInit", device)


def synchronize() -> None:
    call("omHipSynchronize")


def device_count() -> int:
    return int(lib().omHipGetDeviceCount())


def device_name(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    call("omHipGetDeviceName", device, buf, 256)
    return buf.value.decode()


def stream_handle() -> int:
    s = _vp()
    call("omHipGetStream", ctypes.byref(s))
    return s.value or 0


class Graph:
    """A captured sequence of library calls (omHipGraphBeginCapture ... EndCapture), replayed
    on the compute stream. Capture a sequence after one eager run of it."""

    def __init__(self, fn):
        self.handle = None
        call("omHipGraphBeginCapture")
        g = _vp()
        try:
            fn()
        except BaseException:
            # end the recording and drop what was recorded, then report the failure
            if lib().omHipGraphEndCapture(ctypes.byref(g)) == 0 and g.value:
                lib().omHipGraphDestroy(g.value)
            raise
        call("omHipGraphEndCapture", ctypes.byref(g))
        self.handle = g.value

    def launch(self) -> None:
        call("omHipGraphLaunch", self.handle)

    def destroy(self) -> None:
        if getattr(self, "handle", None) and _LIB is not None:
            call("omHipGraphDestroy", self.handle)
        self.handle = None

    def __del__(self):
        if getattr(self, "handle", None) and _LIB is not None:
            lib().omHipGraphDestroy(self.handle)
            self.handle = None


def set_stream(handle: Optional[int]) -> None:
    """Routes later library calls to a caller-owned hipStream_t (None: the library stream)."""
    call("omHipSetStream", handle)


def release_stream(handle: int) -> None:
    """Hands a caller stream's workspace back (call before destroying the stream)."""
    call("omHipReleaseStream", handle)


class ResNet18Infer:
    """Device-resident ResNet-18 classifier and its batch inference pipeline
    (EngineBridge::inferBatch, EngineBridge.cpp:3525-3772, classification branch).
    params: the flat float32 array of omHipResNet18Create's layout."""

    def __init__(self, params: np.ndarray, num_classes: int, max_batch: int = 32):
        params = np.ascontiguousarray(params, np.float32)
        h = _vp()
        call("omHipResNet18Create", params.ctypes.data, params.size, num_classes, max_batch, ctypes.byref(h))
        self.handle, self.nc = h.value, num_classes

    def forward(self, d_input, d_logits, batch: int) -> None:
        call("omHipResNet18Forward", self.handle, d_input.ptr, d_logits.ptr, batch)

    def infer_batch(self, images: np.ndarray, batch_size: int = 32, imagenet_norm: bool = True,
                    conf_threshold: float = 0.0, with_probs: bool = True):
        """images [n, 3, 224, 224] float32 (host) -> (classes int32 [n], confidences [n], probs [n, nc])."""
        images = np.ascontiguousarray(images, np.float32)
        n = images.shape[0]
        cls = np.empty(n, np.int32)
        conf = np.empty(n, np.float32)
        probs = np.empty((n, self.nc), np.float32) if with_probs else None
        call("omHipResNet18InferBatch", self.handle, images.ctypes.data, n, images.shape[1], images.shape[2],
             images.shape[3], batch_size, 1 if imagenet_norm else 0, conf_threshold, cls.ctypes.data,
             conf.ctypes.data, probs.ctypes.data if probs is not None else None)
        return cls, conf, probs

    def __del__(self):
        if getattr(self, "handle", None) and _LIB is not None:
            lib().omHipResNet18Destroy(self.handle)
            self.handle = None


class DeviceBuffer:
    """Device allocation from the library pool (omHipMalloc / omHipFree)."""

    def __init__(self, nbytes: int, dtype=np.float32, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = _vp()
        call("omHipMalloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = int(p.value)

    @classmethod
    def empty(cls, shape, dtype=np.float32) -> "DeviceBuffer":
        shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        n = int(np.prod(shape)) if len(shape) else 1
        return cls(n * np.dtype(dtype).itemsize, dtype, shape)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, a.dtype, a.shape)
        if a.nbytes:
            call("omHipCopyH2D", b.ptr, a.ctypes.data, a.nbytes)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes <= self.nbytes
        if a.nbytes:
            call("omHipCopyH2D", self.ptr, a.ctypes.data, a.nbytes)

    def numpy(self, shape=None, dtype=None) -> np.ndarray:
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        shp = tuple(shape) if shape is not None else self.shape
        out = np.empty(shp, dt)
        if out.nbytes:
            call("omHipCopyD2H", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def free(self) -> None:
        if getattr(self, "ptr", 0) and _LIB is not None:
            _LIB.omHipFree(self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __int__(self) -> int:
        return self.ptr


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    return int(x)


class HIPBackend:
    """The HAL with CPUBackend names and argument order, on device pointers.

    Method signatures follow src/hal/om.hal.cpu_backend.ixx (line numbers in
    each docstring); entries the reference builds by composition (A x B^T,
    fused conv+BN+ReLU, half-precision GEMM) are the extra methods at the end.
    Every pointer argument is a device pointer (int or DeviceBuffer).
    """

    # ---- fills / copy (cpu_backend.ixx:65-77, :444-446) ----
    @staticmethod
    def fillZeros(pData, nCount: int) -> None:
        call("omHipFillZeros", _ptr(pData), nCount)

    @staticmethod
    def fillOnes(pData, nCount: int) -> None:
        call("omHipFillOnes", _ptr(pData), nCount)

    @staticmethod
    def fillValue(pData, nCount: int, fValue: float) -> None:
        call("omHipFillValue", _ptr(pData), nCount, fValue)

    @staticmethod
    def copy(pSrc, pDst, nCount: int) -> None:
        call("omHipCopy", _ptr(pSrc), _ptr(pDst), nCount)

    # ---- GEMM (cpu_backend.ixx:239-286, :1520-1539) ----
    @staticmethod
    def matmul(pA, pB, pC, nM: int, nK: int, nN: int) -> None:
        call("omHipMatmul", _ptr(pA), _ptr(pB), _ptr(pC), nM, nK, nN)

    @staticmethod
    def batchedMatmul(pA, pB, pC, nBatch: int, nM: int, nK: int, nN: int) -> None:
        call("omHipBatchedMatmul", _ptr(pA), _ptr(pB), _ptr(pC), nBatch, nM, nK, nN)

    @staticmethod
    def transpose2d(pA, pB, nRows: int, nCols: int) -> None:
        call("omHipTranspose", _ptr(pA), _ptr(pB), nRows, nCols)

    # ---- reductions (CUDABackend::sum cuda_backend.ixx:732; omCudaMean cuda_kernels.cu:1506) ----
    @staticmethod
    def sum(pData, pResult, nCount: int) -> None:
        """pResult[0] (device) = sum of pData[0..nCount) (tensorSum's GPU branch, tensor_ops.ixx:413-417)."""
        call("omHipSum", _ptr(pData), _ptr(pResult), nCount)

    @staticmethod
    def mean(pData, pResult, nCount: int) -> None:
        call("omHipMean", _ptr(pData), _ptr(pResult), nCount)

    # ---- ViT attention on fp32 data (cuda_backend.ixx:967-985; vit.ixx:163-187) ----
    @staticmethod
    def qkvSplitHeads(pQkv, pQ, pK, pV, nBatch, nSeqLen, nHeads, nHeadDim, fScale) -> None:
        call("omHipQkvSplitHeads", _ptr(pQkv), _ptr(pQ), _ptr(pK), _ptr(pV), nBatch, nSeqLen, nHeads, nHeadDim,
             fScale)

    @staticmethod
    def mergeHeads(pIn, pOut, nBatch, nSeqLen, nHeads, nHeadDim) -> None:
        call("omHipMergeHeads", _ptr(pIn), _ptr(pOut), nBatch, nSeqLen, nHeads, nHeadDim)

    @staticmethod
    def attention(pQKV, pOut, nBatch, nSeq, nHeads, nHeadDim, fScale) -> None:
        """qkvSplitHeads .. mergeHeads of MultiHeadAttention::forward's GPU branch on fp32 data."""
        call("omHipAttention", _ptr(pQKV), _ptr(pOut), nBatch, nSeq, nHeads, nHeadDim, fScale)

    # ---- activations / bias (cpu_backend.ixx:317-346, :433-440) ----
    @staticmethod
    def relu(pIn, pOut, nCount: int) -> None:
        call("omHipReLU", _ptr(pIn), _ptr(pOut), nCount)

    @staticmethod
    def reluBackward(pIn, pGradOut, pGradIn, nCount: int) -> None:
        call("omHipReLUBackward", _ptr(pIn), _ptr(pGradOut), _ptr(pGradIn), nCount)

    @staticmethod
    def addBias(pA, pBias, pOut, nBatch: int, nCols: int) -> None:
        call("omHipAddBias", _ptr(pA), _ptr(pBias), _ptr(pOut), nBatch, nCols, 1)

    @staticmethod
    def addBiasBackward(pGradOut, pGradBias, nN: int, nC: int, nHW: int = 1) -> None:
        """AddBiasBackward's column sum (autograd.ixx:399-433; cuda_backend.ixx:747)."""
        call("omHipAddBiasBackward", _ptr(pGradOut), _ptr(pGradBias), nN, nC, nHW)

    # ---- softmax / cross-entropy (cpu_backend.ixx:352-410) ----
    @staticmethod
    def softmax(pIn, pOut, nBatch: int, nClasses: int) -> None:
        call("omHipSoftmax", _ptr(pIn), _ptr(pOut), nBatch, nClasses)

    @staticmethod
    def crossEntropyForward(pSoftmax, pTarget, pResult, nBatch: int, nClasses: int) -> None:
        """CUDABackend::crossEntropyForward (cuda_backend.ixx:823) with CPUBackend::crossEntropy's
        rule (cpu_backend.ixx:375-388): the loss is written to the device scalar pResult."""
        call("omHipCrossEntropy", _ptr(pSoftmax), _ptr(pTarget), _ptr(pResult), nBatch, nClasses)

    @staticmethod
    def crossEntropySoftmaxBackward(pSoftmax, pTarget, pGradInput, nBatch: int, nClasses: int) -> None:
        call("omHipSoftmaxCrossEntropyBackward", _ptr(pSoftmax), _ptr(pTarget), _ptr(pGradInput), nBatch, nClasses)

    @staticmethod
    def softmaxCrossEntropy(pLogits, pTarget, pSoftmax, pLoss, pGradLogits, nBatch: int, nClasses: int) -> None:
        """softmax -> crossEntropy -> crossEntropySoftmaxBackward in one launch (any output may be None)."""
        call("omHipSoftmaxCrossEntropy", _ptr(pLogits), _ptr(pTarget), _ptr(pSoftmax), _ptr(pLoss),
             _ptr(pGradLogits), nBatch, nClasses)

    # ---- conv / BN (cpu_backend.ixx:544-575, :619-658, :781-842) ----
    @staticmethod
    def im2col(pInput, nCin, nH, nW, nKH, nKW, nPadH, nPadW, nStrideH, nStrideW, pCol) -> None:
        call("omHipIm2col", _ptr(pInput), nCin, nH, nW, nKH, nKW, nPadH, nPadW, nStrideH, nStrideW, _ptr(pCol))

    @staticmethod
    def conv2d(pInput, pWeight, pBias, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad) -> None:
        call("omHipConv2d", _ptr(pInput), _ptr(pWeight), _ptr(pBias), _ptr(pOutput),
             nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad)

    @staticmethod
    def batchNorm2d(pInput, pOutput, pGamma, pBeta, pRunMean, pRunVar, pSavedMean, pSavedInvStd,
                    nBatch, nChannels, nH, nW, fEps, fMomentum, bTraining) -> None:
        call("omHipBatchNorm2d", _ptr(pInput), _ptr(pOutput), _ptr(pGamma), _ptr(pBeta), _ptr(pRunMean),
             _ptr(pRunVar), _ptr(pSavedMean), _ptr(pSavedInvStd), nBatch, nChannels, nH, nW, fEps, fMomentum,
             1 if bTraining else 0)

    @staticmethod
    def conv2dBackwardInput(pGradOutput, pWeight, pGradInput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride,
                            nPad) -> None:
        """CPUBackend::conv2dBackwardInput (cpu_backend.ixx:666-705)."""
        call("omHipConv2dBackwardInput", _ptr(pGradOutput), _ptr(pWeight), _ptr(pGradInput), nBatch, nCin, nH, nW,
             nCout, nKH, nKW, nStride, nPad)

    @staticmethod
    def conv2dBackwardWeight(pInput, pGradOutput, pGradWeight, pGradBias, nBatch, nCin, nH, nW, nCout, nKH, nKW,
                             nStride, nPad) -> None:
        """CPUBackend::conv2dBackwardWeight (cpu_backend.ixx:710-772); pGradBias may be None."""
        call("omHipConv2dBackwardWeight", _ptr(pInput), _ptr(pGradOutput), _ptr(pGradWeight), _ptr(pGradBias),
             nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad)

    @staticmethod
    def batchNorm2dBackward(pGradOutput, pInput, pSavedMean, pSavedInvStd, pGamma, pGradInput, pGradGamma,
                            pGradBeta, nBatch, nChannels, nH, nW, fEps: float = 1e-5) -> None:
        """CPUBackend::batchNorm2dBackward (cpu_backend.ixx:847-890)."""
        call("omHipBatchNorm2dBackward", _ptr(pGradOutput), _ptr(pInput), _ptr(pSavedMean), _ptr(pSavedInvStd),
             _ptr(pGamma), _ptr(pGradInput), _ptr(pGradGamma), _ptr(pGradBeta), nBatch, nChannels, nH, nW, fEps)

    @staticmethod
    def batchNorm2dBackwardRelu(pGradOutput, pReluInput, pInput, pSavedMean, pSavedInvStd, pGamma, pGradInput,
                                pGradGamma, pGradBeta, nBatch, nChannels, nH, nW, fEps: float = 1e-5) -> None:
        """batchNorm2dBackward of reluBackward(pReluInput, pGradOutput), one pass, bit-identical."""
        call("omHipBatchNorm2dBackwardRelu", _ptr(pGradOutput), _ptr(pReluInput), _ptr(pInput), _ptr(pSavedMean),
             _ptr(pSavedInvStd), _ptr(pGamma), _ptr(pGradInput), _ptr(pGradGamma), _ptr(pGradBeta), nBatch,
             nChannels, nH, nW, fEps)

    @staticmethod
    def batchNorm2dTrainAct(pInput, pOutput, pGamma, pBeta, pRunningMean, pRunningVar, pSavedMean, pSavedInvStd,
                            nBatch, nChannels, nH, nW, fEps, fMomentum, pResidual, nAct) -> None:
        """act(batchNorm2d(training) [+ residual]) in one pass, bit-identical to the separate calls."""
        call("omHipBatchNorm2dTrainAct", _ptr(pInput), _ptr(pOutput), _ptr(pGamma), _ptr(pBeta), _ptr(pRunningMean),
             _ptr(pRunningVar), _ptr(pSavedMean), _ptr(pSavedInvStd), nBatch, nChannels, nH, nW, fEps, fMomentum,
             _ptr(pResidual), nAct)

    @staticmethod
    def maxPool2d(pInput, pOutput, pIndices, nBatch, nChannels, nH, nW, nKH, nKW, nStride, nPad) -> None:
        """CPUBackend::maxPool2d (cpu_backend.ixx:897-934); pIndices (int32) may be None."""
        call("omHipMaxPool2d", _ptr(pInput), _ptr(pOutput), _ptr(pIndices), nBatch, nChannels, nH, nW, nKH, nKW,
             nStride, nStride, nPad, nPad)

    @staticmethod
    def maxPool2dBackward(pGradOutput, pIndices, pGradInput, nBatch, nChannels, nHout, nWout, nH, nW) -> None:
        """CPUBackend::maxPool2dBackward (cpu_backend.ixx:937-955): scatter through the indices."""
        call("omHipMaxPool2dBackward", _ptr(pGradOutput), _ptr(pIndices), _ptr(pGradInput), nBatch, nChannels, nH,
             nW, nHout, nWout)

    @staticmethod
    def maxPool2dBackwardEx(pGradOutput, pIndices, pGradInput, nBatch, nChannels, nH, nW, nKH, nKW, nStride,
                            nPad) -> None:
        """Ordered gather form of maxPool2dBackward (bit-identical to the reference)."""
        call("omHipMaxPool2dBackwardEx", _ptr(pGradOutput), _ptr(pIndices), _ptr(pGradInput), nBatch, nChannels, nH,
             nW, nKH, nKW, nStride, nStride, nPad, nPad)

    @staticmethod
    def avgPool2d(pInput, pOutput, nBatch, nChannels, nH, nW, nKH, nKW, nStride, nPad) -> None:
        """CPUBackend::avgPool2d (cpu_backend.ixx:958-990)."""
        call("omHipAvgPool2d", _ptr(pInput), _ptr(pOutput), nBatch, nChannels, nH, nW, nKH, nKW, nStride, nStride,
             nPad, nPad)

    @staticmethod
    def avgPool2dBackward(pGradOutput, pGradInput, nBatch, nChannels, nH, nW, nHout, nWout, nKH, nKW, nStride,
                          nPad) -> None:
        """CPUBackend::avgPool2dBackward (cpu_backend.ixx:994-1023)."""
        call("omHipAvgPool2dBackward", _ptr(pGradOutput), _ptr(pGradInput), nBatch, nChannels, nH, nW, nKH, nKW,
             nStride, nStride, nPad, nPad)

    @staticmethod
    def adaptiveAvgPool2d(pInput, pOutput, nBatch, nChannels, nH, nW, nOutH, nOutW) -> None:
        """CPUBackend::adaptiveAvgPool2d (cpu_backend.ixx:1467-1488)."""
        call("omHipAdaptiveAvgPool2d", _ptr(pInput), _ptr(pOutput), nBatch, nChannels, nH, nW, nOutH, nOutW)

    @staticmethod
    def adaptiveAvgPool2dBackward(pGradOutput, pGradInput, nBatch, nChannels, nH, nW, nOutH, nOutW) -> None:
        """CPUBackend::adaptiveAvgPool2dBackward (cpu_backend.ixx:1491-1510)."""
        call("omHipAdaptiveAvgPool2dBackward", _ptr(pGradOutput), _ptr(pGradInput), nBatch, nChannels, nH, nW, nOutH,
             nOutW)

    @staticmethod
    def add(pA, pB, pOut, nCount) -> None:
        """CPUBackend::add (cpu_backend.ixx:147-160)."""
        call("omHipAdd", _ptr(pA), _ptr(pB), _ptr(pOut), nCount)

    @staticmethod
    def addReluBackward(pA, pInput, pGradOutput, pOut, nCount) -> None:
        """add(pA, reluBackward(pInput, pGradOutput)) in one pass, bit-identical."""
        call("omHipAddReluBackward", _ptr(pA), _ptr(pInput), _ptr(pGradOutput), _ptr(pOut), nCount)

    @staticmethod
    def conv2dBiasBnAddAct(pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, pResidual, nAct, pOutput,
                           nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad) -> None:
        """conv2d -> batchNorm2d(eval) -> add(shortcut) -> relu in one kernel (resnet.ixx:55-79)."""
        call("omHipConv2dBiasBnAddAct", _ptr(pInput), _ptr(pWeight), _ptr(pBias), _ptr(pGamma), _ptr(pBeta),
             _ptr(pMean), _ptr(pVar), fEps, _ptr(pResidual), nAct, _ptr(pOutput), nBatch, nCin, nH, nW, nCout, nKH,
             nKW, nStride, nPad)

    @staticmethod
    def attentionHalf(pQKV, pOut, nBatch, nSeq, nHeads, nHeadDim, fScale, bf16: bool = False,
                      outHalf: bool = False) -> None:
        """Fused QKV split + softmax(scale Q K^T) V + head merge (vit.ixx:150-239)."""
        call("omHipAttentionHalf", 1 if bf16 else 0, _ptr(pQKV), _ptr(pOut), 1 if outHalf else 0, nBatch, nSeq, nHeads,
             nHeadDim, fScale)

    @staticmethod
    def linearHalf(pInput, pWeight, pBias, pOutput, nM, nK, nN, bf16: bool = False, transW: bool = False,
                   act: int = 0, outHalf: bool = False) -> None:
        """Linear::forward (linear.ixx:50-58) on half inputs: act(x W + b), W [K,N] (or [N,K])."""
        call("omHipLinearHalf", 1 if bf16 else 0, _ptr(pInput), _ptr(pWeight), 1 if transW else 0, _ptr(pBias), act,
             _ptr(pOutput), 1 if outHalf else 0, nM, nK, nN)

    @staticmethod
    def multiHeadAttentionHalf(pX, pWqkv, pBqkv, pWout, pBout, pOut, nBatch, nSeq, nHeads, nHeadDim,
                               bf16: bool = False, outHalf: bool = False) -> None:
        """MultiHeadAttention::forward (vit.ixx:150-239): QKV Linear, attention, output Linear."""
        call("omHipMultiHeadAttentionHalf", 1 if bf16 else 0, _ptr(pX), _ptr(pWqkv), _ptr(pBqkv), _ptr(pWout),
             _ptr(pBout), _ptr(pOut), 1 if outHalf else 0, nBatch, nSeq, nHeads, nHeadDim)

    # ---- entries the reference builds by composition ----
    @staticmethod
    def matmulTransB(pA, pB, pC, nM: int, nK: int, nN: int) -> None:
        """C = A[M,K] x B[N,K]^T (reference: transpose2d + matmul, autograd.ixx:261-273)."""
        call("omHipMatmulTransB", _ptr(pA), _ptr(pB), _ptr(pC), nM, nK, nN)

    @staticmethod
    def matmulTransA(pA, pB, pC, nM: int, nK: int, nN: int) -> None:
        """C = A[K,M]^T x B[K,N] (reference: transpose2d + matmul, autograd.ixx:276-286)."""
        call("omHipMatmulTransA", _ptr(pA), _ptr(pB), _ptr(pC), nM, nK, nN)

    @staticmethod
    def linearBiasAct(pA, pW, pBias, pOut, nM: int, nK: int, nN: int, nAct: int) -> None:
        """act(A[M,K] * W[K,N] + bias[N]) in one pass (bias may be None; nAct 0 / 1 = ReLU)."""
        call("omHipLinearBiasAct", _ptr(pA), _ptr(pW), _ptr(pBias), _ptr(pOut), nM, nK, nN, nAct)

    @staticmethod
    def linearBackward(pInput, pGradOut, pWeight, pGate, pGradWeight, pGradBias, pGradInput, nBatch: int, nIn: int,
                       nOut: int) -> None:
        """A Linear layer's backward in one launch (MatMulBackward autograd.ixx:261-286, AddBiasBackward
        :399-433, and the ReLU backward below it when pGate is given): dW = X^T G, db = column sums of
        G, dX = G W^T (kept where pGate > 0)."""
        call("omHipLinearBackward", _ptr(pInput), _ptr(pGradOut), _ptr(pWeight), _ptr(pGate), _ptr(pGradWeight),
             _ptr(pGradBias), _ptr(pGradInput), nBatch, nIn, nOut)

    @staticmethod
    def linearSoftmaxCrossEntropyStep(pInput, pWeight, pBias, pTarget, pGate, pLogits, pLoss, pGradLogits,
                                      pGradWeight, pGradBias, pGradInput, nBatch: int, nIn: int,
                                      nClasses: int) -> None:
        """The classifier head of a training step in one launch: logits = X W + b, softmax cross-entropy
        (loss and g = (p - T) / nBatch), gW = X^T g, gb = column sums of g, gX = g W^T kept where
        pGate > 0 (linear.ixx:50-58, tensor_ops.ixx:583-633, autograd.ixx:261-286, :399-488)."""
        call("omHipLinearSoftmaxCrossEntropyStep", _ptr(pInput), _ptr(pWeight), _ptr(pBias), _ptr(pTarget),
             _ptr(pGate), _ptr(pLogits), _ptr(pLoss), _ptr(pGradLogits), _ptr(pGradWeight), _ptr(pGradBias),
             _ptr(pGradInput), nBatch, nIn, nClasses)

    @staticmethod
    def batchedMatmulTransB(pA, pB, pC, nBatch: int, nM: int, nK: int, nN: int) -> None:
        call("omHipBatchedMatmulTransB", _ptr(pA), _ptr(pB), _ptr(pC), nBatch, nM, nK, nN)

    @staticmethod
    def conv2dIm2col(pInput, pWeight, pBias, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad) -> None:
        call("omHipConv2dIm2col", _ptr(pInput), _ptr(pWeight), _ptr(pBias), _ptr(pOutput),
             nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad)

    @staticmethod
    def conv2dBiasBnAct(pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, nAct, pOutput,
                        nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad) -> None:
        """conv2d -> batchNorm2d(eval) -> relu in one kernel (tensor_ops.ixx:672-833, :511-536)."""
        call("omHipConv2dBiasBnAct", _ptr(pInput), _ptr(pWeight), _ptr(pBias), _ptr(pGamma), _ptr(pBeta),
             _ptr(pMean), _ptr(pVar), fEps, nAct, _ptr(pOutput), nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad)

    @staticmethod
    def gemmStridedBatched(bTransA, bTransB, nBatch, nM, nN, nK, pA, nLda, nStrideA, pB, nLdb, nStrideB,
                           pC, nLdc, nStrideC) -> None:
        call("omHipGemmStridedBatched", int(bTransA), int(bTransB), nBatch, nM, nN, nK, _ptr(pA), nLda, nStrideA,
             _ptr(pB), nLdb, nStrideB, _ptr(pC), nLdc, nStrideC)

    @staticmethod
    def convertToHalf(pIn, pOut, nCount: int, bf16: bool = False) -> None:
        call("omHipConvertF32ToBF16" if bf16 else "omHipConvertF32ToF16", _ptr(pIn), _ptr(pOut), nCount)

    @staticmethod
    def convertFromHalf(pIn, pOut, nCount: int, bf16: bool = False) -> None:
        call("omHipConvertBF16ToF32" if bf16 else "omHipConvertF16ToF32", _ptr(pIn), _ptr(pOut), nCount)

    @staticmethod
    def matmulHalf(pA, pB, pC, nM: int, nK: int, nN: int, bf16: bool = False, transB: bool = False) -> None:
        name = {(False, False): "omHipMatmulF16", (True, False): "omHipMatmulBF16",
                (False, True): "omHipMatmulTransBF16", (True, True): "omHipMatmulTransBBF16"}[(bf16, transB)]
        call(name, _ptr(pA), _ptr(pB), _ptr(pC), nM, nK, nN)

    @staticmethod
    def gemmStridedBatchedHalf(nDtype, bTransA, bTransB, nBatch, nM, nN, nK, pA, nLda, nStrideA, pB, nLdb,
                               nStrideB, pC, nLdc, nStrideC) -> None:
        call("omHipGemmStridedBatchedHalf", nDtype, int(bTransA), int(bTransB), nBatch, nM, nN, nK, _ptr(pA), nLda,
             nStrideA, _ptr(pB), nLdb, nStrideB, _ptr(pC), nLdc, nStrideC)
