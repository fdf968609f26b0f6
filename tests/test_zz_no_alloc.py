"""omHipGemmStridedBatchedNoAlloc: omHipGemmStridedBatched with its split-K partial sums in
a fixed device array instead of an allocated workspace.

Called through the C ABI, its output must equal omHipGemmStridedBatched's bit for bit (the
same plan and the same fixed summation order), including on consecutive calls whose second
is smaller than the first (the array still holds the first call's partials), and must be
within the 1e-4 K-scaled bar of the float64 product. The library's pool must hold and hand
out the same bytes before and after (the entry allocates nothing).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu

# (transA, transB, batch, M, N, K): pairs of calls in a row, the second smaller. Partials
# are whole 64x64 tiles (16 KiB each per split). On a 256-CU device 128x4096x4096 splits K
# 4 ways (128 tiles: 8 MiB of partials), 64x1024x2048 8 ways (16 tiles: 2 MiB), and
# 448x4672x2048 (511 tiles) 2 ways: 16.7 MB, the largest plan any shape reaches there (the
# bound a CPU test checks over a grid of shapes).
PAIRS = [
    ((0, 0, 1, 448, 4672, 2048), (0, 0, 1, 128, 4096, 4096)),
    ((0, 0, 1, 128, 4096, 4096), (0, 0, 1, 64, 1024, 2048)),
    ((0, 1, 1, 128, 4096, 4096), (0, 1, 2, 64, 256, 2048)),
    ((1, 0, 3, 128, 512, 4096), (1, 1, 1, 96, 200, 1536)),
    ((0, 0, 1, 512, 512, 512), (0, 0, 1, 37, 29, 53)),          # no split: the scratch is unused
]


def _pool(om):
    held, used = ctypes.c_size_t(), ctypes.c_size_t()
    om.call("omHipPoolStats", ctypes.byref(held), ctypes.byref(used))
    return held.value, used.value


def _operands(case, seed):
    ta, tb, b, M, N, K = case
    A = O.randn((b, K, M) if ta else (b, M, K), seed)
    B = O.randn((b, N, K) if tb else (b, K, N), seed + 1)
    return A, B


def _call(om, entry, case, dA, dB, dC):
    ta, tb, b, M, N, K = case
    lda, ldb = (M if ta else K), (K if tb else N)
    om.call(entry, ta, tb, b, M, N, K, dA.ptr, lda, M * K, dB.ptr, ldb, K * N, dC.ptr, N, M * N)


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: "{}-then-{}".format(*["x".join(map(str, c)) for c in p]))
def test_no_alloc_matches_allocating_entry(hip, pair):
    bufs = []
    for i, case in enumerate(pair):
        A, B = _operands(case, 50 + 10 * i + case[3])
        ta, tb, b, M, N, K = case
        bufs.append((case, A, B, to_dev(hip, A), to_dev(hip, B), empty_dev(hip, (b, M, N)),
                     empty_dev(hip, (b, M, N))))
    hip.synchronize()
    before = _pool(hip)
    for case, A, B, dA, dB, dC, _ in bufs:              # two no-allocation calls in a row
        print(f"case no-alloc {case}", flush=True)
        _call(hip, "omHipGemmStridedBatchedNoAlloc", case, dA, dB, dC)
    hip.synchronize()
    assert _pool(hip) == before
    for case, A, B, dA, dB, dC, dRef in bufs:
        _call(hip, "omHipGemmStridedBatched", case, dA, dB, dRef)
        got, want = dC.numpy(), dRef.numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case
        ta, tb, b, M, N, K = case
        for i in range(b):
            C64, bound = O.gemm_f64(A[i], B[i], transA=bool(ta), transB=bool(tb))
            assert O.normalized_error(got[i], C64, bound) <= O.TOL_FP32, case


def test_no_alloc_degenerate(hip):
    """K = 0 zeroes C (cpu_backend.ixx:246-251) without touching the scratch; M = 0 writes nothing."""
    dC = to_dev(hip, np.full((1, 4, 5), 7.0, np.float32))
    hip.call("omHipGemmStridedBatchedNoAlloc", 0, 0, 1, 4, 5, 0, None, 1, 0, None, 5, 0, dC.ptr, 5, 20)
    assert np.all(dC.numpy() == 0.0)
    dC.upload(np.full((1, 4, 5), 7.0, np.float32))
    hip.call("omHipGemmStridedBatchedNoAlloc", 0, 0, 1, 0, 5, 3, None, 3, 0, None, 5, 0, dC.ptr, 5, 20)
    assert np.all(dC.numpy() == 7.0)
    with pytest.raises(hip.OmHipError, match="leading dimension"):
        A, B = to_dev(hip, np.ones((4, 3), np.float32)), to_dev(hip, np.ones((3, 5), np.float32))
        hip.call("omHipGemmStridedBatchedNoAlloc", 0, 0, 1, 4, 5, 3, A.ptr, 2, 12, B.ptr, 5, 15, dC.ptr, 5, 20)


class _Streams:
    """Two caller-owned HIP streams (non-blocking, default priority)."""

    def __init__(self):
        path = "libamdhip64.so"
        for d in ("/opt/rocm/lib", "/opt/rocm/lib64"):
            if os.path.exists(os.path.join(d, path)):
                path = os.path.join(d, path)
                break
        self.rt = ctypes.CDLL(path)
        self.made = []

    def create(self) -> int:
        s = ctypes.c_void_p()
        assert self.rt.hipStreamCreateWithFlags(ctypes.byref(s), ctypes.c_uint(1)) == 0
        self.made.append(s.value)
        return s.value

    def destroy_all(self, om) -> None:
        for s in self.made:
            om.release_stream(s)
            self.rt.hipStreamDestroy(ctypes.c_void_p(s))
        self.made = []


def test_no_alloc_two_streams_ordered(hip):
    """Split-K no-allocation calls alternate between two caller streams with no host wait: the
    calls share one fixed array, so each must be ordered after the previous one (an event wait
    on the device). Every output must equal the allocating entry's on the library stream, bit
    for bit."""
    cases = [(0, 0, 1, 128, 4096, 4096), (0, 1, 1, 128, 4096, 4096), (0, 0, 1, 64, 1024, 2048),
             (1, 0, 2, 128, 512, 4096)]
    data = []
    for i, case in enumerate(cases):
        A, B = _operands(case, 300 + 7 * i)
        ta, tb, b, M, N, K = case
        data.append((case, to_dev(hip, A), to_dev(hip, B), empty_dev(hip, (b, M, N)), empty_dev(hip, (b, M, N))))
    for case, dA, dB, _, dRef in data:
        _call(hip, "omHipGemmStridedBatched", case, dA, dB, dRef)
    hip.synchronize()
    st = _Streams()
    try:
        s = [st.create(), st.create()]
        for rep in range(3):
            for i, (case, dA, dB, dC, _) in enumerate(data):
                hip.set_stream(s[(i + rep) % 2])
                print(f"case no-alloc stream {(i + rep) % 2} {case}", flush=True)
                _call(hip, "omHipGemmStridedBatchedNoAlloc", case, dA, dB, dC)
            for x in s:
                assert st.rt.hipStreamSynchronize(ctypes.c_void_p(x)) == 0
            hip.set_stream(None)
            for case, _, _, dC, dRef in data:
                assert np.array_equal(_bits(dC.numpy()), _bits(dRef.numpy())), (rep, case)
    finally:
        hip.set_stream(None)
        st.destroy_all(hip)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)
