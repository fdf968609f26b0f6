"""Workspace safety across caller streams and captured graphs.

The split-K GEMM / conv paths keep partial sums in a library workspace. These
tests hold the library to three rules: each stream has its own workspace (two
caller streams alternating split-K work give the same bits as one stream), an
outgrown workspace stays allocated while a captured graph may still use it
(a replay after growth neither reads nor writes memory the pool handed to the
caller), and a capture that would need a new workspace or lookup table fails
with a message instead of recording a stale address.

Bars: results are compared bit for bit with the same op run alone on the
library stream (split sums are added in a fixed order), and that run against
the oracle with the 1e-4 K-scaled bar.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


class _Streams:
    """Caller-owned HIP streams (hipStreamCreateWithFlags, non-blocking, default priority)."""

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

    def sync(self, s: int) -> None:
        assert self.rt.hipStreamSynchronize(ctypes.c_void_p(s)) == 0

    def destroy_all(self, om) -> None:
        for s in self.made:
            om.release_stream(s)          # its workspace goes back before the handle can be reused
            self.rt.hipStreamDestroy(ctypes.c_void_p(s))
        self.made = []


@pytest.fixture
def streams(hip):
    st = _Streams()
    yield st
    hip.set_stream(None)
    st.destroy_all(hip)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _bn(C, seed):
    return [O.uniform((C,), seed, 0.5, 1.5), O.randn((C,), seed + 1, 0.1), O.randn((C,), seed + 2, 0.1),
            O.uniform((C,), seed + 3, 0.5, 1.5)]


def test_two_caller_streams_split_k(hip, streams):
    """Split-K GEMMs (128x4096x4096: 8 K slices) and split-K convs (2x256x14x14 -> 512, 3x3 s2:
    16 output tiles) alternate between two caller streams with no host wait in between; every
    output must equal the single-stream result bit for bit."""
    H = hip.HIPBackend
    M, K, N = 128, 4096, 4096
    A = [O.randn((M, K), 11 + i) for i in range(2)]
    B = [O.randn((K, N), 21 + i) for i in range(2)]
    x = [O.randn((2, 256, 14, 14), 31 + i) for i in range(2)]
    w = O.uniform((512, 256, 3, 3), 41, -0.03, 0.03)
    bn = _bn(512, 50)
    dA, dB, dx = [to_dev(hip, a) for a in A], [to_dev(hip, b) for b in B], [to_dev(hip, a) for a in x]
    dw, dbn = to_dev(hip, w), [to_dev(hip, a) for a in bn]
    dC = [empty_dev(hip, (M, N)) for _ in range(2)]
    dy = [empty_dev(hip, (2, 512, 7, 7)) for _ in range(2)]

    def gemm(i):
        H.matmul(dA[i], dB[i], dC[i], M, K, N)

    def conv(i):
        H.conv2dBiasBnAct(dx[i], dw, None, *dbn, 1e-5, 1, dy[i], 2, 256, 14, 14, 512, 3, 3, 2, 1)

    ref_C, ref_y = [], []
    for i in range(2):                      # each op alone on the library stream
        gemm(i)
        conv(i)
        ref_C.append(dC[i].numpy().copy())
        ref_y.append(dy[i].numpy().copy())
    C64, bound = O.gemm_f64(A[0], B[0])
    assert O.normalized_error(ref_C[0], C64, bound) <= O.TOL_FP32
    y64, yb = O.conv_f64(x[1], w, None, 2, 1, *bn, act=1)
    assert O.normalized_error(ref_y[1], y64, yb) <= O.TOL_FP32

    for i in range(2):
        H.fillValue(dC[i], M * N, 5.0)
        H.fillValue(dy[i], 2 * 512 * 49, 5.0)
    hip.synchronize()
    sA, sB = streams.create(), streams.create()
    print(f"[streams] alternating split-K work on streams {sA:#x} / {sB:#x}", flush=True)
    for _ in range(3):
        hip.set_stream(sA); gemm(0)
        hip.set_stream(sB); gemm(1)
        hip.set_stream(sA); conv(0)
        hip.set_stream(sB); conv(1)
    streams.sync(sA)
    streams.sync(sB)
    hip.set_stream(None)
    for i in range(2):
        assert np.array_equal(_bits(dC[i].numpy()), _bits(ref_C[i])), f"gemm on stream {i}"
        assert np.array_equal(_bits(dy[i].numpy()), _bits(ref_y[i])), f"conv on stream {i}"


def test_graph_replay_after_workspace_growth(hip):
    """A graph captured with the 2 MiB workspace of a small split-K GEMM (64x1024x2048) is
    replayed after a larger split-K GEMM (128x4096x4096, 16 MiB) grew the stream's workspace
    and after the caller allocated a buffer of the old workspace's size: the replay must give
    the eager result and leave that buffer untouched."""
    H = hip.HIPBackend
    m, k, n = 64, 2048, 1024
    a, b = to_dev(hip, O.randn((m, k), 61)), to_dev(hip, O.randn((k, n), 62))
    c = empty_dev(hip, (m, n))
    c_ref = empty_dev(hip, (m, n))
    H.matmul(a, b, c, m, k, n)                      # eager run first: workspace and plan exist
    graph = hip.Graph(lambda: H.matmul(a, b, c, m, k, n))
    try:
        M, K, N = 128, 4096, 4096
        A, B = to_dev(hip, O.randn((M, K), 63)), to_dev(hip, O.randn((K, N), 64))
        C = empty_dev(hip, (M, N))
        H.matmul(A, B, C, M, K, N)                  # grows the workspace 2 -> 16 MiB
        other = empty_dev(hip, ((2 << 20) // 4,))   # the old workspace's size
        H.fillValue(other, (2 << 20) // 4, 3.0)
        a_new, b_new = O.randn((m, k), 65), O.randn((k, n), 66)
        a.upload(a_new)
        b.upload(b_new)
        H.matmul(a, b, c_ref, m, k, n)              # eager result on the new inputs
        H.fillValue(c, m * n, 9.0)
        for r in range(2):
            graph.launch()
            hip.synchronize()
            assert np.array_equal(_bits(c.numpy()), _bits(c_ref.numpy())), r
            assert np.all(other.numpy() == np.float32(3.0)), r
        c64, bound = O.gemm_f64(a_new, b_new)
        assert O.normalized_error(c.numpy(), c64, bound) <= O.TOL_FP32
    finally:
        graph.destroy()


def test_capture_refuses_new_workspace_and_tables(hip, streams):
    """On a fresh caller stream, capturing a split-K GEMM before any eager run (no workspace
    yet) and a conv of a geometry never run before (no tap table yet) both fail with a
    message; after one eager run the same captures record and replay correctly."""
    H = hip.HIPBackend
    m, k, n = 64, 2048, 1024
    a, b = to_dev(hip, O.randn((m, k), 71)), to_dev(hip, O.randn((k, n), 72))
    c, c_ref = empty_dev(hip, (m, n)), empty_dev(hip, (m, n))
    x = to_dev(hip, O.randn((2, 7, 11, 11), 73))
    w = to_dev(hip, O.randn((5, 7, 3, 3), 74, 0.2))
    y, y_ref = empty_dev(hip, (2, 5, 11, 11)), empty_dev(hip, (2, 5, 11, 11))
    s = streams.create()
    hip.set_stream(s)
    with pytest.raises(hip.OmHipError, match="records a graph"):
        hip.Graph(lambda: H.matmul(a, b, c, m, k, n))
    with pytest.raises(hip.OmHipError, match="records a graph"):
        hip.Graph(lambda: H.conv2d(x, w, None, y, 2, 7, 11, 11, 5, 3, 3, 1, 1))
    H.matmul(a, b, c_ref, m, k, n)
    H.conv2d(x, w, None, y_ref, 2, 7, 11, 11, 5, 3, 3, 1, 1)
    g1 = hip.Graph(lambda: H.matmul(a, b, c, m, k, n))
    g2 = hip.Graph(lambda: H.conv2d(x, w, None, y, 2, 7, 11, 11, 5, 3, 3, 1, 1))
    try:
        g1.launch()
        g2.launch()
        streams.sync(s)
        assert np.array_equal(_bits(c.numpy()), _bits(c_ref.numpy()))
        assert np.array_equal(_bits(y.numpy()), _bits(y_ref.numpy()))
    finally:
        g1.destroy()
        g2.destroy()


def test_free_on_one_stream_reuse_on_another(hip, streams):
    """A buffer freed on stream A while A's GEMM still reads it must not be handed to stream B:
    B's first split-K GEMM (128x4096x4096, 8 MiB of partials: a fresh workspace block of the
    freed buffer's size) runs right after the free with no host wait. A's product must equal
    the single-stream result bit for bit, and so must B's."""
    H = hip.HIPBackend
    M, K, N = 512, 4096, 4096                        # A operand: 8 MiB, read by a 17 GFLOP product
    A_np, B_np = O.randn((M, K), 81), O.randn((K, N), 82)
    m, k, n = 128, 4096, 4096
    a_np, b_np = O.randn((m, k), 83), O.randn((k, n), 84)
    dB, db = to_dev(hip, B_np), to_dev(hip, b_np)
    da = to_dev(hip, a_np)
    C, C_ref = empty_dev(hip, (M, N)), empty_dev(hip, (M, N))
    c, c_ref = empty_dev(hip, (m, n)), empty_dev(hip, (m, n))
    dA_ref = to_dev(hip, A_np)
    H.matmul(dA_ref, dB, C_ref, M, K, N)             # references on the library stream
    H.matmul(da, db, c_ref, m, k, n)
    hip.synchronize()
    sA, sB = streams.create(), streams.create()
    print(f"[streams] free on {sA:#x}, reuse on {sB:#x}", flush=True)
    for r in range(3):
        dA = to_dev(hip, A_np)                       # uploaded and synchronised on the library stream
        hip.set_stream(sA)
        H.matmul(dA, dB, C, M, K, N)
        dA.free()                                    # ordered on A: A's GEMM may still be reading it
        hip.set_stream(sB)
        H.matmul(da, db, c, m, k, n)                 # split-K on B: a workspace of dA's size
        streams.sync(sA)
        streams.sync(sB)
        hip.set_stream(None)
        assert np.array_equal(_bits(C.numpy()), _bits(C_ref.numpy())), r
        assert np.array_equal(_bits(c.numpy()), _bits(c_ref.numpy())), r
        hip.release_stream(sB)                       # B's workspace goes back: the next round grows it again


def test_release_stream_refused_while_graph_lives(hip, streams):
    """omHipReleaseStream fails while a graph captured on that stream exists, and succeeds once
    the graph is destroyed; the graph replays correctly meanwhile."""
    H = hip.HIPBackend
    m, k, n = 64, 2048, 1024
    a, b = to_dev(hip, O.randn((m, k), 91)), to_dev(hip, O.randn((k, n), 92))
    c, c_ref = empty_dev(hip, (m, n)), empty_dev(hip, (m, n))
    s = streams.create()
    hip.set_stream(s)
    H.matmul(a, b, c_ref, m, k, n)
    g = hip.Graph(lambda: H.matmul(a, b, c, m, k, n))
    try:
        hip.set_stream(None)
        with pytest.raises(hip.OmHipError, match="graph"):
            hip.release_stream(s)
        g.launch()
        streams.sync(s)
        assert np.array_equal(_bits(c.numpy()), _bits(c_ref.numpy()))
    finally:
        g.destroy()
    hip.release_stream(s)
