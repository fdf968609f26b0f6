"""fp16 / bf16 GEMM (fp32 accumulate) parity.

Two bars, both K-scaled (|C - C_ref| <= tol * sum_k |a_ik||b_kj|):
  * against the oracle CPUBackend matmul on the SAME rounded inputs
    (halfToFloat(A), halfToFloat(B), matmul): tol 1e-4 (only accumulation
    order differs: every fp16/bf16 product is exact in fp32);
  * against CPUBackend on the ORIGINAL fp32 inputs: tol 1e-2.
Inputs are rounded to nearest-even (the reference's own FP16Converter
truncates, fp16.ixx:92; the rounding rule is stated, not reproduced).
Shapes: the ViT-B/16 projections (tokens 12608 = 64 x 197) on a token subset,
and batched attention Q.K^T / P.V at the ragged 197.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def _round(x, bf16):
    return O.bf16_round(x) if bf16 else x.astype(np.float16).astype(np.float32)


def _bits(x, bf16):
    return O.bf16_bits(x) if bf16 else x.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("transB", [False, True], ids=["NN", "NT"])
@pytest.mark.parametrize("M,K,N", [(2, 3, 4), (197, 768, 2304), (394, 768, 768), (256, 768, 3072), (256, 3072, 768),
                                   (33, 40, 17), (512, 512, 512), (1024, 1024, 1024)])
def test_matmul_half(hip, bf16, transB, M, K, N):
    A = O.randn((M, K), M + K)
    B = O.randn((N, K) if transB else (K, N), N + 1, 0.02 if K >= 768 else 1.0)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dC = empty_dev(hip, (M, N))
    hip.HIPBackend.matmulHalf(dA, dB, dC, M, K, N, bf16=bf16, transB=transB)
    C = dC.numpy()
    Ar, Br = _round(A, bf16), _round(B, bf16)
    ref_rounded = O.matmul_transB(Ar, Br) if transB else O.matmul(Ar, Br)
    _, bound_r = O.gemm_f64(Ar, Br, transB=transB)
    assert O.normalized_error(C, ref_rounded, bound_r) <= 1e-4
    ref_fp32 = O.matmul_transB(A, B) if transB else O.matmul(A, B)
    _, bound = O.gemm_f64(A, B, transB=transB)
    assert O.normalized_error(C, ref_fp32, bound) <= O.TOL_HALF


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_attention_batched(hip, bf16):
    """Q.K^T (NT, 12 heads x 197 x 64 x 197) and P.V (NN, 197 x 197 x 64), 2 images."""
    BH, S, D = 24, 197, 64
    Q, Kt, V = O.randn((BH, S, D), 1), O.randn((BH, S, D), 2), O.randn((BH, S, D), 3)
    P = O.uniform((BH, S, S), 4, 0, 2.0 / S)
    dQ, dK, dV, dP = (to_dev(hip, _bits(a, bf16)) for a in (Q, Kt, V, P))
    dS, dO = empty_dev(hip, (BH, S, S)), empty_dev(hip, (BH, S, D))
    dt = 1 if bf16 else 0
    hip.HIPBackend.gemmStridedBatchedHalf(dt, 0, 1, BH, S, S, D, dQ, D, S * D, dK, D, S * D, dS, S, S * S)
    hip.HIPBackend.gemmStridedBatchedHalf(dt, 0, 0, BH, S, D, S, dP, S, S * S, dV, D, S * D, dO, D, S * D)
    Qr, Kr, Vr, Pr = (_round(a, bf16) for a in (Q, Kt, V, P))
    S_ref = O.batched_matmul_transB(Qr, Kr)
    _, bS = O.gemm_f64(Qr, Kr, transB=True)
    assert O.normalized_error(dS.numpy(), S_ref, bS) <= 1e-4
    O_ref = O.batched_matmul(Pr, Vr)
    _, bO = O.gemm_f64(Pr, Vr)
    assert O.normalized_error(dO.numpy(), O_ref, bO) <= 1e-4
    _, bS32 = O.gemm_f64(Q, Kt, transB=True)
    assert O.normalized_error(dS.numpy(), O.batched_matmul_transB(Q, Kt), bS32) <= O.TOL_HALF


# (batch, M, N, K): on a 256-CU MI355X these select the 192x256 tile (first; the
# 256x256 tile in the TN / TT layouts, whose A is R-major), the 128x128 tile
# (second) and the 64x64 tile (third); every one has ragged
# M, N and a K that ends inside a 64-deep slice. The last shape has N % 4 != 0,
# so C leaves through 32-bit stores.
FAST_SHAPES = [(40, 392, 392, 136), (24, 392, 392, 72), (4, 296, 264, 136), (3, 104, 262, 200)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("transA,transB", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("batch,M,N,K", FAST_SHAPES)
def test_half_layouts_tiles(hip, bf16, transA, transB, batch, M, N, K):
    """Every operand layout through gemmStridedBatchedHalf, against float64 on the rounded inputs."""
    seed = batch * 7 + M + N + K + 2 * transA + transB
    A = O.randn((batch, K, M) if transA else (batch, M, K), seed)
    B = O.randn((batch, N, K) if transB else (batch, K, N), seed + 1)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dC = empty_dev(hip, (batch, M, N))
    lda = M if transA else K
    ldb = K if transB else N
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, transA, transB, batch, M, N, K, dA, lda, M * K, dB, ldb,
                                          N * K, dC, N, M * N)
    C64, bound = O.gemm_f64(_round(A, bf16), _round(B, bf16), transA=bool(transA), transB=bool(transB))
    assert O.normalized_error(dC.numpy(), C64, bound) <= 1e-4


# (batch, M, N, K, transB, gap): one tile holds a batch's whole C, whose rows
# (N % 4 != 0, or a batch stride M*N + gap with gap % 4 != 0) cannot leave
# through 16-byte row stores: C is written through LDS as one contiguous run
# per batch. On a 256-CU MI355X the tile model picks 256x256 (197 rows in LDS
# passes of 128 and 69; 200 rows in passes of 192 and 8), 128x128 (one pass;
# two passes of 64 rows) and 64x64 tiles. The first shape is the ViT-B/16 b64
# Q.K^T itself (K = 64: one slice, so 64x64 tiles and element stores).
COMPACT_SHAPES = [(768, 197, 197, 64, 1, 0), (768, 197, 197, 72, 1, 0), (400, 200, 130, 80, 0, 0),
                  (512, 100, 102, 72, 0, 0), (512, 120, 128, 96, 1, 3), (512, 50, 61, 72, 1, 0),
                  (2048, 33, 47, 88, 0, 0)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("batch,M,N,K,transB,gap", COMPACT_SHAPES)
def test_half_compact_store(hip, bf16, batch, M, N, K, transB, gap):
    """Whole-C-in-one-tile batches: values against float64 on sampled batches, every gap and the
    bytes past the last batch untouched."""
    seed = batch + M + N + K + transB + gap
    A = O.randn((batch, M, K), seed)
    B = O.randn((batch, N, K) if transB else (batch, K, N), seed + 1)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    sC = M * N + gap
    tail = 67
    C0 = np.full(batch * sC + tail, np.nan, np.float32)   # no product of finite inputs is NaN
    dC = to_dev(hip, C0)
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, 0, transB, batch, M, N, K, dA, K, M * K, dB,
                                          K if transB else N, N * K, dC, N, sC)
    C = dC.numpy()
    Ar, Br = _round(A, bf16), _round(B, bf16)
    picks = sorted({0, 1, 2, batch // 2 - 1, batch // 2, batch - 2, batch - 1})
    for b in picks:
        C64, bound = O.gemm_f64(Ar[b], Br[b], transB=bool(transB))
        got = C[b * sC:b * sC + M * N].reshape(M, N)
        assert O.normalized_error(got, C64, bound) <= 1e-4, f"batch {b}"
    runs = C[:batch * sC].reshape(batch, sC)
    assert np.all(np.isnan(runs[:, M * N:])), "batch gaps must stay untouched"
    assert np.all(np.isnan(C[batch * sC:])), "nothing past the last batch is written"
    assert not np.any(np.isnan(runs[:, :M * N])), "every element of every batch is written"


# Many small A . B^T with K = 64 (the attention scores: one workgroup per batch entry, B in LDS,
# 16-row blocks of A): a partial last column tile (N = 250, 7), whole tiles only (N = 256), M past
# the 16-row blocks (1000, 17), ldc wider than N and batch strides with gaps (left untouched).
HEAD_SCORE_SHAPES = [(300, 100, 250, 256, 40), (256, 1000, 7, 9, 5), (512, 17, 256, 256, 0)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("batch,M,N,ldc,gap", HEAD_SCORE_SHAPES)
def test_half_head_scores(hip, bf16, batch, M, N, ldc, gap):
    K = 64
    seed = batch + M + N
    A = O.randn((batch, M, K), seed)
    B = O.randn((batch, N, K), seed + 1)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    sC = M * ldc + gap
    C0 = np.full(batch * sC + 33, np.nan, np.float32)
    dC = to_dev(hip, C0)
    print(f"case head scores {batch}x{M}x{N} ldc {ldc}", flush=True)
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, 0, 1, batch, M, N, K, dA, K, M * K, dB, K, N * K, dC, ldc,
                                          sC)
    C = dC.numpy()
    Ar, Br = _round(A, bf16), _round(B, bf16)
    for b in sorted({0, 1, batch // 2, batch - 1}):
        C64, bound = O.gemm_f64(Ar[b], Br[b], transB=True)
        got = C[b * sC:b * sC + M * ldc].reshape(M, ldc)
        assert O.normalized_error(got[:, :N], C64, bound) <= 1e-4, f"batch {b}"
    runs = C[:batch * sC].reshape(batch, sC)
    assert not np.any(np.isnan(runs[:, :M * ldc].reshape(batch, M, ldc)[:, :, :N])), "every element is written"
    assert np.all(np.isnan(runs[:, :M * ldc].reshape(batch, M, ldc)[:, :, N:])), "columns past N stay untouched"
    assert np.all(np.isnan(runs[:, M * ldc:])), "batch gaps stay untouched"
    assert np.all(np.isnan(C[batch * sC:])), "nothing past the last batch is written"


# Many small A . B with 64 output columns (the attention context P . V: one workgroup per batch
# entry, V in LDS read through transposing reads, P rows at any half offset): K = 197 (the ViT
# keys), 250 and 256 (full steps), 33 and 1; odd lda and sub-view offsets make the P rows ragged;
# A's padding halves past K hold Inf (they must be zeroed, not multiplied by V's zero rows);
# ldc wider than 64 leaves columns untouched.
HEAD_CONTEXT_SHAPES = [(256, 197, 197, 197, 64, 0), (300, 100, 250, 251, 68, 1), (256, 1000, 33, 40, 64, 0),
                       (512, 17, 256, 256, 64, 3), (256, 5, 1, 2, 64, 1)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("batch,M,K,lda,ldc,offA", HEAD_CONTEXT_SHAPES)
def test_half_head_context(hip, bf16, batch, M, K, lda, ldc, offA):
    N = 64
    seed = batch + M + K + lda
    A = O.randn((batch, M, lda), seed)
    B = O.randn((batch, K, N), seed + 1)
    Ab = _bits(A, bf16)
    Ab[:, :, K:] = 0x7c00 if not bf16 else 0x7f80   # +Inf in the row padding
    flat = np.concatenate([np.zeros(offA, np.uint16), Ab.reshape(-1), np.zeros(8, np.uint16)])
    dAall, dB = to_dev(hip, flat), to_dev(hip, _bits(B, bf16))
    sC = M * ldc + 4
    dC = to_dev(hip, np.full(batch * sC + 20, np.nan, np.float32))
    print(f"case head context {batch}x{M}x{K} lda {lda} off {offA}", flush=True)
    hip.call("omHipGemmStridedBatchedHalf", 1 if bf16 else 0, 0, 0, batch, M, N, K, dAall.ptr + 2 * offA, lda,
             M * lda, dB.ptr, N, K * N, dC.ptr, ldc, sC)
    C = dC.numpy()
    Ar, Br = _round(A[:, :, :K], bf16), _round(B, bf16)
    for b in sorted({0, 1, batch // 2, batch - 1}):
        C64, bound = O.gemm_f64(Ar[b], Br[b])
        got = C[b * sC:b * sC + M * ldc].reshape(M, ldc)
        assert O.normalized_error(got[:, :N], C64, bound) <= 1e-4, f"batch {b}"
    runs = C[:batch * sC].reshape(batch, sC)[:, :M * ldc].reshape(batch, M, ldc)
    assert np.all(np.isfinite(runs[:, :, :N])), "every element is written, and finite"
    assert np.all(np.isnan(runs[:, :, N:])), "columns past N stay untouched"
    assert np.all(np.isnan(C.reshape(-1)[batch * sC:])), "nothing past the last batch is written"


def test_half_strided_views(hip):
    """Leading dimensions wider than the rows and batch strides with gaps (sub-matrix views)."""
    batch, M, N, K = 3, 72, 80, 96
    lda, ldb, ldc = K + 24, N + 16, N + 8
    sA, sB, sC = M * lda + 64, K * ldb + 32, M * ldc + 16
    A = O.randn((batch * sA,), 11)
    B = O.randn((batch * sB,), 12)
    dA, dB = to_dev(hip, _bits(A, False)), to_dev(hip, _bits(B, False))
    C0 = np.full(batch * sC, -7.0, np.float32)
    dC = to_dev(hip, C0)
    hip.HIPBackend.gemmStridedBatchedHalf(0, 0, 0, batch, M, N, K, dA, lda, sA, dB, ldb, sB, dC, ldc, sC)
    C = dC.numpy()
    Ar, Br = _round(A, False), _round(B, False)
    for b in range(batch):
        a = Ar[b * sA:b * sA + M * lda].reshape(M, lda)[:, :K]
        bm = Br[b * sB:b * sB + K * ldb].reshape(K, ldb)[:, :N]
        C64, bound = O.gemm_f64(a, bm)
        got = C[b * sC:b * sC + M * ldc].reshape(M, ldc)
        assert O.normalized_error(got[:, :N], C64, bound) <= 1e-4
        assert np.all(got[:, N:] == -7.0), "columns past N must stay untouched"
    for b in range(batch - 1):
        assert np.all(C[b * sC + M * ldc:(b + 1) * sC] == -7.0), "batch gaps must stay untouched"


def test_half_known_answer(hip):
    A = np.array([[1, 2], [3, 4]], np.float16).view(np.uint16)
    B = np.array([[5, 6], [7, 8]], np.float16).view(np.uint16)
    dA, dB, dC = to_dev(hip, A), to_dev(hip, B), empty_dev(hip, (2, 2))
    hip.HIPBackend.matmulHalf(dA, dB, dC, 2, 2, 2)
    assert dC.numpy().tolist() == [[19, 22], [43, 50]]


# K-major operands whose rows start at odd halves (odd K): the ragged loader.
# (batch, M, N, K) chosen so the tile model picks, on a 256-CU MI355X, the
# 256x256 tile (first), the 128x128 tile (second) and the 64x64 tile (third:
# the ViT P.V shape, 197 keys). K ends 1, 13 and 5 halves into its last
# 64-deep slice, so the zeroing of the halves past K (where the next row's
# data lies) decides the result.
RAGGED_SHAPES = [(16, 600, 1000, 65), (3, 1300, 1300, 77), (48, 197, 64, 197)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("transB", [0, 1], ids=["NN", "NT"])
@pytest.mark.parametrize("batch,M,N,K", RAGGED_SHAPES)
def test_half_ragged_k(hip, bf16, transB, batch, M, N, K):
    seed = batch + M + N + K + transB
    A = O.randn((batch, M, K), seed)
    B = O.randn((batch, N, K) if transB else (batch, K, N), seed + 1)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dC = empty_dev(hip, (batch, M, N))
    ldb = K if transB else N
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, 0, transB, batch, M, N, K, dA, K, M * K, dB, ldb, N * K,
                                          dC, N, M * N)
    C64, bound = O.gemm_f64(_round(A, bf16), _round(B, bf16), transB=bool(transB))
    assert O.normalized_error(dC.numpy(), C64, bound) <= 1e-4


@pytest.mark.parametrize("transB", [0, 1], ids=["NN", "NT"])
@pytest.mark.parametrize("offA,offB", [(1, 3), (3, 1), (2, 0)])
def test_half_ragged_views(hip, transB, offA, offB):
    """Operands that start at odd halves (sub-buffer views), odd leading dimensions and
    odd batch strides with an even K: only the alignment makes the K-major rows ragged."""
    batch, M, N, K = 3, 70, 88, 96
    lda = K + 3
    ldb = (K + 5) if transB else N
    sA, sB = M * lda + 7, (N * ldb + 9) if transB else K * ldb
    A = O.randn((offA + batch * sA,), 21)
    B = O.randn((offB + batch * sB,), 22)
    dA, dB = to_dev(hip, _bits(A, False)), to_dev(hip, _bits(B, False))
    dC = empty_dev(hip, (batch, M, N))
    hip.HIPBackend.gemmStridedBatchedHalf(0, 0, transB, batch, M, N, K, int(dA) + 2 * offA, lda, sA,
                                          int(dB) + 2 * offB, ldb, sB, dC, N, M * N)
    Ar, Br = _round(A, False), _round(B, False)
    C = dC.numpy()
    for b in range(batch):
        a = Ar[offA + b * sA:offA + b * sA + M * lda].reshape(M, lda)[:, :K]
        if transB:
            bm = Br[offB + b * sB:offB + b * sB + N * ldb].reshape(N, ldb)[:, :K]
        else:
            bm = Br[offB + b * sB:offB + b * sB + K * ldb].reshape(K, ldb)
        C64, bound = O.gemm_f64(a, bm, transB=bool(transB))
        assert O.normalized_error(C[b], C64, bound) <= 1e-4


# 256 x 256 tiles in a single round (150 tiles on 256 CUs: the ViT-B/16 output projection over
# 12608 tokens, and ragged M / N with a partial last K slice in the NT layout): fp32 output
# leaves through the staged streaming store, as does the half output of the fused Linear.
ONE_ROUND_SHAPES = [(12608, 768, 768, 0), (12603, 760, 1000, 1)]


def _sample_rows(M):
    return np.unique(np.concatenate([np.arange(0, M, 97), np.arange(M - 5, M)]))


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("M,N,K,transB", ONE_ROUND_SHAPES, ids=lambda v: str(v))
def test_half_one_round_staged(hip, bf16, M, N, K, transB):
    """Against float64 on sampled rows of the rounded inputs (all columns), and the fused
    Linear epilogue (bias, ReLU, half output) equal to gemm -> addBias -> relu -> convert."""
    H = hip.HIPBackend
    A = O.randn((M, K), M + K + 3)
    B = O.randn((N, K) if transB else (K, N), N + 5, 0.02)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dt = 1 if bf16 else 0
    C = empty_dev(hip, (M, N))
    H.gemmStridedBatchedHalf(dt, 0, transB, 1, M, N, K, dA, K, 0, dB, K if transB else N, 0, C, N, 0)
    c = C.numpy()
    rows = _sample_rows(M)
    Ar, Br = _round(A, bf16)[rows].astype(np.float64), _round(B, bf16).astype(np.float64)
    Bm = Br.T if transB else Br
    assert O.normalized_error(c[rows], Ar @ Bm, np.abs(Ar) @ np.abs(Bm)) <= 1e-4
    bias = O.randn((N,), N + 11, 0.5)
    db = to_dev(hip, bias)
    out16 = empty_dev(hip, (M, N), np.uint16)
    H.linearHalf(dA, dB, db, out16, M, K, N, bf16=bf16, transW=bool(transB), act=1, outHalf=True)
    H.addBias(C, db, C, M, N)
    H.relu(C, C, M * N)
    chain16 = empty_dev(hip, (M, N), np.uint16)
    H.convertToHalf(C, chain16, M * N, bf16=bf16)
    assert np.array_equal(out16.numpy(), chain16.numpy())


# (M, N, K): one round of 192 x 256 tiles on a 256-CU MI355X (the tile model prefers it
# when 256 x 256 tiles would leave more CUs idle: 8000 x 1500 is 252 tiles against 192);
# ragged M, N and K, an odd K (the ragged K-major loader) and the ViT-B/16 b64 output
# projection itself.
TILE192_SHAPES = [(8000, 1500, 200), (8000, 1500, 201), (12608, 768, 768)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("transB", [0, 1], ids=["NN", "NT"])
@pytest.mark.parametrize("M,N,K", TILE192_SHAPES, ids=lambda v: str(v))
def test_half_tile_192(hip, bf16, transB, M, N, K):
    """Sampled rows (every 97th and the last five, all columns) against float64, and every
    row sum and column sum of C against A (B 1) and (1^T A) B, K-scaled (tol 1e-4)."""
    A = O.randn((M, K), M + N + K)
    B = O.randn((N, K) if transB else (K, N), M + N + K + 1, 0.05)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dC = empty_dev(hip, (M, N))
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, 0, transB, 1, M, N, K, dA, K, 0, dB,
                                          K if transB else N, 0, dC, N, 0)
    C = dC.numpy()
    A64 = _round(A, bf16).astype(np.float64)
    B64 = _round(B, bf16).astype(np.float64)
    B64 = B64.T if transB else B64
    rows = _sample_rows(M)
    assert O.normalized_error(C[rows], A64[rows] @ B64, np.abs(A64[rows]) @ np.abs(B64)) <= 1e-4
    C64 = C.astype(np.float64)
    rs_bound = np.abs(A64) @ np.abs(B64).sum(axis=1)
    assert np.max(np.abs(C64.sum(axis=1) - A64 @ B64.sum(axis=1)) / rs_bound) <= 1e-4
    cs_bound = np.abs(A64).sum(axis=0) @ np.abs(B64)
    assert np.max(np.abs(C64.sum(axis=0) - A64.sum(axis=0) @ B64) / cs_bound) <= 1e-4
