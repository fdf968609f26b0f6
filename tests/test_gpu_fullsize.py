"""Parity at the full sizes the benchmark times (ViT-B/16 at batch 64: 12608 tokens,
768 attention heads; ResNet-18 training at batch 32).

Every element of every output is covered by two float64 checks on the same rounded
inputs, each within the K-scaled bar sum_k |a_ik||b_kj| (tol 1e-4, fp32 accumulate):
  * sampled rows (every 97th row and the last five: each 256-row tile holds two or
    three), all columns, element by element;
  * the row sums and column sums of C against A (B 1) and (1^T A) B, whose bars are the
    row / column sums of |A||B|: a wrong, missing or repeated tile anywhere moves the
    sums of its 64..256 rows and columns far past that bar.
The projections follow Linear::forward (linear.ixx:50-58) over CPUBackend::matmul
(cpu_backend.ixx:239-286); the attention products follow MultiHeadAttention::forward
(vit.ixx:193-236) over batchedMatmul (cpu_backend.ixx:1520-1532).
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu
TOKENS = 64 * 197


def _round(x, bf16):
    return O.bf16_round(x) if bf16 else x.astype(np.float16).astype(np.float32)


def _bits(x, bf16):
    return O.bf16_bits(x) if bf16 else x.astype(np.float16).view(np.uint16)


def _sample_rows(M):
    return np.unique(np.concatenate([np.arange(0, M, 97), np.arange(M - 5, M)]))


def _check_full(C, A, B, transB, tol=1e-4):
    """Sampled rows element by element, then every row sum and column sum (float64)."""
    A64 = A.astype(np.float64)
    B64 = (B.T if transB else B).astype(np.float64)          # K x N
    rows = _sample_rows(A.shape[0])
    e_rows = O.normalized_error(C[rows], A64[rows] @ B64, np.abs(A64[rows]) @ np.abs(B64))
    absA, absB = np.abs(A64), np.abs(B64)
    rs = C.astype(np.float64).sum(axis=1)
    e_rs = np.max(np.abs(rs - A64 @ B64.sum(axis=1)) / (absA @ absB.sum(axis=1)))
    cs = C.astype(np.float64).sum(axis=0)
    e_cs = np.max(np.abs(cs - A64.sum(axis=0) @ B64) / (absA.sum(axis=0) @ absB))
    assert np.all(np.isfinite(C)), "non-finite output"
    assert e_rows <= tol, f"sampled rows {e_rows:.2e}"
    assert e_rs <= tol, f"row sums {e_rs:.2e}"
    assert e_cs <= tol, f"column sums {e_cs:.2e}"
    return max(e_rows, e_rs, e_cs)


# (name, M, N, K): the four ViT-B/16 Linear layers over 64 images x 197 tokens
VIT_PROJ = [("qkv", TOKENS, 2304, 768), ("out_proj", TOKENS, 768, 768), ("fc1", TOKENS, 3072, 768),
            ("fc2", TOKENS, 768, 3072)]
CASES = [(p, 0, 0) for p in VIT_PROJ] + [(p, 1, 0) for p in VIT_PROJ] + [(p, 0, 1) for p in VIT_PROJ]


@pytest.mark.parametrize("proj,transB,bf16", CASES,
                         ids=lambda v: v[0] if isinstance(v, tuple) else str(v))
def test_vit_projection_full(hip, proj, transB, bf16):
    name, M, N, K = proj
    print(f"case {name} {M}x{N}x{K} transB={transB} bf16={bf16}", flush=True)
    A = O.randn((M, K), 900 + K)
    B = O.randn((N, K) if transB else (K, N), 901 + N, 0.02)
    dA, dB = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(B, bf16))
    dC = empty_dev(hip, (M, N))
    hip.HIPBackend.gemmStridedBatchedHalf(1 if bf16 else 0, 0, transB, 1, M, N, K, dA, K, 0, dB,
                                          K if transB else N, 0, dC, N, 0)
    err = _check_full(dC.numpy(), _round(A, bf16), _round(B, bf16), transB)
    print(f"[{name}] worst K-scaled error {err:.2e}")


@pytest.mark.parametrize("N", [2304, 3072], ids=["qkv", "fc1"])
@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_vit_qkv_linear_full(hip, bf16, N):
    """The fused Linear (bias in the epilogue, half output) at the QKV and fc1 sizes, as the ViT
    layer runs it: every element against the unfused chain gemm -> addBias -> convert. fc1
    (600 tiles of 256 x 256) runs as two launches split by rows (the rows of two whole rounds,
    then the rest on 128 x 128 tiles), so the half-output and bias offsets of the second launch
    are checked here too."""
    H = hip.HIPBackend
    M, K = TOKENS, 768
    print(f"case linear {M}x{N}x{K} bf16={bf16}", flush=True)
    A = O.randn((M, K), 31)
    W = O.randn((K, N), 32, 0.02)
    bias = O.randn((N,), 33, 0.1)
    dA, dW, db = to_dev(hip, _bits(A, bf16)), to_dev(hip, _bits(W, bf16)), to_dev(hip, bias)
    out16 = empty_dev(hip, (M, N), np.uint16)
    H.linearHalf(dA, dW, db, out16, M, K, N, bf16=bf16, act=0, outHalf=True)
    C = empty_dev(hip, (M, N))
    H.gemmStridedBatchedHalf(1 if bf16 else 0, 0, 0, 1, M, N, K, dA, K, 0, dW, N, 0, C, N, 0)
    _check_full(C.numpy(), _round(A, bf16), _round(W, bf16), 0)
    H.addBias(C, db, C, M, N)
    chain = empty_dev(hip, (M, N), np.uint16)
    H.convertToHalf(C, chain, M * N, bf16=bf16)
    assert np.array_equal(out16.numpy(), chain.numpy())


def _batched_check(C, A, B, transB, picks, tol=1e-4):
    """Sampled batches element by element; every batch's row and column sums."""
    A64 = A.astype(np.float64)
    B64 = (np.swapaxes(B, 1, 2) if transB else B).astype(np.float64)      # batch x K x N
    for b in picks:
        assert O.normalized_error(C[b], A64[b] @ B64[b], np.abs(A64[b]) @ np.abs(B64[b])) <= tol, f"batch {b}"
    C64 = C.astype(np.float64)
    rs_ref = np.einsum("bmk,bk->bm", A64, B64.sum(axis=2))
    rs_bnd = np.einsum("bmk,bk->bm", np.abs(A64), np.abs(B64).sum(axis=2))
    cs_ref = np.einsum("bk,bkn->bn", A64.sum(axis=1), B64)
    cs_bnd = np.einsum("bk,bkn->bn", np.abs(A64).sum(axis=1), np.abs(B64))
    e_rs = np.max(np.abs(C64.sum(axis=2) - rs_ref) / rs_bnd)
    e_cs = np.max(np.abs(C64.sum(axis=1) - cs_ref) / cs_bnd)
    assert np.all(np.isfinite(C))
    assert e_rs <= tol, f"row sums {e_rs:.2e}"
    assert e_cs <= tol, f"column sums {e_cs:.2e}"


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_vit_attention_products_full(hip, bf16):
    """Q.K^T (NT) and P.V (NN) over all 768 heads of 64 images, 197 tokens, head dimension 64."""
    BH, S, D = 768, 197, 64
    H = hip.HIPBackend
    Q, Kt, V = O.randn((BH, S, D), 51), O.randn((BH, S, D), 52), O.randn((BH, S, D), 53)
    P = O.uniform((BH, S, S), 54, 0, 2.0 / S)
    dQ, dK, dV, dP = (to_dev(hip, _bits(a, bf16)) for a in (Q, Kt, V, P))
    dS, dO = empty_dev(hip, (BH, S, S)), empty_dev(hip, (BH, S, D))
    dt = 1 if bf16 else 0
    H.gemmStridedBatchedHalf(dt, 0, 1, BH, S, S, D, dQ, D, S * D, dK, D, S * D, dS, S, S * S)
    H.gemmStridedBatchedHalf(dt, 0, 0, BH, S, D, S, dP, S, S * S, dV, D, S * D, dO, D, S * D)
    picks = [0, 1, 255, 256, 383, 384, 511, 512, 766, 767]
    Qr, Kr, Vr, Pr = (_round(a, bf16) for a in (Q, Kt, V, P))
    _batched_check(dS.numpy(), Qr, Kr, True, picks)
    _batched_check(dO.numpy(), Pr, Vr, False, picks)


# images of the 64 whose 12 heads are checked: the first and last, and those either side of
# the point where the 768 heads (two per CU) run into their second round
ATTN_IMAGES = [0, 1, 21, 42, 43, 62, 63]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_fused_attention_b64(hip, bf16):
    """The fused half-precision attention at B = 64, S = 197, 12 heads of 64: sampled images
    (all heads) against float64 and the reference chain, every output finite and written."""
    B, S, H, D = 64, 197, 12, 64
    qkv = O.randn((B * S, 3 * H * D), 61, 0.5)
    scale = 1.0 / np.sqrt(D)
    dout = to_dev(hip, np.full((B * S, H * D), np.nan, np.float32))
    hip.HIPBackend.attentionHalf(to_dev(hip, _bits(qkv, bf16)), dout, B, S, H, D, scale, bf16=bf16)
    got = dout.numpy().reshape(B, S, H * D)
    assert np.all(np.isfinite(got)), "every context element is written"
    qr = _round(qkv, bf16).reshape(B, S, 3 * H * D)
    tol = 1e-2 if bf16 else 1e-3
    for b in ATTN_IMAGES:
        ref64, bound = O.attention_f64(qr[b], 1, S, H, D, scale)
        assert O.normalized_error(got[b], ref64, bound) <= tol, f"image {b}"
        assert O.normalized_error(got[b], O.attention(qr[b], 1, S, H, D, scale), bound) <= tol, f"image {b}"


def test_fp32_attention_b64(hip):
    """The fp32 attention entry (the engine's unchanged ViT branch) at B = 64."""
    B, S, H, D = 64, 197, 12, 64
    qkv = O.randn((B * S, 3 * H * D), 62, 0.5)
    scale = 1.0 / np.sqrt(D)
    dout = to_dev(hip, np.full((B * S, H * D), np.nan, np.float32))
    hip.HIPBackend.attention(to_dev(hip, qkv), dout, B, S, H, D, scale)
    got = dout.numpy().reshape(B, S, H * D)
    assert np.all(np.isfinite(got))
    q = qkv.reshape(B, S, 3 * H * D)
    for b in ATTN_IMAGES:
        ref64, bound = O.attention_f64(q[b], 1, S, H, D, scale)
        assert O.normalized_error(got[b], ref64, bound) <= 1e-5, f"image {b}"
        assert O.normalized_error(got[b], O.attention(q[b], 1, S, H, D, scale), bound) <= 1e-5, f"image {b}"


# ResNet-18 weight gradients at batch 32 (N, Cin, H, W, Cout, K, stride, pad): the stem,
# a layer-1 3x3, a layer-3 3x3 and the layer-4 downsample (conv2dBackwardWeight,
# cpu_backend.ixx:722-772)
WGRAD_B32 = [(32, 3, 224, 224, 64, 7, 2, 3), (32, 64, 56, 56, 64, 3, 1, 1), (32, 256, 14, 14, 256, 3, 1, 1),
             (32, 256, 14, 14, 512, 1, 2, 0)]


@pytest.mark.parametrize("shape", WGRAD_B32, ids=lambda s: "N{}C{}H{}W{}o{}k{}s{}p{}".format(*s))
def test_conv_backward_weight_b32(hip, shape):
    """Sampled output channels element by element; every row sum and column sum of dW."""
    N, Cin, H, W, Cout, K, s, p = shape
    print(f"case wgrad {shape}", flush=True)
    Ho, Wo = O.out_hw(H, W, K, K, s, p)
    x = O.randn((N, Cin, H, W), 161 + Cin)
    g = O.randn((N, Cout, Ho, Wo), 162 + Cout)
    dW = empty_dev(hip, (Cout, Cin, K, K))
    dB = empty_dev(hip, (Cout,))
    hip.HIPBackend.conv2dBackwardWeight(to_dev(hip, x), to_dev(hip, g), dW, dB, N, Cin, H, W, Cout, K, K, s, p)
    got = dW.numpy().reshape(Cout, -1).astype(np.float64)
    cols, _, _ = O._im2col64(np.asarray(x, np.float64), K, K, s, p)          # N x Kc x P
    g64 = np.asarray(g, np.float64).reshape(N, Cout, -1)
    rows = np.array([0, 1, Cout // 2 - 1, Cout - 1])
    ref = np.einsum("nop,nkp->ok", g64[:, rows], cols, optimize=True)
    bound = np.einsum("nop,nkp->ok", np.abs(g64[:, rows]), np.abs(cols), optimize=True)
    assert O.normalized_error(got[rows], ref, bound) <= 1e-4
    rs = np.einsum("nop,np->o", g64, cols.sum(axis=1), optimize=True)
    rs_b = np.einsum("nop,np->o", np.abs(g64), np.abs(cols).sum(axis=1), optimize=True)
    assert np.max(np.abs(got.sum(axis=1) - rs) / rs_b) <= 1e-4, "row sums"
    cs = np.einsum("np,nkp->k", g64.sum(axis=1), cols, optimize=True)
    cs_b = np.einsum("np,nkp->k", np.abs(g64).sum(axis=1), np.abs(cols), optimize=True)
    assert np.max(np.abs(got.sum(axis=0) - cs) / cs_b) <= 1e-4, "column sums"
    gb = dB.numpy().astype(np.float64)
    assert np.max(np.abs(gb - g64.sum(axis=(0, 2))) / np.abs(g64).sum(axis=(0, 2))) <= 1e-4


def test_resnet18_train_step_b32(hip):
    """The training step the benchmark times (ResNet-18, batch 32, fused BN / ReLU / residual
    entries), checked in three parts:
      * each forward op against the CPU op applied to the GPU's own input to it (conv outputs,
        saved batch statistics over all 32 images, ReLU / residual / pool outputs): 1e-4
        relative Frobenius, the kernel-parity bar;
      * the whole forward against the CPU forward from the image: 1e-3. Rounding differences
        of ~1e-7 per op grow through 17 batch-normalised layers (BN divides by the batch
        spread, ReLU inputs near zero switch sides); at batch 32 the deepest layers reach
        ~1e-4, so the end-to-end bar is the loose one;
      * every weight gradient within 1e-3 of the reference backward replayed on the GPU's own
        forward state (the split and bar of the batch-2 network test)."""
    from resnet_net import (GpuResNet18, conv_list, cpu_backward, cpu_forward_local, cpu_forward_train,
                            make_params)
    P = make_params(seed=5)
    img = O.randn((32, 3, 224, 224), 44)
    g_logits = O.randn((32, 1000), 45, 0.01)
    net = GpuResNet18(hip, P, 32, train=True, fused=True)
    net.forward_train(to_dev(hip, img))
    net.backward(to_dev(hip, g_logits))
    got = net.grads()
    fwd_gpu = net.forward_state(img)
    local = cpu_forward_local(P, fwd_gpu)
    errs = {k: O.frobenius_rel(fwd_gpu[k].reshape(v.shape), v) for k, v in local.items()}
    del local
    top = sorted(errs.items(), key=lambda kv: -kv[1])[:4]
    print("[resnet18 b32 train step] largest op errors: " + ", ".join(f"{k} {e:.2e}" for k, e in top))
    for k, e in errs.items():
        assert e <= 1e-4, f"{k} (against the op on the GPU's own input)"
    worst_l = top[0][1]
    fwd_cpu = cpu_forward_train(P, img)
    worst_f = 0.0
    for k, v in fwd_gpu.items():
        if k in ("img", "pool.idx"):
            continue
        e = O.frobenius_rel(v.reshape(fwd_cpu[k].shape), fwd_cpu[k])
        worst_f = max(worst_f, e)
        assert e <= 1e-3, k
    del fwd_cpu
    ref = cpu_backward(P, fwd_gpu, g_logits)
    worst = 0.0
    for name in [n for n, *_ in conv_list()] + ["fc.w", "fc.b"]:
        e = O.frobenius_rel(got[name].reshape(ref[name].shape), ref[name])
        worst = max(worst, e)
        assert e <= 1e-3, name
    print(f"[resnet18 b32 train step] worst op error {worst_l:.2e}, end-to-end forward {worst_f:.2e}, "
          f"weight gradients {worst:.2e}")
