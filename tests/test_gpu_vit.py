"""The ViT attention layer on half-precision activations and weights.

omHipLinearHalf is Linear::forward (linear.ixx:50-58: x W + b with W stored
[in, out]) on fp16 / bf16 inputs with fp32 accumulate, the bias add and ReLU
in the GEMM's epilogue and the output in fp32 or rounded to the input type.
Bars: bit-identical to the unfused chain (half GEMM with fp32 output, then
omHipAddBias, omHipReLU, omHipConvertF32To{F16,BF16}); against the oracle on
the same rounded inputs, K-scaled (|C - C_ref| <= tol * (sum_k |x_ik||w_kj| +
|b_j|)) with tol 1e-4 for fp32 output (only accumulation order differs) and
2^-11 / 2^-8 (+1e-4) with the output rounded to fp16 / bf16.

omHipMultiHeadAttentionHalf is MultiHeadAttention::forward (vit.ixx:150-239):
QKV Linear -> heads split with Q scaled by 1/sqrt(d) -> softmax(Q K^T) V ->
heads merged -> output Linear. It is checked at batch 2 against float64 and
against the oracle chain (the reference's matmul, addBias, attention chain
and matmul) on the same rounded inputs. The fused path (head dim 64, at most
384 tokens) rounds the projection, P and the context to the input type; the
reference for it rounds the projection the same way. The unfused path keeps
fp32 up to the context. Bar per output element:
|out - out_ref| <= tol * ((B_ctx + |ctx|) |Wout| + |b_out|), where B_ctx =
sum_j P_ij |V_jd| is the attention's own error budget and tol = 2u + 1e-4
(3u + 1e-4 with half output), u = 2^-11 (fp16) / 2^-8 (bf16): P rounded
(u B_ctx), the context rounded (u |ctx|), the final rounding (u |out|) and
fp32 accumulation. Biases are drawn at 0.5 so that a dropped bias exceeds
the bar.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def _round(x, bf16):
    return O.bf16_round(x) if bf16 else np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _bits(x, bf16):
    return O.bf16_bits(x) if bf16 else np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _from_bits(u, bf16):
    return (u.astype(np.uint32) << 16).view(np.float32) if bf16 else u.view(np.float16).astype(np.float32)


# (4500, 96, 4100): 306 tiles of 256 x 256, more than one round on 256 CUs (the
# register store path for fp32, the staged one for half output).
LINEAR_SHAPES = [(394, 768, 2304), (394, 768, 768), (197, 3072, 768), (33, 40, 17), (128, 256, 260), (2, 3, 4),
                 (4500, 96, 4100)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("transW", [False, True], ids=["W_in_out", "W_out_in"])
@pytest.mark.parametrize("act", [0, 1], ids=["none", "relu"])
@pytest.mark.parametrize("M,K,N", LINEAR_SHAPES, ids=lambda v: str(v))
def test_linear_half(hip, bf16, transW, act, M, K, N):
    H = hip.HIPBackend
    x = O.randn((M, K), M + K)
    w = O.randn((N, K) if transW else (K, N), N + 7, 1.0 / np.sqrt(K))
    b = O.randn((N,), N + 9, 0.5)
    dx, dw, db = to_dev(hip, _bits(x, bf16)), to_dev(hip, _bits(w, bf16)), to_dev(hip, b)
    out32 = empty_dev(hip, (M, N))
    out16 = empty_dev(hip, (M, N), np.uint16)
    H.linearHalf(dx, dw, db, out32, M, K, N, bf16=bf16, transW=transW, act=act)
    H.linearHalf(dx, dw, db, out16, M, K, N, bf16=bf16, transW=transW, act=act, outHalf=True)
    # the unfused chain on the device
    chain = empty_dev(hip, (M, N))
    H.gemmStridedBatchedHalf(1 if bf16 else 0, 0, transW, 1, M, N, K, dx, K, 0, dw, K if transW else N, 0, chain, N, 0)
    H.addBias(chain, db, chain, M, N)
    if act:
        H.relu(chain, chain, M * N)
    chain16 = empty_dev(hip, (M, N), np.uint16)
    H.convertToHalf(chain, chain16, M * N, bf16=bf16)
    got32, got16 = out32.numpy(), out16.numpy()
    assert np.array_equal(got32.view(np.uint32), chain.numpy().view(np.uint32))
    assert np.array_equal(got16, chain16.numpy())
    # the oracle on the same rounded inputs
    xr, wr = _round(x, bf16), _round(w, bf16)
    ref = O.add_bias(O.matmul_transB(xr, wr) if transW else O.matmul(xr, wr), b)
    if act:
        ref = O.relu(ref)
    _, bound = O.gemm_f64(xr, wr, transB=transW)
    bound = bound + np.abs(b)[None, :]
    assert O.normalized_error(got32, ref, bound) <= 1e-4
    half_tol = (2.0 ** -8 if bf16 else 2.0 ** -11) + 1e-4
    assert O.normalized_error(_from_bits(got16, bf16), ref, bound) <= half_tol


def test_linear_half_degenerate(hip):
    """K = 0 (no terms): act(0 + b) in either output type; no bias and fp32 output: zeros."""
    H = hip.HIPBackend
    M, N = 5, 12
    b = np.linspace(-1.0, 1.0, N).astype(np.float32)
    db = to_dev(hip, b)
    out32, out16 = empty_dev(hip, (M, N)), empty_dev(hip, (M, N), np.uint16)
    H.fillValue(out32, M * N, 7.0)
    H.linearHalf(None, None, db, out32, M, 0, N, act=1)
    H.linearHalf(None, None, db, out16, M, 0, N, act=1, outHalf=True)
    want = np.broadcast_to(np.maximum(b, 0), (M, N))
    assert np.array_equal(out32.numpy(), want)
    assert np.array_equal(out16.numpy(), want.astype(np.float16).view(np.uint16))
    H.linearHalf(None, None, None, out32, M, 0, N)
    assert np.all(out32.numpy() == 0)
    with pytest.raises(hip.OmHipError, match="activation"):
        H.linearHalf(None, None, db, out32, M, 0, N, act=2)


def _mha_reference(x, wqkv, bqkv, wo, bo, B, S, Hh, Dh, bf16, fused):
    """float64 chain and its error budget; the oracle chain (fp32, reference ops)."""
    scale = np.float32(1.0 / np.sqrt(np.float32(Dh)))
    qkv64 = x.astype(np.float64) @ wqkv.astype(np.float64) + bqkv.astype(np.float64)
    qkv_in = _round(qkv64.astype(np.float32), bf16) if fused else qkv64
    ctx64, bctx = O.attention_f64(qkv_in, B, S, Hh, Dh, float(scale))
    out64 = ctx64 @ wo.astype(np.float64) + bo.astype(np.float64)
    bound = (bctx + np.abs(ctx64)) @ np.abs(wo.astype(np.float64)) + np.abs(bo.astype(np.float64))
    qkv32 = O.add_bias(O.matmul(x, wqkv), bqkv)
    if fused:
        qkv32 = _round(qkv32, bf16)
    ctx32 = O.attention(qkv32, B, S, Hh, Dh, float(scale))
    out32 = O.add_bias(O.matmul(_round(ctx32, bf16), wo), bo)
    return out64, bound, out32


# (batch, tokens, heads, head dim): ViT-B/16 and a small fused case; head dim
# 32 and 48 and 400 tokens take the unfused chain, over images (heads > batch)
# and over heads (heads <= batch).
MHA_SHAPES = [(2, 197, 12, 64), (2, 50, 2, 64), (2, 33, 3, 32), (2, 400, 2, 64), (4, 20, 2, 48)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("out_half", [False, True], ids=["out32", "outhalf"])
@pytest.mark.parametrize("B,S,Hh,Dh", MHA_SHAPES, ids=lambda v: str(v))
def test_multi_head_attention(hip, bf16, out_half, B, S, Hh, Dh):
    D = Hh * Dh
    seed = B * 1000 + S * 10 + Hh
    x = _round(O.randn((B * S, D), seed), bf16)
    wqkv = _round(O.randn((D, 3 * D), seed + 1, 1.0 / np.sqrt(D)), bf16)
    bqkv = O.randn((3 * D,), seed + 2, 0.5)
    wo = _round(O.randn((D, D), seed + 3, 1.0 / np.sqrt(D)), bf16)
    bo = O.randn((D,), seed + 4, 0.5)
    dev = [to_dev(hip, _bits(a, bf16)) for a in (x, wqkv)] + [to_dev(hip, bqkv), to_dev(hip, _bits(wo, bf16)),
                                                              to_dev(hip, bo)]
    out = empty_dev(hip, (B * S, D), np.uint16 if out_half else np.float32)
    print(f"[mha] B={B} S={S} H={Hh} Dh={Dh} bf16={bf16} out_half={out_half}", flush=True)
    hip.HIPBackend.multiHeadAttentionHalf(*dev, out, B, S, Hh, Dh, bf16=bf16, outHalf=out_half)
    got = out.numpy()
    got = _from_bits(got, bf16) if out_half else got
    fused = Dh == 64 and S <= 384
    out64, bound, ref32 = _mha_reference(x, wqkv, bqkv, wo, bo, B, S, Hh, Dh, bf16, fused)
    u = 2.0 ** -8 if bf16 else 2.0 ** -11
    tol = (3 if out_half else 2) * u + 1e-4
    assert O.normalized_error(got, out64, bound) <= tol
    assert O.normalized_error(got, ref32, bound) <= tol
    # without biases the same chain runs with null bias pointers
    if Dh == 64 and not out_half and not bf16:
        out2 = empty_dev(hip, (B * S, D))
        hip.HIPBackend.multiHeadAttentionHalf(dev[0], dev[1], None, dev[3], None, out2, B, S, Hh, Dh)
        z3, z1 = np.zeros(3 * D, np.float32), np.zeros(D, np.float32)
        o64, bd, r32 = _mha_reference(x, wqkv, z3, wo, z1, B, S, Hh, Dh, False, fused)
        assert O.normalized_error(out2.numpy(), o64, bd) <= tol
