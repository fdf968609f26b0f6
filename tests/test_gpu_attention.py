"""Fused multi-head attention (half-precision inputs, fp32 accumulate) against
float64 and against the reference chain (oracle: split heads with Q scaled,
Q x K^T, softmax, P x V, merge heads — vit.ixx:193-236, cpu_backend.ixx:352-370)
on the same rounded inputs.

Bar, per context element: |O - O_ref| <= tol * sum_j P_ij |V_jd| with
tol = 1e-3 (fp16) / 1e-2 (bf16) for fp32 output and 2e-3 / 1.2e-2 with the
output rounded to the input type: P is rounded to the input type before P x V
(2^-11 resp. 2^-8 relative), everything else is fp32.
"""
import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu


def _rounded(x, bf16):
    return O.bf16_round(x) if bf16 else x.astype(np.float16).astype(np.float32)


def _bits(x, bf16):
    return O.bf16_bits(x) if bf16 else x.astype(np.float16).view(np.uint16)


SHAPES = [(2, 197, 12, 64), (3, 50, 2, 64), (1, 384, 1, 64), (2, 1, 3, 64), (1, 33, 4, 64), (2, 96, 2, 64)]


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("out_half", [False, True], ids=["out32", "outhalf"])
@pytest.mark.parametrize("B,S,H,D", SHAPES, ids=lambda v: str(v))
def test_attention(hip, bf16, out_half, B, S, H, D):
    qkv = O.randn((B * S, 3 * H * D), B * 1000 + S + H, 0.5)
    scale = 1.0 / np.sqrt(D)
    dq = to_dev(hip, _bits(qkv, bf16))
    if out_half:
        dout = empty_dev(hip, (B * S, H * D), np.uint16)
    else:
        dout = empty_dev(hip, (B * S, H * D))
    hip.HIPBackend.attentionHalf(dq, dout, B, S, H, D, scale, bf16=bf16, outHalf=out_half)
    got = dout.numpy()
    if out_half:
        got = (got.astype(np.uint32) << 16).view(np.float32) if bf16 else got.view(np.float16).astype(np.float32)
    qr = _rounded(qkv, bf16)
    ref64, bound = O.attention_f64(qr, B, S, H, D, scale)
    tol = (1.2e-2 if bf16 else 2e-3) if out_half else (1e-2 if bf16 else 1e-3)
    assert O.normalized_error(got, ref64, bound) <= tol
    ref = O.attention(qr, B, S, H, D, scale)            # the reference chain in fp32
    assert O.normalized_error(got, ref, bound) <= tol


# Grids of several rounds (two 8-wave workgroups per CU, 512 per round on 256 CUs): 770 pairs end
# in a partial round, S = 16 is one query block per head, S = 100 seven, S = 197 / 208 thirteen
# (the 13 key tiles of a full last tile at 208).
MANY = [(385, 16, 2, 64), (256, 100, 3, 64), (130, 197, 6, 64), (64, 208, 12, 64)]


@pytest.mark.parametrize("bf16,out_half", [(False, False), (True, True)], ids=["f16-out32", "bf16-outhalf"])
@pytest.mark.parametrize("B,S,H,D", MANY, ids=lambda v: str(v))
def test_attention_many_heads(hip, bf16, out_half, B, S, H, D):
    test_attention(hip, bf16, out_half, B, S, H, D)


def test_attention_rejects_unsupported(hip):
    d = to_dev(hip, np.zeros(3 * 32 * 4, np.uint16))
    o = empty_dev(hip, (4 * 32,))
    with pytest.raises(hip.OmHipError, match="head dimension"):
        hip.HIPBackend.attentionHalf(d, o, 1, 4, 1, 32, 1.0)
    with pytest.raises(hip.OmHipError, match="sequence length"):
        hip.HIPBackend.attentionHalf(d, o, 1, 385, 1, 64, 1.0)
