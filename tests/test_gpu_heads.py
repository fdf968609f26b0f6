"""The fp32 pieces of the engine's ViT attention branch and of tensorSum, through the C ABI:

* omHipQkvSplitHeads / omHipMergeHeads (CUDABackend::qkvSplitHeads / mergeHeads,
  om.hal.cuda_backend.ixx:967-985): bit-exact against the oracle's restatement of the
  CPU branch's loops (vit.ixx:196-232), at the ViT-B/16 b64 size and at shapes that take
  the scalar path (head dimension not a multiple of 4, unaligned pointers);
* omHipAttention (vit.ixx:163-187 on fp32 QKV): against float64 and against the oracle's
  fp32 chain within 1e-5 of sum_j P_ij |V_jd| per context element (fp32 products and
  softmax: expected ~1e-7), and against the golden vector the compiled reference wrote;
* omHipSum / omHipMean (omCudaSum / omCudaMean; CPUBackend::sum cpu_backend.ixx:290-294):
  within 2^-24 * 64 * sum|x| of float64 (the fixed-order tree's chains are far shorter
  than the sequential loop's), repeated calls bit-identical, mean = sum * (1 / n) exactly.

omHipForceReset invalidates every device buffer, so it is exercised in its own process by
the C++ HIPBackend caller (tests/cpp/test_hip_backend.cpp), not here.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from conftest import empty_dev, to_dev

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "reference_cpubackend.npz")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


HEAD_SHAPES = [(64, 197, 12, 64), (2, 197, 12, 64), (3, 5, 4, 6), (1, 7, 3, 4), (2, 9, 5, 3), (4, 1, 1, 1)]


@pytest.mark.parametrize("B,S,H,D", HEAD_SHAPES, ids=lambda v: str(v))
def test_split_merge_exact(hip, B, S, H, D):
    print(f"case split/merge {B}x{S}x{H}x{D}", flush=True)
    qkv = O.randn((B * S, 3 * H * D), 7 * B + S + H + D)
    scale = 1.0 / np.sqrt(D)
    dqkv = to_dev(hip, qkv)
    dq, dk, dv = (empty_dev(hip, (B * H, S, D)) for _ in range(3))
    hip.HIPBackend.qkvSplitHeads(dqkv, dq, dk, dv, B, S, H, D, scale)
    q, k, v = O.qkv_split_heads(qkv, B, S, H, D, scale)
    assert np.array_equal(_bits(dq.numpy()), _bits(q))
    assert np.array_equal(_bits(dk.numpy()), _bits(k))
    assert np.array_equal(_bits(dv.numpy()), _bits(v))
    dout = empty_dev(hip, (B * S, H * D))
    hip.HIPBackend.mergeHeads(dv, dout, B, S, H, D)
    assert np.array_equal(_bits(dout.numpy()), _bits(O.merge_heads(v, B, S, H, D)))
    assert np.array_equal(_bits(dout.numpy()), _bits(qkv[:, 2 * H * D:]))   # merge inverts the split


def test_split_merge_unaligned(hip):
    """Pointers one float off 16-byte alignment take the element path; results stay exact."""
    B, S, H, D = 2, 11, 3, 8
    qkv = O.randn((B * S, 3 * H * D), 71)
    big = to_dev(hip, np.concatenate([np.zeros(1, np.float32), qkv.reshape(-1)]))
    n = B * H * S * D
    outs = empty_dev(hip, (3 * n + 4,))
    base = outs.ptr + 4
    hip.call("omHipQkvSplitHeads", big.ptr + 4, base, base + 4 * n, base + 8 * n, B, S, H, D,
             ctypes.c_float(0.25))
    got = outs.numpy()[1:1 + 3 * n].reshape(3, B * H, S, D)
    for g, want in zip(got, O.qkv_split_heads(qkv, B, S, H, D, 0.25)):
        assert np.array_equal(_bits(g), _bits(want))
    m = empty_dev(hip, (B * S * H * D + 1,))
    hip.call("omHipMergeHeads", base, m.ptr + 4, B, S, H, D)
    assert np.array_equal(_bits(m.numpy()[1:].reshape(B * S, H * D)), _bits(qkv[:, :H * D] * np.float32(0.25)))


ATTN_SHAPES = [(2, 197, 12, 64), (3, 50, 2, 64), (1, 33, 4, 32), (2, 7, 3, 4), (1, 1, 2, 8), (5, 20, 3, 16)]


@pytest.mark.parametrize("B,S,H,D", ATTN_SHAPES, ids=lambda v: str(v))
def test_attention_fp32(hip, B, S, H, D):
    print(f"case attention fp32 {B}x{S}x{H}x{D}", flush=True)
    qkv = O.randn((B * S, 3 * H * D), 1000 + B * S + H * D, 0.5)
    scale = 1.0 / np.sqrt(D)
    dq = to_dev(hip, qkv)
    dout = empty_dev(hip, (B * S, H * D))
    hip.HIPBackend.attention(dq, dout, B, S, H, D, scale)
    got = dout.numpy()
    ref64, bound = O.attention_f64(qkv, B, S, H, D, scale)
    assert O.normalized_error(got, ref64, bound) <= 1e-5
    assert O.normalized_error(got, O.attention(qkv, B, S, H, D, scale), bound) <= 1e-5


def test_attention_fp32_vit_b64_sampled(hip):
    """The full ViT-B/16 b64 shape (768 heads of 197 tokens, the outer loop over 12 heads each
    batching 64 images) against float64 on four sampled images, every head of each; every
    output element finite."""
    B, S, H, D = 64, 197, 12, 64
    qkv = O.randn((B * S, 3 * H * D), 4242, 0.5)
    dq = to_dev(hip, qkv)
    dout = empty_dev(hip, (B * S, H * D))
    hip.HIPBackend.attention(dq, dout, B, S, H, D, 0.125)
    got = dout.numpy().reshape(B, S, H * D)
    assert np.all(np.isfinite(got))
    for b in (0, 17, 40, 63):
        ref64, bound = O.attention_f64(qkv.reshape(B, S, -1)[b], 1, S, H, D, 0.125)
        assert O.normalized_error(got[b], ref64, bound) <= 1e-5, b


def test_attention_fp32_golden_vector(hip):
    """The attention core the compiled reference computed from its own transpose2d,
    batchedMatmul and softmax (2 images, 7 tokens, 3 heads of 4, scale 0.5)."""
    with np.load(GOLD, allow_pickle=False) as z:
        qkv, want = z["attention_2x7x3x4.qkv"], z["attention_2x7x3x4.out"]
    dq = to_dev(hip, qkv)
    dout = empty_dev(hip, want.shape)
    hip.HIPBackend.attention(dq, dout, 2, 7, 3, 4, 0.5)
    _, bound = O.attention_f64(qkv, 2, 7, 3, 4, 0.5)
    assert O.normalized_error(dout.numpy(), want, bound) <= 1e-5


SUM_SIZES = [1, 3, 64, 1000, 4096, 4097, 65537, 1 << 20, 10_000_019]


@pytest.mark.parametrize("n", SUM_SIZES)
def test_sum_mean(hip, n):
    print(f"case sum {n}", flush=True)
    x = O.randn((n,), 500 + n % 97, 2.0) + np.float32(0.25)
    dx = to_dev(hip, x)
    r = empty_dev(hip, (4,))
    hip.HIPBackend.sum(dx, r, n)
    s1 = r.numpy()[0]
    exact = x.astype(np.float64).sum()
    budget = 2.0 ** -24 * 64 * np.abs(x).astype(np.float64).sum()
    assert abs(float(s1) - exact) <= budget
    seq = O.sum_(x)                     # the reference's sequential loop, for scale
    assert abs(float(s1) - exact) <= abs(float(seq) - exact) + budget
    hip.HIPBackend.sum(dx, r, n)
    assert r.numpy()[0].view(np.uint32) == s1.view(np.uint32)   # fixed order
    hip.HIPBackend.mean(dx, r, n)
    assert r.numpy()[0].view(np.uint32) == np.float32(s1 * np.float32(1.0 / np.float32(n))).view(np.uint32)


def test_sum_known_answers_and_edges(hip):
    r = to_dev(hip, np.full(2, 9.0, np.float32))
    ones = to_dev(hip, np.ones(3_000_001, np.float32))
    hip.HIPBackend.sum(ones, r, 3_000_001)
    assert r.numpy()[0] == np.float32(3_000_001)
    hip.HIPBackend.sum(ones, r, 0)                          # nothing to add: 0
    assert r.numpy()[0] == 0.0
    ints = O.rng(5).integers(-50, 50, 1_000_003).astype(np.float32)
    dints = to_dev(hip, ints)
    hip.HIPBackend.sum(dints, r, ints.size)                 # integers: every order is exact
    assert r.numpy()[0] == np.float32(ints.astype(np.int64).sum())
    off = to_dev(hip, np.concatenate([np.zeros(1, np.float32), ints]))   # unaligned start
    hip.call("omHipSum", off.ptr + 4, r.ptr, ints.size)
    assert r.numpy()[0] == np.float32(ints.astype(np.int64).sum())
    hip.HIPBackend.mean(ones, r, 1000)
    assert r.numpy()[0] == np.float32(1.0)
    with pytest.raises(hip.OmHipError, match="null"):
        hip.HIPBackend.sum(None, r, 5)
