// test_hip_backend.cpp — C++23 caller of om::HIPBackend (the drop-in HAL
// class), written like the reference's own GTest cases. Needs a GPU; run by
// tests/test_gpu_cpp_backend.py. Exit status 0 = every check passed.
//
// Known answers are the reference's: Matmul2D / MatmulNonSquare
// (tests/test_tensor_ops.cpp:55-82), BatchedMatmulForward
// (tests/test_phase5.cpp:206-222), LinearWithBias zero input
// (tests/test_nn.cpp:34-48), Conv2dForward shapes on all-ones input
// (tests/test_conv.cpp:21-49; interior value = sum of weights).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <vector>

#include "omhip_backend.hpp"

using om::HIPBackend;

static int g_fail = 0;
#define EXPECT_NEAR(a, b, tol)                                                                            \
    do {                                                                                                  \
        const double a_ = (a), b_ = (b);                                                                  \
        if (!(std::fabs(a_ - b_) <= (tol))) {                                                             \
            std::printf("FAIL %s:%d: %s = %.9g, expected %.9g\n", __FILE__, __LINE__, #a, a_, b_);        \
            ++g_fail;                                                                                     \
        }                                                                                                 \
    } while (0)

struct Dev {
    float* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { p = static_cast<float*>(HIPBackend::malloc(count * sizeof(float))); }
    Dev(const std::vector<float>& h) : Dev(h.size()) { HIPBackend::copyH2D(p, h.data(), h.size() * sizeof(float)); }
    ~Dev() { HIPBackend::free(p); }
    std::vector<float> host() const {
        std::vector<float> h(n);
        HIPBackend::copyD2H(h.data(), p, n * sizeof(float));
        return h;
    }
};

static void testMatmul2D() {
    Dev a(std::vector<float>{1, 2, 3, 4}), b(std::vector<float>{5, 6, 7, 8}), c(4);
    HIPBackend::matmul(a.p, b.p, c.p, 2, 2, 2);
    auto h = c.host();
    EXPECT_NEAR(h[0], 19, 0); EXPECT_NEAR(h[1], 22, 0); EXPECT_NEAR(h[2], 43, 0); EXPECT_NEAR(h[3], 50, 0);
    std::printf("Matmul2D done\n");
}

static void testMatmulNonSquare() {
    Dev a(std::vector<float>{1, 2, 3, 4, 5, 6}), b(std::vector<float>{7, 8, 9, 10, 11, 12}), c(4);
    HIPBackend::matmul(a.p, b.p, c.p, 2, 3, 2);
    auto h = c.host();
    EXPECT_NEAR(h[0], 58, 0); EXPECT_NEAR(h[1], 64, 0); EXPECT_NEAR(h[2], 139, 0); EXPECT_NEAR(h[3], 154, 0);
    // the same product with B given as [N,K] (Linear weight layout)
    Dev bt(std::vector<float>{7, 9, 11, 8, 10, 12}), c2(4);
    HIPBackend::matmulTransB(a.p, bt.p, c2.p, 2, 3, 2);
    auto h2 = c2.host();
    EXPECT_NEAR(h2[0], 58, 0); EXPECT_NEAR(h2[1], 64, 0); EXPECT_NEAR(h2[2], 139, 0); EXPECT_NEAR(h2[3], 154, 0);
    std::printf("MatmulNonSquare done\n");
}

static void testBatchedMatmulForward() {
    const int B = 2, M = 3, K = 4, N = 5;
    Dev a(std::vector<float>(B * M * K, 1.f)), b(std::vector<float>(B * K * N, 1.f)), c(B * M * N);
    HIPBackend::batchedMatmul(a.p, b.p, c.p, B, M, K, N);
    for (float v : c.host()) EXPECT_NEAR(v, 4.0, 1e-5);
    std::printf("BatchedMatmulForward done\n");
}

static void testLinearZeroInput() {
    // y = x @ W + b with x = 0, b = 0 -> y = 0 (Linear stores W[in,out], linear.ixx:31,52)
    const int batch = 2, in = 4, out = 3;
    Dev x(std::vector<float>(batch * in, 0.f)), w(std::vector<float>{.1f, .2f, .3f, .4f, .5f, .6f, .7f, .8f, .9f, 1.f, 1.1f, 1.2f});
    Dev bias(std::vector<float>(out, 0.f)), y(batch * out);
    HIPBackend::matmul(x.p, w.p, y.p, batch, in, out);
    HIPBackend::addBias(y.p, bias.p, y.p, batch, out);
    for (float v : y.host()) EXPECT_NEAR(v, 0.0, 0);
    std::printf("LinearZeroInput done\n");
}

static void testConvAllOnes() {
    // Conv2d(1,4,3,stride=1,pad=1) on [1,1,8,8] ones: shape [1,4,8,8]; interior = sum of weights
    std::vector<float> wh(4 * 9);
    for (size_t i = 0; i < wh.size(); ++i) wh[i] = 0.125f * (float)(i % 7) - 0.25f;
    Dev x(std::vector<float>(64, 1.f)), w(wh), y(4 * 64), y2(4 * 36);
    HIPBackend::conv2d(x.p, w.p, nullptr, y.p, 1, 1, 8, 8, 4, 3, 3, 1, 1);
    auto h = y.host();
    for (int co = 0; co < 4; ++co) {
        double s = 0;
        for (int t = 0; t < 9; ++t) s += wh[co * 9 + t];
        for (int r = 1; r < 7; ++r)
            for (int c = 1; c < 7; ++c) EXPECT_NEAR(h[co * 64 + r * 8 + c], s, 1e-6);
    }
    // no padding: (8-3)/1+1 = 6 -> every output is interior
    HIPBackend::conv2d(x.p, w.p, nullptr, y2.p, 1, 1, 8, 8, 4, 3, 3, 1, 0);
    auto h2 = y2.host();
    for (int co = 0; co < 4; ++co) {
        double s = 0;
        for (int t = 0; t < 9; ++t) s += wh[co * 9 + t];
        for (int i = 0; i < 36; ++i) EXPECT_NEAR(h2[co * 36 + i], s, 1e-6);
    }
    std::printf("ConvAllOnes done\n");
}

static void testReluAndErrors() {
    Dev x(std::vector<float>{-1.f, 0.f, 2.f, NAN, -0.f}), y(5);
    HIPBackend::relu(x.p, y.p, 5);
    auto h = y.host();
    EXPECT_NEAR(h[0], 0, 0); EXPECT_NEAR(h[2], 2, 0); EXPECT_NEAR(h[3], 0, 0);
    EXPECT_NEAR(std::signbit(h[4]) ? 1 : 0, 0, 0);
    bool threw = false;
    try {
        HIPBackend::conv2d(x.p, x.p, nullptr, y.p, 1, 1, 1, 1, 1, 1, 1, 0, 0);   // stride 0
    } catch (const std::runtime_error& e) {
        threw = true;
        std::printf("expected error: %s\n", e.what());
    }
    if (!threw) { std::printf("FAIL: conv2d with stride 0 did not throw\n"); ++g_fail; }
    std::printf("ReluAndErrors done\n");
}

// One training step's pieces on closed-form inputs.
static void testTrainingPieces() {
    // BN training on one channel holding 1, 2, 3, 4: mean 2.5, biased var 1.25
    Dev x(std::vector<float>{1.f, 2.f, 3.f, 4.f}), y(4), g(std::vector<float>{1.f}), b(std::vector<float>{0.f});
    Dev rm(std::vector<float>{0.f}), rv(std::vector<float>{1.f}), sm(1), si(1);
    HIPBackend::batchNorm2d(x.p, y.p, g.p, b.p, rm.p, rv.p, sm.p, si.p, 1, 1, 2, 2, 1e-5f, 0.1f, true);
    const double inv = 1.0 / std::sqrt(1.25 + 1e-5);
    auto yh = y.host();
    for (int i = 0; i < 4; ++i) EXPECT_NEAR(yh[i], (i + 1 - 2.5) * inv, 1e-6);
    EXPECT_NEAR(sm.host()[0], 2.5, 1e-7);
    EXPECT_NEAR(rm.host()[0], 0.25, 1e-7);
    EXPECT_NEAR(rv.host()[0], 0.9 + 0.125, 1e-6);
    // input gradient of a 3x3 all-ones conv (8x8 input, no padding) for an all-ones
    // output gradient: each input element counts the windows covering it
    std::vector<float> ones9(9, 1.f), ones36(36, 1.f);
    Dev w(ones9), go(ones36), gi(64);
    HIPBackend::conv2dBackwardInput(go.p, w.p, gi.p, 1, 1, 8, 8, 1, 3, 3, 1, 0);
    auto gh = gi.host();
    auto cover = [](int i) { return std::min(i, 2) - std::max(0, i - 5) + 1; };
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) EXPECT_NEAR(gh[i * 8 + j], cover(i) * cover(j), 0);
    // weight gradient: every tap sees the 6x6 window of an all-ones input
    std::vector<float> ones64(64, 1.f);
    Dev xi(ones64), gw(9), gb(1);
    HIPBackend::conv2dBackwardWeight(xi.p, go.p, gw.p, gb.p, 1, 1, 8, 8, 1, 3, 3, 1, 0);
    auto wh = gw.host();
    for (int t = 0; t < 9; ++t) EXPECT_NEAR(wh[t], 36, 0);
    EXPECT_NEAR(gb.host()[0], 36, 0);
    std::printf("TrainingPieces done\n");
}

static void testLinearBiasAct() {
    // relu([1 2 3; -4 -5 -6] @ W + b) with W = [[1, 0], [0, 1], [1, 1]] (in = 3, out = 2), b = [0.5, -10]
    Dev x(std::vector<float>{1, 2, 3, -4, -5, -6}), w(std::vector<float>{1, 0, 0, 1, 1, 1});
    Dev b(std::vector<float>{0.5f, -10.f}), y(4), z(4);
    HIPBackend::linearBiasAct(x.p, w.p, b.p, y.p, 2, 3, 2, 1);
    auto h = y.host();
    EXPECT_NEAR(h[0], 4.5, 0); EXPECT_NEAR(h[1], 0, 0); EXPECT_NEAR(h[2], 0, 0); EXPECT_NEAR(h[3], 0, 0);
    HIPBackend::linearBiasAct(x.p, w.p, b.p, z.p, 2, 3, 2, 0);   // no activation
    auto g = z.host();
    EXPECT_NEAR(g[0], 4.5, 0); EXPECT_NEAR(g[1], -5, 0); EXPECT_NEAR(g[2], -9.5, 0); EXPECT_NEAR(g[3], -21, 0);
    std::printf("LinearBiasAct done\n");
}

static void testLinearBackward() {
    // x = [[1 2 0], [3 0 4]] (a ReLU output: batch 2, in 3), gY = [[1 -1], [2 0.5]] (out 2),
    // W = [[1 0], [0 1], [1 1]] (in 3 x out 2): dW = x^T gY, db = column sums of gY,
    // gX = (x > 0 ? gY W^T : 0)
    Dev x(std::vector<float>{1, 2, 0, 3, 0, 4}), g(std::vector<float>{1, -1, 2, 0.5f});
    Dev w(std::vector<float>{1, 0, 0, 1, 1, 1}), gw(6), gb(2), gx(6);
    HIPBackend::linearBackward(x.p, g.p, w.p, x.p, gw.p, gb.p, gx.p, 2, 3, 2);
    const float wantW[6] = {7, 0.5f, 2, -2, 8, 2}, wantX[6] = {1, -1, 0, 2, 0, 2.5f};
    auto hw = gw.host(), hb = gb.host(), hx = gx.host();
    for (int i = 0; i < 6; ++i) {
        EXPECT_NEAR(hw[i], wantW[i], 0);
        EXPECT_NEAR(hx[i], wantX[i], 0);
    }
    EXPECT_NEAR(hb[0], 3, 0); EXPECT_NEAR(hb[1], -0.5, 0);
    std::printf("LinearBackward done\n");
}

// MultiHeadAttention::forward's GPU branch (vit.ixx:163-187) written as the engine writes it,
// with HIPBackend in CUDABackend's place: qkvSplitHeads, tensorTranspose2dBatched (transpose
// per head), tensorBatchedMatmul, tensorSoftmaxLastDim (softmax), tensorBatchedMatmul,
// mergeHeads. Known answers for the split and merge; the chain equals HIPBackend::attention.
static void testVitBranchAndSum() {
    const int B = 2, S = 3, H = 2, D = 4, Dm = H * D, BH = B * H;
    std::vector<float> qkvH(B * S * 3 * Dm);
    for (size_t i = 0; i < qkvH.size(); ++i) qkvH[i] = 0.01f * (float)((i * 37) % 101) - 0.5f;
    Dev qkv(qkvH), q(BH * S * D), k(BH * S * D), v(BH * S * D);
    const float scale = 0.5f;   // 1 / sqrt(D)
    HIPBackend::qkvSplitHeads(qkv.p, q.p, k.p, v.p, B, S, H, D, scale);
    auto hq = q.host(), hk = k.host(), hv = v.host();
    for (int n = 0; n < B; ++n)
        for (int s = 0; s < S; ++s)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    const size_t o = (((size_t)n * H + h) * S + s) * D + d, r = ((size_t)n * S + s) * 3 * Dm;
                    EXPECT_NEAR(hq[o], qkvH[r + h * D + d] * scale, 0);
                    EXPECT_NEAR(hk[o], qkvH[r + Dm + h * D + d], 0);
                    EXPECT_NEAR(hv[o], qkvH[r + 2 * Dm + h * D + d], 0);
                }
    Dev kT(BH * D * S), scores(BH * S * S), attnW(BH * S * S), ctx(BH * S * D), outFlat(B * S * Dm);
    for (int b = 0; b < BH; ++b) HIPBackend::transpose(k.p + b * S * D, kT.p + b * S * D, S, D);
    HIPBackend::batchedMatmul(q.p, kT.p, scores.p, BH, S, D, S);
    HIPBackend::softmax(scores.p, attnW.p, BH * S, S);
    HIPBackend::batchedMatmul(attnW.p, v.p, ctx.p, BH, S, S, D);
    HIPBackend::mergeHeads(ctx.p, outFlat.p, B, S, H, D);
    Dev fused(B * S * Dm);
    HIPBackend::attention(qkv.p, fused.p, B, S, H, D, scale);
    auto ho = outFlat.host(), hf = fused.host(), hc = ctx.host();
    for (size_t i = 0; i < ho.size(); ++i) EXPECT_NEAR(hf[i], ho[i], 1e-6);
    for (int n = 0; n < B; ++n)   // merge is the inverse map of the split's
        for (int s = 0; s < S; ++s)
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d)
                    EXPECT_NEAR(ho[((size_t)n * S + s) * Dm + h * D + d], hc[(((size_t)n * H + h) * S + s) * D + d], 0);
    // tensorSum's GPU branch (tensor_ops.ixx:413-417): the sum lands on the device
    // (integer values whose every partial sum stays below 2^24, so any order is exact)
    std::vector<float> ramp(10000);
    for (int i = 0; i < 10000; ++i) ramp[i] = (float)(i % 100 + 1);
    Dev r(ramp), res(1);
    HIPBackend::sum(r.p, res.p, 10000);
    EXPECT_NEAR(res.host()[0], 505000.0, 0);
    HIPBackend::mean(r.p, res.p, 100);
    EXPECT_NEAR(res.host()[0], 50.5, 0);
    EXPECT_NEAR(HIPBackend::sum(r.p, (size_t)100), 5050.0, 0);
    std::printf("VitBranchAndSum done\n");
}

// EngineBridge's recovery call (EngineBridge.cpp:4047): the library comes back on the next call.
static void testForceReset() {
    HIPBackend::forceReset();
    Dev a(std::vector<float>{1, 2, 3, 4}), b(std::vector<float>{5, 6, 7, 8}), c(4);
    HIPBackend::matmul(a.p, b.p, c.p, 2, 2, 2);
    auto h = c.host();
    EXPECT_NEAR(h[0], 19, 0); EXPECT_NEAR(h[3], 50, 0);
    std::printf("ForceReset done\n");
}

int main() {
    try {
        HIPBackend::init(0);
        testMatmul2D();
        testMatmulNonSquare();
        testBatchedMatmulForward();
        testLinearZeroInput();
        testLinearBiasAct();
        testLinearBackward();
        testConvAllOnes();
        testReluAndErrors();
        testTrainingPieces();
        testVitBranchAndSum();
        testForceReset();
        HIPBackend::synchronize();
    } catch (const std::exception& e) {
        std::printf("FAIL: exception %s\n", e.what());
        return 2;
    }
    std::printf(g_fail ? "FAILED %d checks\n" : "ALL PASSED\n", g_fail);
    return g_fail ? 1 : 0;
}
