// infer.hip — a device-resident ResNet-18 classifier and the batch inference
// pipeline around it: the counterpart of EngineBridge::inferBatch
// (src/engine/bridge/EngineBridge.cpp:3525-3772) for classification models on
// this backend.
//
// The reference packs each batch (at most 32 images) on the host, normalises
// it there (normalizeImage, om.engine.data_pipeline.ixx:744-803), uploads it
// with a blocking copy, runs the forward, copies the logits back and applies
// softmax / argmax / the confidence threshold per image. Here:
//   * parameters and activations stay resident in device memory (allocated
//     once, sized for the largest batch);
//   * each batch is packed into one of two page-locked staging slots and
//     uploaded on the transfer stream while the previous batch computes; the
//     compute stream waits on an event, not on the host;
//   * normalisation is a kernel on the uploaded batch; every conv runs with
//     its BatchNorm (running statistics) and ReLU — and, for the second conv
//     of a block, the shortcut — fused in the epilogue;
//   * only the logits come back (to a page-locked slot); softmax, argmax and
//     the threshold run on the host exactly as the reference writes them.
#include "omhip_internal.hpp"
#include "conv.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

namespace omhip {
namespace {

constexpr float kBnEps = 1e-5f;
constexpr int kMaxBatch = 32;   // EngineBridge::inferBatch clamps the batch to [1, 32]

// (x - mean[p]) * invStd[p], p = min(c, 2) for 3+ channels, 0 otherwise
// (om.engine.data_pipeline.ixx:770-803).
__global__ void normalize_kernel(float* __restrict__ x, long long total, int C, int HW, float m0, float m1, float m2,
                                 float i0, float i1, float i2) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int c = (int)((i / HW) % C);
        const int p = C >= 3 ? min(c, 2) : 0;
        const float m = p == 0 ? m0 : (p == 1 ? m1 : m2);
        const float is = p == 0 ? i0 : (p == 1 ? i1 : i2);
        x[i] = (x[i] - m) * is;
    }
}

struct Conv {
    int cin, h, cout, k, s, p;
    size_t w, bn;   // float offsets of the weight and of gamma (beta, mean, var follow)
};

struct Block {
    int conv1, conv2, ds;   // indices into convs; ds = -1 without downsample
    int cin, cout, s, h;
};

struct Net {
    int nc = 0, maxBatch = 0;
    float* params = nullptr;   // device copy of the flat parameter array
    std::vector<Conv> convs;
    std::vector<Block> blocks;
    size_t fcW = 0, fcB = 0;
    // device activations
    float* in[2] = {nullptr, nullptr};
    float* a0 = nullptr;   // stem output [B,64,112,112]
    float* act[3] = {nullptr, nullptr, nullptr};   // block ping-pong + conv1 output
    float* sc = nullptr;   // downsample output
    float* pooled = nullptr;
    float* logits = nullptr;
    // page-locked host staging and the pipeline events
    float* hIn[2] = {nullptr, nullptr};
    float* hLogits[2] = {nullptr, nullptr};
    hipEvent_t evUp[2] = {nullptr, nullptr};
    hipEvent_t evDone[2] = {nullptr, nullptr};

    ~Net() {
        for (int k = 0; k < 2; ++k) {
            if (evUp[k]) (void)hipEventDestroy(evUp[k]);
            if (evDone[k]) (void)hipEventDestroy(evDone[k]);
            if (hIn[k]) (void)omHipFreeHost(hIn[k]);
            if (hLogits[k]) (void)omHipFreeHost(hLogits[k]);
            if (in[k]) (void)omHipFree(in[k]);
        }
        for (float* p : {params, a0, act[0], act[1], act[2], sc, pooled, logits})
            if (p) (void)omHipFree(p);
    }
};

// Parameter layout (floats): for each conv in network order — stem, then per
// BasicBlock conv1, conv2 and (first block of stages 2-4) the 1x1 downsample —
// weight [Cout][Cin][K][K], BN gamma, beta, running mean, running var [Cout];
// then the FC weight [512][nClasses] (Linear layout [in, out]) and bias [nClasses].
size_t buildLayout(Net& n) {
    size_t off = 0;
    auto addConv = [&](int cin, int h, int cout, int k, int s, int p) {
        Conv c{cin, h, cout, k, s, p, off, 0};
        off += (size_t)cout * cin * k * k;
        c.bn = off;
        off += 4 * (size_t)cout;
        n.convs.push_back(c);
        return (int)n.convs.size() - 1;
    };
    addConv(3, 224, 64, 7, 2, 3);
    const int stages[4][3] = {{64, 64, 1}, {64, 128, 2}, {128, 256, 2}, {256, 512, 2}};
    int hw = 56;
    for (const auto& st : stages) {
        for (int b = 0; b < 2; ++b) {
            const int ci = b == 0 ? st[0] : st[1];
            const int co = st[1];
            const int s = b == 0 ? st[2] : 1;
            const int o = (hw + 2 - 3) / s + 1;
            Block blk{};
            blk.cin = ci; blk.cout = co; blk.s = s; blk.h = hw;
            blk.conv1 = addConv(ci, hw, co, 3, s, 1);
            blk.conv2 = addConv(co, o, co, 3, 1, 1);
            blk.ds = (b == 0 && (s != 1 || ci != co)) ? addConv(ci, hw, co, 1, s, 0) : -1;
            n.blocks.push_back(blk);
            hw = o;
        }
    }
    n.fcW = off;
    off += (size_t)512 * n.nc;
    n.fcB = off;
    off += (size_t)n.nc;
    return off;
}

int convBn(const char* name, const Net& n, const Conv& c, const float* x, const float* res, int act, float* out,
           int B) {
    const float* P = n.params;
    return conv2dFused(name, x, P + c.w, nullptr, P + c.bn, P + c.bn + c.cout, P + c.bn + 2 * c.cout,
                       P + c.bn + 3 * c.cout, kBnEps, res, act, out, B, c.cin, c.h, c.h, c.cout, c.k, c.k, c.s, c.p);
}

// Inference forward of B images at x (device, normalised) into n.logits.
int forward(Net& n, const float* x, int B) {
    const char* name = "omHipResNet18Forward";
    if (convBn(name, n, n.convs[0], x, nullptr, 1, n.a0, B)) return -1;
    float* cur = n.act[0];
    float* nxt = n.act[1];
    float* t1 = n.act[2];
    if (omHipMaxPool2d(n.a0, cur, nullptr, B, 64, 112, 112, 3, 3, 2, 2, 1, 1)) return -1;
    for (const Block& b : n.blocks) {
        if (convBn(name, n, n.convs[b.conv1], cur, nullptr, 1, t1, B)) return -1;
        const float* sc = cur;
        if (b.ds >= 0) {
            if (convBn(name, n, n.convs[b.ds], cur, nullptr, 0, n.sc, B)) return -1;
            sc = n.sc;
        }
        if (convBn(name, n, n.convs[b.conv2], t1, sc, 1, nxt, B)) return -1;
        std::swap(cur, nxt);
    }
    if (omHipAdaptiveAvgPool2d(cur, n.pooled, B, 512, 7, 7, 1, 1)) return -1;
    if (omHipMatmul(n.pooled, n.params + n.fcW, n.logits, B, 512, n.nc)) return -1;
    return omHipAddBias(n.logits, n.params + n.fcB, n.logits, B, n.nc, 1);
}

// Copies a batch into its page-locked slot with up to 8 host threads: one
// thread's memcpy (about 10 GB/s) would take longer than the GPU forward of
// the previous batch it is meant to hide behind.
void packBatch(float* dst, const float* src, size_t bytes) {
    const size_t kMinPerThread = (size_t)4 << 20;
    const int nt = (int)std::min<size_t>(8, std::max<size_t>(1, bytes / kMinPerThread));
    if (nt == 1) {
        std::memcpy(dst, src, bytes);
        return;
    }
    const size_t per = (bytes / nt + 63) / 64 * 64;
    std::vector<std::thread> pool;
    for (int t = 1; t < nt; ++t) {
        const size_t b0 = std::min(bytes, per * t), b1 = std::min(bytes, per * (t + 1));
        if (b1 > b0)
            pool.emplace_back([=] {
                std::memcpy(reinterpret_cast<char*>(dst) + b0, reinterpret_cast<const char*>(src) + b0, b1 - b0);
            });
    }
    std::memcpy(dst, src, std::min(bytes, per));
    for (auto& th : pool) th.join();
}

// EngineBridge.cpp:3733-3762: stable softmax, argmax (strict >), confidence threshold.
void classify(const float* logits, int nc, float threshold, int* cls, float* conf, float* probsOut) {
    std::vector<float> probs(nc);
    const float fMax = *std::max_element(logits, logits + nc);
    float fSum = 0.0f;
    for (int c = 0; c < nc; ++c) {
        probs[c] = std::exp(logits[c] - fMax);
        fSum += probs[c];
    }
    int nBest = 0;
    float fBestP = 0.0f;
    for (int c = 0; c < nc; ++c) {
        probs[c] /= std::max(fSum, 1e-8f);
        if (probs[c] > fBestP) {
            fBestP = probs[c];
            nBest = c;
        }
    }
    *cls = fBestP < threshold ? -1 : nBest;
    *conf = fBestP;
    if (probsOut) std::memcpy(probsOut, probs.data(), sizeof(float) * nc);
}

}  // namespace
}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipResNet18Create(const float* pParams, long long nParamFloats, int nClasses, int nMaxBatch, void** ppNet) {
    clearError();
    if (!ppNet) return fail("omHipResNet18Create: null output");
    *ppNet = nullptr;
    if (!pParams || nClasses <= 0 || nMaxBatch <= 0) return fail("omHipResNet18Create: invalid arguments");
    auto n = std::make_unique<Net>();
    n->nc = nClasses;
    n->maxBatch = std::min(nMaxBatch, kMaxBatch);
    const size_t need = buildLayout(*n);
    if ((size_t)nParamFloats != need)
        return fail("omHipResNet18Create: %lld parameter floats given, the layout holds %zu", nParamFloats, need);
    const int B = n->maxBatch;
    auto alloc = [](float** p, size_t floats) { return omHipMalloc(reinterpret_cast<void**>(p), floats * 4); };
    if (alloc(&n->params, need) || omHipCopyH2D(n->params, pParams, need * 4)) return -1;
    const size_t inF = (size_t)B * 3 * 224 * 224;
    const size_t actF = (size_t)B * 64 * 56 * 56;   // the largest block activation
    if (alloc(&n->in[0], inF) || alloc(&n->in[1], inF) || alloc(&n->a0, (size_t)B * 64 * 112 * 112) ||
        alloc(&n->act[0], actF) || alloc(&n->act[1], actF) || alloc(&n->act[2], actF) || alloc(&n->sc, actF) ||
        alloc(&n->pooled, (size_t)B * 512) || alloc(&n->logits, (size_t)B * nClasses))
        return -1;
    for (int k = 0; k < 2; ++k) {
        if (omHipMallocHost(reinterpret_cast<void**>(&n->hIn[k]), inF * 4) ||
            omHipMallocHost(reinterpret_cast<void**>(&n->hLogits[k]), (size_t)B * nClasses * 4))
            return -1;
        OMHIP_CHECK(hipEventCreateWithFlags(&n->evUp[k], hipEventDisableTiming));
        OMHIP_CHECK(hipEventCreateWithFlags(&n->evDone[k], hipEventDisableTiming));
    }
    *ppNet = n.release();
    return 0;
}

int omHipResNet18Destroy(void* pNet) {
    clearError();
    if (!pNet) return 0;
    Net* n = static_cast<Net*>(pNet);
    (void)hipStreamSynchronize(stream());
    (void)omHipSyncTransferStream();
    delete n;
    return 0;
}

int omHipResNet18Forward(void* pNet, const float* pInput, float* pLogits, int nBatch) {
    clearError();
    if (!pNet || !pInput || !pLogits) return fail("omHipResNet18Forward: null pointer");
    Net& n = *static_cast<Net*>(pNet);
    if (nBatch <= 0 || nBatch > n.maxBatch) return fail("omHipResNet18Forward: batch %d outside [1, %d]", nBatch,
                                                        n.maxBatch);
    if (forward(n, pInput, nBatch)) return -1;
    return omHipCopyD2D(pLogits, n.logits, (size_t)nBatch * n.nc * 4);
}

int omHipResNet18InferBatch(void* pNet, const float* pImages, int nImages, int nC, int nH, int nW, int nBatchSize,
                            int nNormPreset, float fConfThreshold, int* pClasses, float* pConfidences,
                            float* pProbs) {
    clearError();
    const char* name = "omHipResNet18InferBatch";
    if (!pNet || !pClasses || !pConfidences) return fail("%s: null pointer", name);
    if (nImages <= 0) return 0;
    if (!pImages) return fail("%s: null images", name);
    if (nC != 3 || nH != 224 || nW != 224) return fail("%s: the network takes 3x224x224 images", name);
    if (nNormPreset != 0 && nNormPreset != 1) return fail("%s: unknown normalisation preset %d", name, nNormPreset);
    Net& n = *static_cast<Net*>(pNet);
    const int B = std::max(1, std::min({nBatchSize, kMaxBatch, n.maxBatch}));
    const size_t img = (size_t)nC * nH * nW;
    hipStream_t xfer = transferStream();
    if (!xfer) return -1;
    // ImageNet preset (normalizeImage): invStd = 1 / std, std clamped at 1e-7
    const float mean[3] = {0.485f, 0.456f, 0.406f};
    float inv[3];
    const float sd[3] = {0.229f, 0.224f, 0.225f};
    for (int c = 0; c < 3; ++c) inv[c] = 1.0f / std::max(sd[c], 1e-7f);

    const int nBatches = (nImages + B - 1) / B;
    auto finish = [&](int b) -> int {
        // results of batch b are in hLogits[b & 1] once evDone fired
        const int k = b & 1;
        OMHIP_CHECK(hipEventSynchronize(n.evDone[k]));
        const int s0 = b * B, cnt = std::min(B, nImages - s0);
        for (int i = 0; i < cnt; ++i)
            classify(n.hLogits[k] + (size_t)i * n.nc, n.nc, fConfThreshold, pClasses + s0 + i,
                     pConfidences + s0 + i, pProbs ? pProbs + (size_t)(s0 + i) * n.nc : nullptr);
        return 0;
    };
    for (int b = 0; b < nBatches; ++b) {
        const int k = b & 1;
        if (b >= 2 && finish(b - 2)) return -1;   // frees slot k
        const int s0 = b * B, cnt = std::min(B, nImages - s0);
        packBatch(n.hIn[k], pImages + (size_t)s0 * img, (size_t)cnt * img * 4);
        OMHIP_CHECK(hipMemcpyAsync(n.in[k], n.hIn[k], (size_t)cnt * img * 4, hipMemcpyHostToDevice, xfer));
        OMHIP_CHECK(hipEventRecord(n.evUp[k], xfer));
        OMHIP_CHECK(hipStreamWaitEvent(stream(), n.evUp[k], 0));
        if (nNormPreset == 1) {
            const long long total = (long long)cnt * img;
            const int grid = (int)std::min<long long>((total + 255) / 256, (long long)cuCount() * 16);
            hipLaunchKernelGGL(normalize_kernel, dim3(grid), dim3(256), 0, stream(), n.in[k], total, nC, nH * nW,
                               mean[0], mean[1], mean[2], inv[0], inv[1], inv[2]);
            OMHIP_CHECK_LAUNCH();
        }
        if (forward(n, n.in[k], cnt)) return -1;
        OMHIP_CHECK(hipMemcpyAsync(n.hLogits[k], n.logits, (size_t)cnt * n.nc * 4, hipMemcpyDeviceToHost, stream()));
        OMHIP_CHECK(hipEventRecord(n.evDone[k], stream()));
    }
    for (int b = std::max(0, nBatches - 2); b < nBatches; ++b)
        if (finish(b)) return -1;
    return 0;
}

}  // extern "C"
