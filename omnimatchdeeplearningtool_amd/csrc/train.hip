// train.hip — the training half of the conv / BatchNorm path:
// conv2d input and weight gradients, BatchNorm2d training statistics and its
// backward pass.
//
// Reference: CPUBackend::conv2dBackwardInput / conv2dBackwardWeight
// (src/hal/om.hal.cpu_backend.ixx:666-772), batchNorm2d's training branch
// (:796-822) and batchNorm2dBackward (:847-890); C ABI counterparts
// omCudaConv2dBackwardInput / Weight and omCudaBatchNorm2dBackward
// (src/cuda/cuda_kernels.cuh:295-316).
//
// Input gradient. For stride 1 it is itself a stride-1 convolution of the
// output gradient with the weights swapped over (Cout, Cin) and flipped in
// (kh, kw), padded by K-1-pad: it runs on the forward implicit-GEMM kernel.
// A stride-s gradient splits into s*s output phases (ih mod s, iw mod s),
// each again a stride-1 convolution of the output gradient with a flipped
// sub-kernel, written straight to its pixels of the input gradient — no
// column buffer, no col2im, no work on taps that cannot reach a pixel.
//
// Weight gradient: an implicit GEMM over every output pixel of the batch
// (conv_wgrad.hip), no column matrix. Bias gradient and the BatchNorm
// reductions are per-channel sums over N x H x W: each (channel, part)
// workgroup sums a contiguous range of images in a fixed order, a second
// kernel adds the parts in order — deterministic.
#include "omhip_internal.hpp"
#include "conv.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

// ---- input gradient by output phase -------------------------------------------------
// For stride s, the input-gradient pixels with ih = a (mod s) receive only the
// taps kh = (a + p) (mod s): kh = r + s*j, oh = i + floor((a+p)/s) - j for
// ih = a + s*i. Over those pixels the gradient is a stride-1 correlation of
// gradOutput with the sub-kernel flipped in j (top pad KHa - 1 - floor((a+p)/s),
// possibly negative), and likewise in w. Stride 1 is the single phase (0, 0)
// with the whole flipped kernel and pad K - 1 - p.

// Taps k in [0, K) of phase a: k = (a + p) (mod s).
__host__ __device__ inline int phaseTaps(int K, int s, int p, int a) {
    const int r = (a + p) % s;
    return r < K ? (K - r + s - 1) / s : 0;
}
__host__ __device__ inline int phaseTapsBefore(int K, int s, int p, int a) {
    int n = 0;
    for (int b = 0; b < a; ++b) n += phaseTaps(K, s, p, b);
    return n;
}
// Offset (floats) of phase (a, b)'s sub-kernel in the phase-major buffer.
__host__ __device__ inline long long phaseOffset(int Cout, int Cin, int KH, int KW, int s, int p, int a, int b) {
    return (long long)Cin * Cout *
           ((long long)phaseTapsBefore(KH, s, p, a) * KW + (long long)phaseTaps(KH, s, p, a) * phaseTapsBefore(KW, s, p, b));
}

// Phase (a, b) sub-kernel: wf[ci][co][jf][lf] = W[co][ci][ra + s*(KHa-1-jf)][rb + s*(KWb-1-lf)].
// Every tap belongs to exactly one phase, so the sub-kernels tile a buffer of W's size.
__global__ void phase_flip_kernel(const float* __restrict__ w, float* __restrict__ wf, int Cout, int Cin, int KH,
                                  int KW, int s, int p) {
    const long long total = (long long)Cout * Cin * KH * KW;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const int kw = (int)(i % KW);
        const int kh = (int)((i / KW) % KH);
        const int ci = (int)((i / ((long long)KW * KH)) % Cin);
        const int co = (int)(i / ((long long)KW * KH * Cin));
        const int a = ((kh % s) - (p % s) + s) % s;
        const int b = ((kw % s) - (p % s) + s) % s;
        const int KHa = phaseTaps(KH, s, p, a), KWb = phaseTaps(KW, s, p, b);
        const int jf = KHa - 1 - kh / s, lf = KWb - 1 - kw / s;
        wf[phaseOffset(Cout, Cin, KH, KW, s, p, a, b) + (((long long)ci * Cout + co) * KHa + jf) * KWb + lf] = w[i];
    }
}

__global__ void zero_fill_kernel(float* __restrict__ y, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        y[i] = 0.f;
}

static int gridFor(long long n) {
    return (int)std::max<long long>(1, std::min<long long>((n + 255) / 256, (long long)cuCount() * 16));
}

// ---- per-channel reductions ------------------------------------------------------
// Parts per channel: enough (channel, part) workgroups to fill the chip, from
// the shape alone so the summation order does not depend on the device.
static int channelParts(int N, int C) { return std::max(1, std::min(N, (2048 + C - 1) / C)); }

template <int NV>
__device__ __forceinline__ void blockSum(float (&v)[NV], float* red) {
    // fixed-order tree over the 256 threads of the workgroup
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NV; ++k) red[k * 256 + tid] = v[k];
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s)
#pragma unroll
            for (int k = 0; k < NV; ++k) red[k * 256 + tid] += red[k * 256 + tid + s];
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = red[k * 256];
}

// MODE 0: sum x.  MODE 1: sum (x - mean)^2.  MODE 2: sum dy*xhat and sum dy,
// xhat = (x - mean) * invStd. part[(c*P + p)*2 + k].
template <int MODE>
__global__ __launch_bounds__(256) void chan_partial_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ invStd, float* __restrict__ part,
                                                           int N, int C, int HW, int P) {
    __shared__ float red[2 * 256];
    const int c = blockIdx.x, p = blockIdx.y;
    const int n0 = (int)((long long)p * N / P), n1 = (int)((long long)(p + 1) * N / P);
    const float m = MODE ? mean[c] : 0.f;
    const float is = MODE == 2 ? invStd[c] : 0.f;
    float v[2] = {0.f, 0.f};
    for (int n = n0; n < n1; ++n) {
        const long long base = ((long long)n * C + c) * HW;
        for (int s = threadIdx.x; s < HW; s += 256) {
            if constexpr (MODE == 0) {
                v[0] += x[base + s];
            } else if constexpr (MODE == 1) {
                const float d = x[base + s] - m;
                v[0] = __builtin_fmaf(d, d, v[0]);
            } else {
                const float g = dy[base + s];
                const float xh = (x[base + s] - m) * is;
                v[0] = __builtin_fmaf(g, xh, v[0]);
                v[1] += g;
            }
        }
    }
    blockSum<2>(v, red);
    if (threadIdx.x == 0) {
        part[((long long)c * P + p) * 2] = v[0];
        part[((long long)c * P + p) * 2 + 1] = v[1];
    }
}

// Sums the P parts of each channel in order; out0[c] = sum / divisor (and out1).
// The division is the reference's `sum /= count` (a true division; 1 leaves
// the sum unchanged).
__global__ void chan_finish_kernel(const float* __restrict__ part, float* out0, float* out1, int C, int P,
                                   float divisor, int accumulate) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    float a = 0.f, b = 0.f;
    for (int p = 0; p < P; ++p) {
        a += part[((long long)c * P + p) * 2];
        b += part[((long long)c * P + p) * 2 + 1];
    }
    if (out0) out0[c] = accumulate ? out0[c] + a / divisor : a / divisor;
    if (out1) out1[c] = accumulate ? out1[c] + b / divisor : b / divisor;
}

// Training statistics (cpu_backend.ixx:796-822): batch mean and biased
// variance are already in mean / var; saved stats and the running averages.
__global__ void bn_train_stats_kernel(const float* mean, const float* var, float* savedMean, float* savedInvStd,
                                      float* runMean, float* runVar, int C, float eps, float momentum) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    if (savedMean) savedMean[c] = mean[c];
    if (savedInvStd) savedInvStd[c] = 1.0f / sqrtf(var[c] + eps);
    runMean[c] = __builtin_fmaf(1.0f - momentum, runMean[c], momentum * mean[c]);
    runVar[c] = __builtin_fmaf(1.0f - momentum, runVar[c], momentum * var[c]);
}

// y = gamma*((x-mean)*invStd)+beta, invStd = 1/sqrt(var+eps) (cpu_backend.ixx:832-840).
__global__ void bn_apply_kernel(const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
                                const float* __restrict__ beta, const float* __restrict__ mean,
                                const float* __restrict__ var, int C, int HW, float eps, int plane0) {
    const int plane = plane0 + blockIdx.y;
    const int c = plane % C;
    const float mu = mean[c];
    const float inv = 1.0f / sqrtf(var[c] + eps);
    const float g = gamma[c], b = beta[c];
    const long long base = (long long)plane * HW;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < HW; i += gridDim.x * blockDim.x)
        y[base + i] = __builtin_fmaf(g, (x[base + i] - mu) * inv, b);
}

// dx = gamma*invStd*(1/cnt) * (cnt*dy - sum(dy) - xhat*sum(dy*xhat)) (cpu_backend.ixx:883-886),
// with the multiply-adds fused as the reference compiled by clang fuses them.
__global__ void bn_backward_apply_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                         const float* __restrict__ mean, const float* __restrict__ invStd,
                                         const float* __restrict__ gamma, const float* __restrict__ sumDyXh,
                                         const float* __restrict__ sumDy, float* __restrict__ dx, int C, int HW,
                                         float cnt, float invCnt, int plane0) {
    const int plane = plane0 + blockIdx.y;
    const int c = plane % C;
    const float m = mean[c], is = invStd[c], g = gamma[c];
    const float sg = sumDyXh[c], sb = sumDy[c];
    const float k = g * is * invCnt;
    const long long base = (long long)plane * HW;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < HW; i += gridDim.x * blockDim.x) {
        const float xh = (x[base + i] - m) * is;
        dx[base + i] = k * __builtin_fmaf(-xh, sg, __builtin_fmaf(cnt, dy[base + i], -sb));
    }
}

// Launches a per-plane kernel over N*C planes (grid.y <= 65535 per launch).
template <class F>
static int forPlanes(int planes, int HW, F launch) {
    const int bx = std::max(1, std::min((HW + 255) / 256, std::max(1, 4096 / std::max(1, planes))));
    for (int p0 = 0; p0 < planes; p0 += 65535) {
        const int cnt = std::min(65535, planes - p0);
        launch(dim3(bx, cnt), p0);
        OMHIP_CHECK_LAUNCH();
    }
    return 0;
}

// Per-channel sums into out0/out1 (divided by divisor): MODE as chan_partial_kernel.
template <int MODE>
static int channelSums(const float* x, const float* dy, const float* mean, const float* invStd, float* out0,
                       float* out1, int N, int C, int HW, float divisor, bool accumulate) {
    const int P = channelParts(N, C);
    float* part = static_cast<float*>(workspace((size_t)C * P * 2 * sizeof(float)));
    if (!part) return fail("channel reduction: no workspace");
    hipLaunchKernelGGL(chan_partial_kernel<MODE>, dim3(C, P), dim3(256), 0, stream(), x, dy, mean, invStd, part, N, C,
                       HW, P);
    OMHIP_CHECK_LAUNCH();
    hipLaunchKernelGGL(chan_finish_kernel, dim3((C + 255) / 256), dim3(256), 0, stream(), part, out0, out1, C, P,
                       divisor, accumulate ? 1 : 0);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// Device scratch for a few per-channel vectors, freed by the caller.
struct ChannelScratch {
    float* p = nullptr;
    ~ChannelScratch() {
        if (p) (void)omHipFree(p);
    }
    float* get(int C, int k) {
        if (!p && omHipMalloc(reinterpret_cast<void**>(&p), (size_t)C * k * sizeof(float)) != 0) return nullptr;
        return p;
    }
};

int batchNorm2dTrain(const float* x, float* y, const float* gamma, const float* beta, float* runMean, float* runVar,
                     float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps, float momentum) {
    const int HW = H * W;
    const float cnt = (float)((long long)N * HW);
    ChannelScratch scratch;
    float* st = scratch.get(C, 2);
    if (!st) return -1;
    float* mean = st;
    float* var = st + C;
    // two passes, as the reference: mean = sum(x)/cnt, var = sum((x-mean)^2)/cnt
    if (channelSums<0>(x, nullptr, nullptr, nullptr, mean, nullptr, N, C, HW, cnt, false)) return -1;
    if (channelSums<1>(x, nullptr, mean, nullptr, var, nullptr, N, C, HW, cnt, false)) return -1;
    hipLaunchKernelGGL(bn_train_stats_kernel, dim3((C + 255) / 256), dim3(256), 0, stream(), mean, var, savedMean,
                       savedInvStd, runMean, runVar, C, eps, momentum);
    OMHIP_CHECK_LAUNCH();
    return forPlanes(N * C, HW, [&](dim3 g, int p0) {
        hipLaunchKernelGGL(bn_apply_kernel, g, dim3(256), 0, stream(), x, y, gamma, beta, mean, var, C, HW, eps, p0);
    });
}

static int validateConvGrad(const char* name, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride,
                            int pad, int& Ho, int& Wo) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0)
        return fail("%s: invalid geometry", name);
    Ho = (H + 2 * pad - KH) / stride + 1;
    Wo = (W + 2 * pad - KW) / stride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("%s: kernel larger than the padded input", name);
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipConv2dBackwardInput(const float* pGradOutput, const float* pWeight, float* pGradInput, int nBatch,
                             int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    clearError();
    const char* name = "omHipConv2dBackwardInput";
    int Ho, Wo;
    if (validateConvGrad(name, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad, Ho, Wo)) return -1;
    if (!pGradOutput || !pWeight || !pGradInput) return fail("%s: null pointer", name);
    const int s = nStride, p = nPad;
    const long long wsz = (long long)nCout * nCin * nKH * nKW;
    // Pixels of a phase without taps (stride > kernel) get no contribution.
    bool emptyPhase = false;
    for (int a = 0; a < std::min(s, nH); ++a)
        for (int b = 0; b < std::min(s, nW); ++b)
            if (phaseTaps(nKH, s, p, a) == 0 || phaseTaps(nKW, s, p, b) == 0) emptyPhase = true;
    if (emptyPhase) {
        const long long n = (long long)nBatch * nCin * nH * nW;
        hipLaunchKernelGGL(zero_fill_kernel, dim3(gridFor(n)), dim3(256), 0, stream(), pGradInput, n);
        OMHIP_CHECK_LAUNCH();
    }
    float* wf = nullptr;
    if (omHipMalloc(reinterpret_cast<void**>(&wf), (size_t)wsz * sizeof(float))) return -1;
    hipLaunchKernelGGL(phase_flip_kernel, dim3(gridFor(wsz)), dim3(256), 0, stream(), pWeight, wf, nCout, nCin, nKH,
                       nKW, s, p);
    int rc = hipGetLastError() == hipSuccess ? 0 : fail("%s: flip launch failed", name);
    for (int a = 0; a < std::min(s, nH) && !rc; ++a) {
        const int KHa = phaseTaps(nKH, s, p, a);
        if (KHa == 0) continue;
        const int Hp = (nH - a + s - 1) / s;
        for (int b = 0; b < std::min(s, nW) && !rc; ++b) {
            const int KWb = phaseTaps(nKW, s, p, b);
            if (KWb == 0) continue;
            const int Wp = (nW - b + s - 1) / s;
            rc = conv2dToGrid(name, pGradOutput, wf + phaseOffset(nCout, nCin, nKH, nKW, s, p, a, b), pGradInput,
                              nBatch, nCout, Ho, Wo, nCin, KHa, KWb, KHa - 1 - (a + p) / s, KWb - 1 - (b + p) / s, Hp,
                              Wp, nH, nW, s, a, b);
        }
    }
    (void)omHipFree(wf);   // stream-ordered reuse: later work on the stream runs after the convs
    return rc;
}

int omHipConv2dBackwardWeight(const float* pInput, const float* pGradOutput, float* pGradWeight, float* pGradBias,
                              int nBatch, int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride,
                              int nPad) {
    clearError();
    const char* name = "omHipConv2dBackwardWeight";
    int Ho, Wo;
    if (validateConvGrad(name, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad, Ho, Wo)) return -1;
    if (!pInput || !pGradOutput || !pGradWeight) return fail("%s: null pointer", name);
    if (conv2dWeightGrad(name, pInput, pGradOutput, pGradWeight, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride,
                         nPad))
        return -1;
    const long long HWo = (long long)Ho * Wo;
    if (pGradBias) return channelSums<0>(pGradOutput, nullptr, nullptr, nullptr, pGradBias, nullptr, nBatch, nCout,
                                         (int)HWo, 1.0f, false);
    return 0;
}

int omHipBatchNorm2dBackward(const float* pGradOutput, const float* pInput, const float* pMean, const float* pInvStd,
                             const float* pGamma, float* pGradInput, float* pGradGamma, float* pGradBeta, int nBatch,
                             int nChannels, int nH, int nW, float fEps) {
    clearError();
    (void)fEps;   // the saved inverse standard deviation already carries eps
    if (nBatch <= 0 || nChannels <= 0 || nH <= 0 || nW <= 0) return 0;
    if (!pGradOutput || !pInput || !pMean || !pInvStd || !pGamma || !pGradInput)
        return fail("omHipBatchNorm2dBackward: null pointer");
    const int C = nChannels, HW = nH * nW;
    ChannelScratch scratch;
    float* st = nullptr;
    float* sg = pGradGamma;
    float* sb = pGradBeta;
    if (!sg || !sb) {
        st = scratch.get(C, 2);
        if (!st) return -1;
        if (!sg) sg = st;
        if (!sb) sb = st + C;
    }
    if (channelSums<2>(pInput, pGradOutput, pMean, pInvStd, sg, sb, nBatch, C, HW, 1.0f, false)) return -1;
    const long long cnt = (long long)nBatch * HW;
    const float fcnt = (float)cnt;
    const float invCnt = 1.0f / fcnt;
    return forPlanes(nBatch * C, HW, [&](dim3 g, int p0) {
        hipLaunchKernelGGL(bn_backward_apply_kernel, g, dim3(256), 0, stream(), pGradOutput, pInput, pMean, pInvStd,
                           pGamma, sg, sb, pGradInput, C, HW, fcnt, invCnt, p0);
    });
}

}  // extern "C"
