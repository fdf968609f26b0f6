// loss.hip — the loss end of a Linear network's training step and the Linear
// bias gradient: softmax over the last axis, the cross-entropy of softmax
// outputs against one-hot targets, their joint gradient, and the bias
// gradient (sum of the output gradient over every axis but the channel).
//
// Reference (CPUBackend, the parity target): softmax cpu_backend.ixx:352-370,
// crossEntropy :375-388, crossEntropySoftmaxBackward :393-410; the bias
// gradient of AddBiasBackward autograd.ixx:428-433. The GPU path the
// reference calls: omCudaSoftmax / omCudaCrossEntropy /
// omCudaSoftmaxCrossEntropyBackward / omCudaAddBiasBackward
// (cuda_kernels.cuh:122, :399, :288, :348).
//
// Rows are small (a batch of class scores), so every kernel is latency- and
// launch-bound, not HBM-bound: a wave owns a row, lanes stride its classes,
// and every reduction has a fixed order (butterfly within a wave, waves and
// row contributions added in index order), so results do not depend on the
// device or the launch.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

namespace {

__device__ __forceinline__ float waveSum(float v) {
    // fixed butterfly: every lane ends with the same sum in the same order
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// max with the reference's semantics: the scan keeps a candidate unless an
// element is strictly greater, so NaN elements are skipped (and a NaN first
// element is kept, handled by the caller).
__device__ __forceinline__ float gtMax(float m, float v) { return v > m ? v : m; }

__device__ __forceinline__ float waveMax(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = gtMax(v, __shfl_xor(v, off, 64));
    return v;
}

// Row maximum as the reference's scan computes it (cpu_backend.ixx:356-358):
// the first element when it is NaN, else the largest non-NaN element.
__device__ __forceinline__ float rowMax(const float* r, int cols, int lane) {
    float m = -INFINITY;
    for (int j = lane; j < cols; j += 64) m = gtMax(m, r[j]);
    m = waveMax(m);
    const float r0 = r[0];
    return r0 != r0 ? r0 : gtMax(r0, m);
}

// Softmax of one row by one wave: exp(x - max) stored to o, wave sum, then
// o /= sum (each lane rereads only what it wrote).
__device__ __forceinline__ void softmaxRow(const float* r, float* o, int cols, int lane) {
    const float m = rowMax(r, cols, lane);
    float s = 0.f;
    for (int j = lane; j < cols; j += 64) {
        const float e = expf(r[j] - m);
        o[j] = e;
        s += e;
    }
    s = waveSum(s);
    for (int j = lane; j < cols; j += 64) o[j] = o[j] / s;
}

// One row's cross-entropy terms (cpu_backend.ixx:378-384): -log(max(p, 1e-7))
// where the target exceeds 0.5, summed over the row by the wave.
__device__ __forceinline__ float rowLoss(const float* p, const float* t, int cols, int lane) {
    float acc = 0.f;
    for (int j = lane; j < cols; j += 64) {
        if (t[j] > 0.5f) {
            float q = p[j];
            if (q < 1e-7f) q = 1e-7f;
            acc -= logf(q);
        }
    }
    return waveSum(acc);
}

constexpr int kLossWaves = 16;   // the loss kernels run as one workgroup of 16 waves

// Adds the 16 waves' loss partials in wave order and writes sum / batch.
__device__ __forceinline__ void finishLoss(float waveAcc, float* result, int rows, float* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = waveAcc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float tot = 0.f;
        for (int w = 0; w < kLossWaves; ++w) tot += lds[w];
        result[0] = tot / (float)rows;
    }
}

}  // namespace

__global__ void __launch_bounds__(256) softmax_rows_kernel(const float* in, float* out, int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    softmaxRow(in + row * cols, out + row * cols, cols, lane);
}

// Wave w takes rows w, w+16, ...; its partial adds the row sums in row order.
__global__ void __launch_bounds__(1024) cross_entropy_kernel(const float* pred, const float* tgt, float* result,
                                                             int rows, int cols) {
    __shared__ float lds[kLossWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r = wave; r < rows; r += kLossWaves) acc += rowLoss(pred + r * cols, tgt + r * cols, cols, lane);
    finishLoss(acc, result, rows, lds);
}

__global__ void softmax_ce_backward_kernel(const float* s, const float* t, float* g, long long n, float scale) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        g[i] = (s[i] - t[i]) * scale;
}

// softmax -> crossEntropy -> crossEntropySoftmaxBackward in one workgroup, with
// the same per-row code and loss order as the three kernels above (so each
// output is bit-identical to theirs). Any output pointer may be null; the
// softmax row is written to `prob` when given, else to `grad` (and then
// overwritten by the gradient), else kept in the scratch row `rowBuf`.
__global__ void __launch_bounds__(1024) softmax_ce_fused_kernel(const float* logits, const float* tgt, float* prob,
                                                                float* loss, float* grad, float* rowBuf, int rows,
                                                                int cols, float scale) {
    __shared__ float lds[kLossWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r = wave; r < rows; r += kLossWaves) {
        float* p = prob ? prob + r * cols : (grad ? grad + r * cols : rowBuf + (long long)wave * cols);
        const float* t = tgt + r * cols;
        softmaxRow(logits + r * cols, p, cols, lane);
        if (loss) acc += rowLoss(p, t, cols, lane);
        if (grad)
            for (int j = lane; j < cols; j += 64) grad[r * cols + j] = (p[j] - t[j]) * scale;
    }
    if (loss) finishLoss(acc, loss, rows, lds);
}

// The same fused pass for rows of at most 64 * CPL classes with the row in
// registers: a wave loads RB rows at once (logits and targets, lane l holding
// classes l, l+64, ...), then each row runs the same operations in the same
// order as softmaxRow / rowLoss / the gradient above — only the values stay in
// registers instead of being written and read back — so every output is
// bit-identical to the three kernels'.
template <int CPL>
__global__ void __launch_bounds__(1024) softmax_ce_fused_reg_kernel(const float* logits, const float* tgt, float* prob,
                                                                    float* loss, float* grad, int rows, int cols,
                                                                    float scale) {
    __shared__ float lds[kLossWaves];
    constexpr int RB = 8;   // rows of a wave whose loads are in flight together
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r0 = wave; r0 < rows; r0 += (long long)kLossWaves * RB) {
        float x[RB][CPL], t[RB][CPL];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const long long r = r0 + (long long)i * kLossWaves;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int j = lane + 64 * c;
                const bool ok = r < rows && j < cols;
                x[i][c] = ok ? logits[r * cols + j] : 0.f;
                t[i][c] = ok ? tgt[r * cols + j] : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const long long r = r0 + (long long)i * kLossWaves;
            if (r >= rows) break;   // wave-uniform
            // rowMax: the first element when it is NaN, else the largest non-NaN element
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (lane + 64 * c < cols) m = gtMax(m, x[i][c]);
            m = waveMax(m);
            const float e0 = __shfl(x[i][0], 0, 64);
            m = e0 != e0 ? e0 : gtMax(e0, m);
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (lane + 64 * c < cols) {
                    const float e = expf(x[i][c] - m);
                    x[i][c] = e;
                    sum += e;
                }
            sum = waveSum(sum);
            float la = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int j = lane + 64 * c;
                if (j >= cols) continue;
                const float pv = x[i][c] / sum;
                if (prob) prob[r * cols + j] = pv;
                if (loss && t[i][c] > 0.5f) {
                    float q = pv;
                    if (q < 1e-7f) q = 1e-7f;
                    la -= logf(q);
                }
                if (grad) grad[r * cols + j] = (pv - t[i][c]) * scale;
            }
            if (loss) acc += waveSum(la);
        }
    }
    if (loss) finishLoss(acc, loss, rows, lds);
}

// Bias gradient, nHW == 1 (a Linear layer's [rows, cols] gradient): a thread per
// column adds the rows in order, starting from 0 — the reference's loop order
// (autograd.ixx:428-433), so the result is bit-identical to it.
__global__ void bias_grad_cols_kernel(const float* g, float* gb, int rows, int cols) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    const float* p = g + c;
    float acc = 0.f;
    int r = 0;
    for (; r + 64 <= rows; r += 64) {   // 64 loads in flight, then the adds in row order
        float a[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) a[i] = p[(long long)(r + i) * cols];
#pragma unroll
        for (int i = 0; i < 64; ++i) acc += a[i];
    }
    for (; r < rows; ++r) acc += p[(long long)r * cols];
    gb[c] = acc;
}

// Bias gradient for many rows: block = 64 columns x 16 row parts; each part adds
// its contiguous rows in order, then the parts are added in order.
__global__ void __launch_bounds__(1024) bias_grad_cols_parts_kernel(const float* g, float* gb, int rows, int cols) {
    __shared__ float part[16][65];
    const int cl = threadIdx.x & 63, pi = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    const int len = (rows + 15) / 16;
    const int r0 = pi * len, r1 = min(rows, r0 + len);
    float acc = 0.f;
    if (c < cols)
        for (int r = r0; r < r1; ++r) acc += g[(long long)r * cols + c];
    part[pi][cl] = acc;
    __syncthreads();
    if (pi == 0 && c < cols) {
        float tot = 0.f;
        for (int q = 0; q < 16; ++q) tot += part[q][cl];
        gb[c] = tot;
    }
}

// Bias gradient of an [N, C, HW] gradient (conv layout): a workgroup per channel,
// thread t adds elements hw = t, t+256, ... of every image in (image, hw) order,
// then a fixed tree over the 256 partials.
__global__ void __launch_bounds__(256) bias_grad_planes_kernel(const float* g, float* gb, int N, int C, int HW) {
    __shared__ float red[256];
    const int c = blockIdx.x;
    float acc = 0.f;
    for (int n = 0; n < N; ++n) {
        const float* p = g + ((long long)n * C + c) * HW;
        for (int i = threadIdx.x; i < HW; i += 256) acc += p[i];
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s >= 1; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) gb[c] = red[0];
}

static int checkRows(const char* name, const void* a, const void* b, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return fail("%s: rows and classes must be positive (%d, %d)", name, rows, cols);
    if (!a || !b) return fail("%s: null pointer", name);
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipSoftmax(const float* pIn, float* pOut, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipSoftmax", pIn, pOut, nBatch, nClasses)) return -1;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((nBatch + 3) / 4), dim3(256), 0, stream(), pIn, pOut, nBatch,
                       nClasses);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipCrossEntropy(const float* pSoftmax, const float* pTarget, float* pResult, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipCrossEntropy", pSoftmax, pTarget, nBatch, nClasses)) return -1;
    if (!pResult) return fail("omHipCrossEntropy: null result");
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(1), dim3(64 * kLossWaves), 0, stream(), pSoftmax, pTarget, pResult,
                       nBatch, nClasses);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipSoftmaxCrossEntropyBackward(const float* pSoftmax, const float* pTarget, float* pGradLogits, int nBatch,
                                     int nClasses) {
    clearError();
    if (checkRows("omHipSoftmaxCrossEntropyBackward", pSoftmax, pTarget, nBatch, nClasses)) return -1;
    if (!pGradLogits) return fail("omHipSoftmaxCrossEntropyBackward: null output");
    const float scale = 1.0f / static_cast<float>(nBatch);   // as cpu_backend.ixx:395
    const long long n = (long long)nBatch * nClasses;
    const int blocks = (int)std::min<long long>((n + 255) / 256, (long long)cuCount() * 16);
    hipLaunchKernelGGL(softmax_ce_backward_kernel, dim3(blocks), dim3(256), 0, stream(), pSoftmax, pTarget,
                       pGradLogits, n, scale);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipSoftmaxCrossEntropy(const float* pLogits, const float* pTarget, float* pSoftmax, float* pLoss,
                             float* pGradLogits, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipSoftmaxCrossEntropy", pLogits, pTarget, nBatch, nClasses)) return -1;
    if (!pSoftmax && !pGradLogits && (long long)kLossWaves * nClasses > (1LL << 20))
        return fail("omHipSoftmaxCrossEntropy: %d classes need the softmax or gradient output", nClasses);
    float* rowBuf = nullptr;
    if (!pSoftmax && !pGradLogits && nClasses > 256) {
        rowBuf = static_cast<float*>(workspace((size_t)kLossWaves * nClasses * sizeof(float)));
        if (!rowBuf) return -1;
    }
    const float scale = 1.0f / static_cast<float>(nBatch);
    if (nClasses <= 64)
        hipLaunchKernelGGL(softmax_ce_fused_reg_kernel<1>, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits,
                           pTarget, pSoftmax, pLoss, pGradLogits, nBatch, nClasses, scale);
    else if (nClasses <= 256)
        hipLaunchKernelGGL(softmax_ce_fused_reg_kernel<4>, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits,
                           pTarget, pSoftmax, pLoss, pGradLogits, nBatch, nClasses, scale);
    else
        hipLaunchKernelGGL(softmax_ce_fused_kernel, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits, pTarget,
                           pSoftmax, pLoss, pGradLogits, rowBuf, nBatch, nClasses, scale);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAddBiasBackward(const float* pGradOut, float* pGradBias, int nN, int nC, int nHW) {
    clearError();
    if (nC <= 0) return 0;
    if (!pGradBias) return fail("omHipAddBiasBackward: null output");
    if (nN < 0 || nHW < 0) return fail("omHipAddBiasBackward: negative size");
    if (nN == 0 || nHW == 0) return omHipFillZeros(pGradBias, nC);
    if (!pGradOut) return fail("omHipAddBiasBackward: null gradient");
    if (nHW == 1 && nN <= 4096)
        hipLaunchKernelGGL(bias_grad_cols_kernel, dim3((nC + 255) / 256), dim3(256), 0, stream(), pGradOut, pGradBias,
                           nN, nC);
    else if (nHW == 1)
        hipLaunchKernelGGL(bias_grad_cols_parts_kernel, dim3((nC + 63) / 64), dim3(1024), 0, stream(), pGradOut,
                           pGradBias, nN, nC);
    else
        hipLaunchKernelGGL(bias_grad_planes_kernel, dim3(nC), dim3(256), 0, stream(), pGradOut, pGradBias, nN, nC,
                           nHW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // extern "C"
