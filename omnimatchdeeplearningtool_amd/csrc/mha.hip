// mha.hip — MultiHeadAttention::forward (src/engine/om.engine.vit.ixx:150-239)
// composed on the device for half-precision activations and weights with fp32
// accumulation:
//   qkv = x Wqkv + bqkv        (Linear, linear.ixx:50-58: W stored [in, out])
//   ctx = merge(softmax(Q K^T) V) with Q = scale * qkv[:, :D] split into heads
//   out = ctx Wout + bout
//
// Head dimension 64 with at most 384 tokens (ViT-B/16 and its relatives) runs
// in three launches: the QKV projection rounds its fp32 result to the input
// type as it stores it, straight into the fused attention kernel's input
// layout; the kernel writes the merged context in the input type, which the
// output projection reads. Other shapes run the reference's unfused order in
// fp32 (qkvSplitHeads' Q scaling, Q K^T, tensorSoftmaxLastDim, P V,
// mergeHeads): the QKV projection with fp32 output, Q scaled in place, then
// per group of images or heads one strided-batched Q K^T that reads the heads
// where they lie in the projection (no split copy), a row softmax in place and
// one strided-batched P V that writes the merged-head layout directly; the
// context is rounded to the input type for the output projection.
//
// Intermediates live in the stream's staging workspace, which the ops called
// here do not use.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

// Multiplies columns [0, cols) of every row by scale: qkvSplitHeads' Q * scale
// (vit.ixx:207), in place on the projection.
__global__ void scale_columns_kernel(float* x, long long rows, int ld, int cols, float scale) {
    const long long total = rows * cols;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const long long r = i / cols;
        const int c = (int)(i - r * cols);
        x[r * ld + c] = x[r * ld + c] * scale;
    }
}

namespace {

constexpr size_t kAlign = 256;
size_t up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

}  // namespace

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipMultiHeadAttentionHalf(int nDtype, const uint16_t* pX, const uint16_t* pWqkv, const float* pBqkv,
                                const uint16_t* pWout, const float* pBout, void* pOut, int nOutHalf, int nBatch,
                                int nSeq, int nHeads, int nHeadDim) {
    const char* name = "omHipMultiHeadAttentionHalf";
    clearError();
    if (nBatch <= 0 || nSeq <= 0 || nHeads <= 0 || nHeadDim <= 0) return 0;
    if (!pX || !pWqkv || !pWout || !pOut) return fail("%s: null pointer", name);
    if (nDtype != 0 && nDtype != 1) return fail("%s: dtype must be 0 (fp16) or 1 (bf16)", name);
    const long long D = (long long)nHeads * nHeadDim;
    const long long T = (long long)nBatch * nSeq;
    if (D > 0x7fffffffLL / 3 || T > 0x7fffffffLL || T * 3 * D > 0x7fffffffLL)
        return fail("%s: %lld tokens x %lld features exceed the 2^31-element limit", name, T, D);
    const int nD = (int)D, nT = (int)T;
    const float scale = 1.0f / std::sqrt((float)nHeadDim);   // MultiHeadAttention's m_fScale

    if (nHeadDim == 64 && nSeq <= 384) {
        uint16_t* qkv = static_cast<uint16_t*>(workspace(up(T * 3 * D * 2) + up(T * D * 2), kWsStaging));
        if (!qkv) return -1;   // workspace() recorded the cause
        uint16_t* ctx = qkv + up(T * 3 * D * 2) / 2;
        if (omHipLinearHalf(nDtype, pX, pWqkv, 0, pBqkv, 0, qkv, 1, nT, nD, 3 * nD)) return -1;
        if (omHipAttentionHalf(nDtype, qkv, ctx, 1, nBatch, nSeq, nHeads, nHeadDim, scale)) return -1;
        return omHipLinearHalf(nDtype, ctx, pWout, 0, pBout, 0, pOut, nOutHalf, nT, nD, nD);
    }

    // Unfused: the outer loop runs over whichever of images / heads is fewer,
    // each step batching the other over one strided GEMM.
    const bool headsOuter = nHeads <= nBatch;
    const int outer = headsOuter ? nHeads : nBatch, inner = headsOuter ? nBatch : nHeads;
    const long long S = nSeq, Dh = nHeadDim;
    const long long ldq = 3 * D;
    const long long innerQ = headsOuter ? S * ldq : Dh;    // Q/K/V step between inner batch entries
    const long long innerC = headsOuter ? S * D : Dh;      // context step between inner batch entries
    if ((long long)inner * S > 0x7fffffffLL || (long long)inner * S * S > (1LL << 40))
        return fail("%s: %d x %lld score rows exceed the limit", name, inner, S);
    const size_t bQkv = up(T * 3 * D * 4), bScores = up((size_t)inner * S * S * 4), bCtx = up(T * D * 4);
    char* base = static_cast<char*>(workspace(bQkv + bScores + bCtx + up(T * D * 2), kWsStaging));
    if (!base) return -1;
    float* qkv = reinterpret_cast<float*>(base);
    float* scores = reinterpret_cast<float*>(base + bQkv);
    float* ctx = reinterpret_cast<float*>(base + bQkv + bScores);
    uint16_t* ctxHalf = reinterpret_cast<uint16_t*>(base + bQkv + bScores + bCtx);

    if (omHipLinearHalf(nDtype, pX, pWqkv, 0, pBqkv, 0, qkv, 0, nT, nD, 3 * nD)) return -1;
    const long long qn = T * D;
    hipLaunchKernelGGL(scale_columns_kernel, dim3((unsigned)std::min<long long>((qn + 255) / 256, 8192)), dim3(256), 0,
                       stream(), qkv, T, (int)ldq, nD, scale);
    OMHIP_CHECK_LAUNCH();
    for (int o = 0; o < outer; ++o) {
        const long long qOff = headsOuter ? o * Dh : o * S * ldq;
        const long long cOff = headsOuter ? o * Dh : o * S * D;
        const float* Q = qkv + qOff;
        const float* K = Q + D;
        const float* V = Q + 2 * D;
        if (omHipGemmStridedBatched(0, 1, inner, nSeq, nSeq, nHeadDim, Q, ldq, innerQ, K, ldq, innerQ, scores, S,
                                    S * S))
            return -1;
        if (omHipSoftmax(scores, scores, inner * nSeq, nSeq)) return -1;
        if (omHipGemmStridedBatched(0, 0, inner, nSeq, nHeadDim, nSeq, scores, S, S * S, V, ldq, innerQ, ctx + cOff, D,
                                    innerC))
            return -1;
    }
    if ((nDtype == 1 ? omHipConvertF32ToBF16 : omHipConvertF32ToF16)(ctx, ctxHalf, (int)(T * D))) return -1;
    return omHipLinearHalf(nDtype, ctxHalf, pWout, 0, pBout, 0, pOut, nOutHalf, nT, nD, nD);
}

}  // extern "C"
