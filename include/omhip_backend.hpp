// omhip_backend.hpp — om::HIPBackend, the C++23 HAL class for MI355X.
//
// Drop-in for the GPU slot of the reference HAL: same static-method shape as
// om::CPUBackend (src/hal/om.hal.cpu_backend.ixx:61-1631) and the slot that
// om::CUDABackend occupies today (src/hal/om.hal.cuda_backend.ixx:283-983),
// selected by the existing `if (isCudaTensor(t))` dispatch
// (src/engine/om.engine.tensor_ops.ixx:35-37). Signatures and argument order are
// CPUBackend's (CUDABackend's conv2d / batchNorm2d orders differ:
// cuda_backend.ixx:438-448, :571-586). Pointers are device pointers.
//
// Error behaviour: every call checks the omHip* status and throws
// std::runtime_error carrying omHipGetLastError(); the reference CUDABackend
// ignores the int it gets back.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "omhip.h"

namespace om {

class HIPBackend {
public:
    // ---- device ----
    static void init(int nDevice = 0) { check(omHipInit(nDevice), "omHipInit"); }
    static void synchronize() { check(omHipSynchronize(), "omHipSynchronize"); }
    // omCudaForceReset (EngineBridge.cpp:4047): device sync, sticky error cleared, library state released
    static void forceReset() { check(omHipForceReset(), "forceReset"); }
    // ---- transfer stream and pinned host memory (cuda_kernels.cuh:56-66, :497-505) ----
    static void* mallocHost(size_t nBytes) {
        void* p = nullptr;
        check(omHipMallocHost(&p, nBytes), "mallocHost");
        return p;
    }
    static void freeHost(void* p) { check(omHipFreeHost(p), "freeHost"); }
    static void asyncCopyH2D(void* pDst, const void* pSrc, size_t nBytes) {
        check(omHipAsyncCopyH2D(pDst, pSrc, nBytes), "asyncCopyH2D");
    }
    static void asyncCopyD2H(void* pDst, const void* pSrc, size_t nBytes) {
        check(omHipAsyncCopyD2H(pDst, pSrc, nBytes), "asyncCopyD2H");
    }
    static void syncTransferStream() { check(omHipSyncTransferStream(), "syncTransferStream"); }
    static void computeWaitTransfer() { check(omHipComputeWaitTransfer(), "computeWaitTransfer"); }
    static void* malloc(size_t nBytes) {
        void* p = nullptr;
        check(omHipMalloc(&p, nBytes), "omHipMalloc");
        return p;
    }
    static void free(void* p) { check(omHipFree(p), "omHipFree"); }
    static void copyH2D(void* pDst, const void* pSrc, size_t nBytes) { check(omHipCopyH2D(pDst, pSrc, nBytes), "omHipCopyH2D"); }
    static void copyD2H(void* pDst, const void* pSrc, size_t nBytes) { check(omHipCopyD2H(pDst, pSrc, nBytes), "omHipCopyD2H"); }

    // ---- fills / copy (cpu_backend.ixx:65-77, :444-446) ----
    static void fillZeros(float* pData, size_t nCount) { check(omHipFillZeros(pData, toInt(nCount)), "fillZeros"); }
    static void fillOnes(float* pData, size_t nCount) { check(omHipFillOnes(pData, toInt(nCount)), "fillOnes"); }
    static void fillValue(float* pData, size_t nCount, float fValue) {
        check(omHipFillValue(pData, toInt(nCount), fValue), "fillValue");
    }
    static void copy(const float* pSrc, float* pDst, size_t nCount) { check(omHipCopy(pSrc, pDst, toInt(nCount)), "copy"); }

    // ---- GEMM (cpu_backend.ixx:239-286, :1520-1539) ----
    static void matmul(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
        check(omHipMatmul(pA, pB, pC, nM, nK, nN), "matmul");
    }
    static void batchedMatmul(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
        check(omHipBatchedMatmul(pA, pB, pC, nBatch, nM, nK, nN), "batchedMatmul");
    }
    static void transpose2d(const float* pA, float* pB, int nRows, int nCols) {
        check(omHipTranspose(pA, pB, nRows, nCols), "transpose2d");
    }
    // CUDABackend's name for the same op (cuda_backend.ixx:340), called per batch by
    // tensorTranspose2dBatched's GPU branch (tensor_ops.ixx:1595-1604)
    static void transpose(const float* pIn, float* pOut, int nRows, int nCols) {
        check(omHipTranspose(pIn, pOut, nRows, nCols), "transpose");
    }

    // ---- reductions (cpu_backend.ixx:290-294; CUDABackend::sum cuda_backend.ixx:732) ----
    // CUDABackend::sum's form, used by tensorSum's GPU branch (tensor_ops.ixx:413-417): the
    // result stays on the device
    static void sum(const float* pData, float* pResult, int nCount) {
        check(omHipSum(pData, pResult, nCount), "sum");
    }
    // CPUBackend::sum's form: the sum is copied back to the host (waits for the stream)
    static float sum(const float* pData, size_t nCount) {
        float* d = nullptr;
        check(omHipMalloc(reinterpret_cast<void**>(&d), sizeof(float)), "sum");
        float v = 0.f;
        const int rc = omHipSum(pData, d, toInt(nCount));
        const int rc2 = rc ? rc : omHipCopyD2H(&v, d, sizeof(float));
        omHipFree(d);
        check(rc2, "sum");
        return v;
    }
    // omCudaMean (cuda_kernels.cu:1506-1513): the sum times 1 / nCount, on the device
    static void mean(const float* pData, float* pResult, int nCount) {
        check(omHipMean(pData, pResult, nCount), "mean");
    }

    // ---- activations / bias (cpu_backend.ixx:317-346, :433-440) ----
    static void relu(const float* pIn, float* pOut, size_t nCount) { check(omHipReLU(pIn, pOut, toInt(nCount)), "relu"); }
    static void reluBackward(const float* pIn, const float* pGradOut, float* pGradIn, size_t nCount) {
        check(omHipReLUBackward(pIn, pGradOut, pGradIn, toInt(nCount)), "reluBackward");
    }
    static void addBias(const float* pA, const float* pBias, float* pOut, int nBatch, int nCols) {
        check(omHipAddBias(pA, pBias, pOut, nBatch, nCols, 1), "addBias");
    }
    // AddBiasBackward's reduction (autograd.ixx:399-433), CUDABackend::addBiasBackward's
    // signature (cuda_backend.ixx:747): gradBias[c] = sum over n, hw of gradOut[n,c,hw].
    static void addBiasBackward(const float* pGradOut, float* pGradBias, int nN, int nC, int nHW) {
        check(omHipAddBiasBackward(pGradOut, pGradBias, nN, nC, nHW), "addBiasBackward");
    }

    // ---- softmax / cross-entropy (cpu_backend.ixx:352-410) ----
    static void softmax(const float* pIn, float* pOut, int nBatch, int nClasses) {
        check(omHipSoftmax(pIn, pOut, nBatch, nClasses), "softmax");
    }
    // CPUBackend::crossEntropy returns the loss: computed on the device, then copied back
    // (waits for the stream).
    static float crossEntropy(const float* pPred, const float* pTarget, int nBatch, int nClasses) {
        float* d = nullptr;
        check(omHipMalloc(reinterpret_cast<void**>(&d), sizeof(float)), "crossEntropy");
        float v = 0.f;
        const int rc = omHipCrossEntropy(pPred, pTarget, d, nBatch, nClasses);
        const int rc2 = rc ? rc : omHipCopyD2H(&v, d, sizeof(float));
        omHipFree(d);
        check(rc2, "crossEntropy");
        return v;
    }
    // CUDABackend::crossEntropyForward (cuda_backend.ixx:823): the loss stays on the device.
    static void crossEntropyForward(const float* pSoftmax, const float* pTarget, float* pResult, int nBatch,
                                    int nClasses) {
        check(omHipCrossEntropy(pSoftmax, pTarget, pResult, nBatch, nClasses), "crossEntropyForward");
    }
    static void crossEntropySoftmaxBackward(const float* pSoftmax, const float* pTarget, float* pGradInput,
                                            int nBatch, int nClasses) {
        check(omHipSoftmaxCrossEntropyBackward(pSoftmax, pTarget, pGradInput, nBatch, nClasses),
              "crossEntropySoftmaxBackward");
    }

    // ---- conv / BN (cpu_backend.ixx:544-575, :619-658, :781-842) ----
    static void im2col(const float* pInput, int nCin, int nH, int nW, int nKH, int nKW, int nPadH, int nPadW,
                       int nStrideH, int nStrideW, float* pCol) {
        check(omHipIm2col(pInput, nCin, nH, nW, nKH, nKW, nPadH, nPadW, nStrideH, nStrideW, pCol), "im2col");
    }
    static void conv2d(const float* pInput, const float* pWeight, const float* pBias, float* pOutput, int nBatch,
                       int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
        check(omHipConv2d(pInput, pWeight, pBias, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad),
              "conv2d");
    }
    // bTraining: batch statistics, saved mean / inverse std and running averages (:796-822).
    static void batchNorm2d(const float* pInput, float* pOutput, const float* pGamma, const float* pBeta,
                            float* pRunMean, float* pRunVar, float* pSavedMean, float* pSavedInvStd, int nBatch,
                            int nChannels, int nH, int nW, float fEps, float fMomentum, bool bTraining) {
        check(omHipBatchNorm2d(pInput, pOutput, pGamma, pBeta, pRunMean, pRunVar, pSavedMean, pSavedInvStd, nBatch,
                               nChannels, nH, nW, fEps, fMomentum, bTraining ? 1 : 0),
              "batchNorm2d");
    }

    // ---- conv / BN training (cpu_backend.ixx:666-772, :847-890) ----
    static void conv2dBackwardInput(const float* pGradOutput, const float* pWeight, float* pGradInput, int nBatch,
                                    int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
        check(omHipConv2dBackwardInput(pGradOutput, pWeight, pGradInput, nBatch, nCin, nH, nW, nCout, nKH, nKW,
                                       nStride, nPad),
              "conv2dBackwardInput");
    }
    static void conv2dBackwardWeight(const float* pInput, const float* pGradOutput, float* pGradWeight,
                                     float* pGradBias, int nBatch, int nCin, int nH, int nW, int nCout, int nKH,
                                     int nKW, int nStride, int nPad) {
        check(omHipConv2dBackwardWeight(pInput, pGradOutput, pGradWeight, pGradBias, nBatch, nCin, nH, nW, nCout, nKH,
                                        nKW, nStride, nPad),
              "conv2dBackwardWeight");
    }
    static void batchNorm2dBackward(const float* pGradOutput, const float* pInput, const float* pSavedMean,
                                    const float* pSavedInvStd, const float* pGamma, float* pGradInput,
                                    float* pGradGamma, float* pGradBeta, int nBatch, int nChannels, int nH, int nW) {
        check(omHipBatchNorm2dBackward(pGradOutput, pInput, pSavedMean, pSavedInvStd, pGamma, pGradInput, pGradGamma,
                                       pGradBeta, nBatch, nChannels, nH, nW, 1e-5f),
              "batchNorm2dBackward");
    }
    // fused training passes (bit-identical to the separate reference ops)
    static void batchNorm2dBackwardRelu(const float* pGradOutput, const float* pReluInput, const float* pInput,
                                        const float* pSavedMean, const float* pSavedInvStd, const float* pGamma,
                                        float* pGradInput, float* pGradGamma, float* pGradBeta, int nBatch,
                                        int nChannels, int nH, int nW) {
        check(omHipBatchNorm2dBackwardRelu(pGradOutput, pReluInput, pInput, pSavedMean, pSavedInvStd, pGamma,
                                           pGradInput, pGradGamma, pGradBeta, nBatch, nChannels, nH, nW, 1e-5f),
              "batchNorm2dBackwardRelu");
    }
    static void batchNorm2dTrainAct(const float* pInput, float* pOutput, const float* pGamma, const float* pBeta,
                                    float* pRunningMean, float* pRunningVar, float* pSavedMean, float* pSavedInvStd,
                                    int nBatch, int nChannels, int nH, int nW, float fEps, float fMomentum,
                                    const float* pResidual, bool bRelu) {
        check(omHipBatchNorm2dTrainAct(pInput, pOutput, pGamma, pBeta, pRunningMean, pRunningVar, pSavedMean,
                                       pSavedInvStd, nBatch, nChannels, nH, nW, fEps, fMomentum, pResidual,
                                       bRelu ? 1 : 0),
              "batchNorm2dTrainAct");
    }

    // ---- pooling and add (cpu_backend.ixx:897-1023, :1467-1510, :147-160) ----
    static void maxPool2d(const float* pInput, float* pOutput, int* pIndices, int nBatch, int nChannels, int nH,
                          int nW, int nKH, int nKW, int nStride, int nPad) {
        check(omHipMaxPool2d(pInput, pOutput, pIndices, nBatch, nChannels, nH, nW, nKH, nKW, nStride, nStride, nPad,
                             nPad),
              "maxPool2d");
    }
    static void maxPool2dBackward(const float* pGradOutput, const int* pIndices, float* pGradInput, int nBatch,
                                  int nChannels, int nHout, int nWout, int nH, int nW) {
        check(omHipMaxPool2dBackward(pGradOutput, pIndices, pGradInput, nBatch, nChannels, nH, nW, nHout, nWout),
              "maxPool2dBackward");
    }
    static void avgPool2d(const float* pInput, float* pOutput, int nBatch, int nChannels, int nH, int nW, int nKH,
                          int nKW, int nStride, int nPad) {
        check(omHipAvgPool2d(pInput, pOutput, nBatch, nChannels, nH, nW, nKH, nKW, nStride, nStride, nPad, nPad),
              "avgPool2d");
    }
    static void avgPool2dBackward(const float* pGradOutput, float* pGradInput, int nBatch, int nChannels, int nH,
                                  int nW, int /*nHout*/, int /*nWout*/, int nKH, int nKW, int nStride, int nPad) {
        check(omHipAvgPool2dBackward(pGradOutput, pGradInput, nBatch, nChannels, nH, nW, nKH, nKW, nStride, nStride,
                                     nPad, nPad),
              "avgPool2dBackward");
    }
    static void adaptiveAvgPool2d(const float* pInput, float* pOutput, int nBatch, int nChannels, int nH, int nW,
                                  int nOutH, int nOutW) {
        check(omHipAdaptiveAvgPool2d(pInput, pOutput, nBatch, nChannels, nH, nW, nOutH, nOutW), "adaptiveAvgPool2d");
    }
    static void adaptiveAvgPool2dBackward(const float* pGradOutput, float* pGradInput, int nBatch, int nChannels,
                                          int nH, int nW, int nOutH, int nOutW) {
        check(omHipAdaptiveAvgPool2dBackward(pGradOutput, pGradInput, nBatch, nChannels, nH, nW, nOutH, nOutW),
              "adaptiveAvgPool2dBackward");
    }
    static void add(const float* pA, const float* pB, float* pOut, size_t nCount) {
        check(omHipAdd(pA, pB, pOut, toInt(nCount)), "add");
    }
    static void addReluBackward(const float* pA, const float* pInput, const float* pGradOutput, float* pOut,
                                size_t nCount) {
        check(omHipAddReluBackward(pA, pInput, pGradOutput, pOut, toInt(nCount)), "addReluBackward");
    }

    // ---- ViT attention on fp32 data (CUDABackend cuda_backend.ixx:967-985; vit.ixx:163-187) ----
    static void qkvSplitHeads(const float* pQkv, float* pQ, float* pK, float* pV, int nBatch, int nSeqLen,
                              int nHeads, int nHeadDim, float fScale) {
        check(omHipQkvSplitHeads(pQkv, pQ, pK, pV, nBatch, nSeqLen, nHeads, nHeadDim, fScale), "qkvSplitHeads");
    }
    static void mergeHeads(const float* pIn, float* pOut, int nBatch, int nSeqLen, int nHeads, int nHeadDim) {
        check(omHipMergeHeads(pIn, pOut, nBatch, nSeqLen, nHeads, nHeadDim), "mergeHeads");
    }
    // qkvSplitHeads .. mergeHeads of the GPU branch in one call: qkv [B*S, 3*H*D] -> out [B*S, H*D]
    static void attention(const float* pQKV, float* pOut, int nBatch, int nSeq, int nHeads, int nHeadDim,
                          float fScale) {
        check(omHipAttention(pQKV, pOut, nBatch, nSeq, nHeads, nHeadDim, fScale), "attention");
    }

    // ---- fused attention (vit.ixx:150-239): qkv [B*S, 3*H*D] half -> out [B*S, H*D] ----
    static void attentionHalf(int nDtype, const uint16_t* pQKV, void* pOut, bool bOutHalf, int nBatch, int nSeq,
                              int nHeads, int nHeadDim, float fScale) {
        check(omHipAttentionHalf(nDtype, pQKV, pOut, bOutHalf ? 1 : 0, nBatch, nSeq, nHeads, nHeadDim, fScale),
              "attentionHalf");
    }
    // Linear::forward (linear.ixx:50-58) on half inputs: act(x W + b), W [K,N] ([N,K] when bTransW)
    static void linearHalf(int nDtype, const uint16_t* pInput, const uint16_t* pWeight, bool bTransW,
                           const float* pBias, int nAct, void* pOutput, bool bOutHalf, int nM, int nK, int nN) {
        check(omHipLinearHalf(nDtype, pInput, pWeight, bTransW ? 1 : 0, pBias, nAct, pOutput, bOutHalf ? 1 : 0, nM,
                              nK, nN),
              "linearHalf");
    }
    // MultiHeadAttention::forward (vit.ixx:150-239): QKV Linear -> attention -> output Linear
    static void multiHeadAttentionHalf(int nDtype, const uint16_t* pX, const uint16_t* pWqkv, const float* pBqkv,
                                       const uint16_t* pWout, const float* pBout, void* pOut, bool bOutHalf,
                                       int nBatch, int nSeq, int nHeads, int nHeadDim) {
        check(omHipMultiHeadAttentionHalf(nDtype, pX, pWqkv, pBqkv, pWout, pBout, pOut, bOutHalf ? 1 : 0, nBatch,
                                          nSeq, nHeads, nHeadDim),
              "multiHeadAttentionHalf");
    }

    // ---- entries the reference builds by composition ----
    // transpose2d(B) + matmul (autograd.ixx:261-273)
    static void matmulTransB(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
        check(omHipMatmulTransB(pA, pB, pC, nM, nK, nN), "matmulTransB");
    }
    // transpose2d(A) + matmul (autograd.ixx:276-286)
    static void matmulTransA(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
        check(omHipMatmulTransA(pA, pB, pC, nM, nK, nN), "matmulTransA");
    }
    // Linear + bias (+ ReLU when nAct = 1) in one pass: act(A * W + bias), W [K, N].
    static void linearBiasAct(const float* pA, const float* pW, const float* pBias, float* pOut, int nM, int nK,
                              int nN, int nAct) {
        check(omHipLinearBiasAct(pA, pW, pBias, pOut, nM, nK, nN, nAct), "linearBiasAct");
    }
    // A Linear layer's backward in one launch: dW = X^T G, db = column sums of G, dX = G W^T
    // gated by the previous layer's ReLU output when pGate is given (pGradBias, pGradInput and
    // pGate nullable).
    static void linearBackward(const float* pInput, const float* pGradOut, const float* pWeight, const float* pGate,
                               float* pGradWeight, float* pGradBias, float* pGradInput, int nBatch, int nIn, int nOut) {
        check(omHipLinearBackward(pInput, pGradOut, pWeight, pGate, pGradWeight, pGradBias, pGradInput, nBatch, nIn,
                                  nOut),
              "linearBackward");
    }
    // The classifier head of a training step in one launch: logits = X W + b, softmax
    // cross-entropy, g = (p - T) / nBatch, gW = X^T g, gb, gX = g W^T (gated by pGate > 0).
    static void linearSoftmaxCrossEntropyStep(const float* pInput, const float* pWeight, const float* pBias,
                                              const float* pTarget, const float* pGate, float* pLogits, float* pLoss,
                                              float* pGradLogits, float* pGradWeight, float* pGradBias,
                                              float* pGradInput, int nBatch, int nIn, int nClasses) {
        check(omHipLinearSoftmaxCrossEntropyStep(pInput, pWeight, pBias, pTarget, pGate, pLogits, pLoss, pGradLogits,
                                                 pGradWeight, pGradBias, pGradInput, nBatch, nIn, nClasses),
              "linearSoftmaxCrossEntropyStep");
    }
    static void batchedMatmulTransB(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
        check(omHipBatchedMatmulTransB(pA, pB, pC, nBatch, nM, nK, nN), "batchedMatmulTransB");
    }
    // conv2d -> batchNorm2d(eval) -> add(shortcut) -> relu (resnet.ixx:55-79)
    static void conv2dBiasBnAddAct(const float* pInput, const float* pWeight, const float* pBias,
                                   const float* pGamma, const float* pBeta, const float* pMean, const float* pVar,
                                   float fEps, const float* pResidual, int nAct, float* pOutput, int nBatch, int nCin,
                                   int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
        check(omHipConv2dBiasBnAddAct(pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, pResidual, nAct,
                                      pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad),
              "conv2dBiasBnAddAct");
    }
    // conv2d -> batchNorm2d(eval) -> relu (tensor_ops.ixx:672-833, :511-536)
    static void conv2dBiasBnAct(const float* pInput, const float* pWeight, const float* pBias, const float* pGamma,
                                const float* pBeta, const float* pMean, const float* pVar, float fEps, int nAct,
                                float* pOutput, int nBatch, int nCin, int nH, int nW, int nCout, int nKH, int nKW,
                                int nStride, int nPad) {
        check(omHipConv2dBiasBnAct(pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, nAct, pOutput, nBatch,
                                   nCin, nH, nW, nCout, nKH, nKW, nStride, nPad),
              "conv2dBiasBnAct");
    }
    // halfToFloat(A), halfToFloat(B), matmul (fp16.ixx:103-164) with fp32 accumulate
    static void matmulF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
        check(omHipMatmulF16(pA, pB, pC, nM, nK, nN), "matmulF16");
    }
    static void matmulBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
        check(omHipMatmulBF16(pA, pB, pC, nM, nK, nN), "matmulBF16");
    }

private:
    static int toInt(size_t n) {
        if (n > static_cast<size_t>(0x7fffffff)) throw std::runtime_error("HIPBackend: element count exceeds INT_MAX");
        return static_cast<int>(n);
    }
    static void check(int rc, const char* what) {
        if (rc != 0) throw std::runtime_error(std::string("HIPBackend::") + what + ": " + omHipGetLastError());
    }
};

// Device-resident ResNet-18 classifier and its batch inference pipeline
// (EngineBridge::inferBatch, EngineBridge.cpp:3525-3772, classification branch).
class ResNet18Infer {
public:
    struct Result {
        std::vector<int> classes;        // -1 below the confidence threshold
        std::vector<float> confidences;  // top probability
        std::vector<float> probs;        // [images][classes]
    };
    ResNet18Infer(const std::vector<float>& params, int nClasses, int nMaxBatch = 32) : m_nc(nClasses) {
        check(omHipResNet18Create(params.data(), static_cast<long long>(params.size()), nClasses, nMaxBatch,
                                  &m_net),
              "ResNet18Infer");
    }
    ~ResNet18Infer() { (void)omHipResNet18Destroy(m_net); }
    ResNet18Infer(const ResNet18Infer&) = delete;
    ResNet18Infer& operator=(const ResNet18Infer&) = delete;

    // images: nImages x 3 x 224 x 224 floats in [0, 1], contiguous
    Result inferBatch(const std::vector<float>& images, int nImages, int nBatchSize = 32, bool bImageNetNorm = true,
                      float fConfThreshold = 0.0f) const {
        Result r;
        r.classes.resize(nImages);
        r.confidences.resize(nImages);
        r.probs.resize(static_cast<size_t>(nImages) * m_nc);
        check(omHipResNet18InferBatch(m_net, images.data(), nImages, 3, 224, 224, nBatchSize, bImageNetNorm ? 1 : 0,
                                      fConfThreshold, r.classes.data(), r.confidences.data(), r.probs.data()),
              "inferBatch");
        return r;
    }

private:
    static void check(int rc, const char* what) {
        if (rc != 0) throw std::runtime_error(std::string("ResNet18Infer::") + what + ": " + omHipGetLastError());
    }
    void* m_net = nullptr;
    int m_nc;
};

}  // namespace om
