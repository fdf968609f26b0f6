/*
 * omhip.h — C ABI of libomhip.so, the gfx950 (MI355X) compute backend for the
 * OmniMatch HAL matmul / conv2d hot path.
 *
 * Conventions (identical to the reference omCuda* ABI, src/cuda/cuda_kernels.cuh:10-535):
 *   - every entry returns int: 0 on success, -1 on a HIP error or invalid
 *     argument (omHipGetLastError() names the cause);
 *   - every data pointer is a DEVICE pointer to row-major contiguous data;
 *   - kernels are asynchronous on one library-owned stream; results become
 *     host-visible after omHipCopyD2H / omHipSynchronize;
 *   - omHipInit(dev) must precede use; it is idempotent and thread-safe.
 *   - GEMM entries with M<=0, N<=0 or K<=0 (or a null input) zero C when C and
 *     its extent are valid and return 0, as CPUBackend::matmul does
 *     (src/hal/om.hal.cpu_backend.ixx:246-251).
 *
 * Each declaration cites the reference interface it replaces (file:line).
 * Entries marked NEW have no omCuda* counterpart; their comment states the
 * reference composition they are equivalent to.
 */
#ifndef OMHIP_H
#define OMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== device management (src/cuda/cuda_kernels.cuh:18-34, :63-69, :184) ===== */

/* replaces omCudaInit (cuda_kernels.cuh:18): select device, create the library stream */
int omHipInit(int nDeviceId);
/* replaces omCudaGetDeviceCount (cuda_kernels.cuh:21); returns the count (0 without GPU) */
int omHipGetDeviceCount(void);
/* replaces omCudaGetDeviceName (cuda_kernels.cuh:24) */
int omHipGetDeviceName(int nDeviceId, char* pNameBuf, int nBufSize);
/* replaces omCudaGetMemInfo (cuda_kernels.cuh:27) */
int omHipGetMemInfo(int nDeviceId, size_t* pFreeMem, size_t* pTotalMem);
/* replaces omCudaGetComputeCapability (cuda_kernels.cuh:34): gfx950 reports 9 / 5 */
int omHipGetComputeCapability(int nDeviceId, int* pMajor, int* pMinor);
/* replaces omCudaSynchronize (cuda_kernels.cuh:184): waits for the library stream */
int omHipSynchronize(void);
/* replaces omCudaSyncComputeStream (cuda_kernels.cuh:66) */
int omHipSyncComputeStream(void);
/* replaces omCudaCleanup (cuda_kernels.cuh:69): frees the pool, destroys the stream */
int omHipCleanup(void);
/* replaces omCudaForceReset (cuda_kernels.cu:429-438; EngineBridge's recovery call,
 * src/engine/bridge/EngineBridge.cpp:143, :4047): waits for the whole device, clears the
 * sticky HIP error, then releases what omHipCleanup releases (pool, workspaces, tables,
 * streams) without resetting the device. Device pointers from omHipMalloc are invalid
 * afterwards; the next call initialises the library again. */
int omHipForceReset(void);
/* NEW: the library stream as a hipStream_t (for event timing / interop) */
int omHipGetStream(void** ppStream);
/* NEW: route subsequent work to a caller-owned hipStream_t (NULL restores the
 * library stream). The caller keeps ownership of the stream. Each stream gets its own
 * split-K workspace (kept until omHipCleanup), so work on different streams may overlap.
 * Memory and streams: omHipFree is ordered on the stream current at the free. Work later
 * enqueued on that stream may receive the block at once; work on another stream receives it
 * only after everything enqueued on the freeing stream before the free has finished (an
 * event, no host wait). Work on a third stream that still reads the block at the free must be
 * ordered before the free by the caller. */
int omHipSetStream(void* pStream);
/* NEW: the caller is done with a stream it passed to omHipSetStream (call before destroying
 * it): waits for the stream, returns its workspace to the pool (held back while any executable
 * graph exists) and, if it is the current stream, restores the library stream. Fails (-1)
 * while a graph captured on that stream exists: destroy such graphs first. */
int omHipReleaseStream(void* pStream);
/* NEW: message of the last failing call on this thread ("" if none) */
const char* omHipGetLastError(void);

/* ===== memory (src/cuda/cuda_kernels.cuh:39-60) ===== */

/* replaces omCudaMalloc (cuda_kernels.cuh:39): caching pool, flush-and-retry on OOM */
int omHipMalloc(void** ppDevPtr, size_t nBytes);
/* replaces omCudaFree (cuda_kernels.cuh:42): returns the block to the pool */
int omHipFree(void* pDevPtr);
/* replaces omCudaCopyH2D (cuda_kernels.cuh:45): synchronous */
int omHipCopyH2D(void* pDst, const void* pSrc, size_t nBytes);
/* replaces omCudaCopyD2H (cuda_kernels.cuh:48): synchronous */
int omHipCopyD2H(void* pDst, const void* pSrc, size_t nBytes);
/* replaces omCudaCopyD2D (cuda_kernels.cuh:51): stream-ordered */
int omHipCopyD2D(void* pDst, const void* pSrc, size_t nBytes);
/* replaces omCudaMemset (cuda_kernels.cuh:54): stream-ordered (a fill kernel, so it may
 * sit inside a captured graph) */
int omHipMemset(void* pDev, int nValue, size_t nBytes);
/* NEW: pool statistics: bytes held by the pool, bytes currently handed out */
int omHipPoolStats(size_t* pHeldBytes, size_t* pUsedBytes);
/* NEW: release every cached (free) block back to the driver */
int omHipPoolTrim(void);

/* ===== transfer stream and pinned host memory (cuda_kernels.cuh:56-66, :497-505) ===== */

/* replaces omCudaMallocHost (cuh:501): page-locked host memory (hipHostMalloc), so the
 * asynchronous copies below are true DMA transfers */
int omHipMallocHost(void** ppPtr, size_t nBytes);
/* replaces omCudaFreeHost (cuh:504) */
int omHipFreeHost(void* pPtr);
/* replaces omCudaAsyncCopyH2D (cuh:57): enqueued on the library transfer stream (a second
 * stream, default priority), returns at once; the host buffer must stay valid until the
 * transfer stream is synchronised */
int omHipAsyncCopyH2D(void* pDst, const void* pSrc, size_t nBytes);
/* replaces omCudaAsyncCopyD2H (cuh:60): as above, device to host */
int omHipAsyncCopyD2H(void* pDst, const void* pSrc, size_t nBytes);
/* replaces omCudaSyncTransferStream (cuh:63) */
int omHipSyncTransferStream(void);
/* NEW: work enqueued on the compute stream after this call waits for every transfer
 * enqueued before it (an event, no host wait) */
int omHipComputeWaitTransfer(void);
/* NEW: transfers enqueued after this call wait for the compute work enqueued before it */
int omHipTransferWaitCompute(void);

/* ===== graphs (cuda_kernels.cuh:507-532: omCudaGraph*) ===== */

/* replaces omCudaGraphBeginCapture (cuh:513): records the library calls that follow on the
 * compute stream (the library stream, or the caller stream set by omHipSetStream) instead of
 * running them. Capture a sequence after running it once eagerly on that stream, so that its
 * workspace, lookup tables and pool blocks already exist: a call that would need a larger
 * workspace or a new table during the recording fails (-1, "records a graph"). */
int omHipGraphBeginCapture(void);
/* replaces omCudaGraphEndCapture (cuh:519): ends the recording, returns an executable graph */
int omHipGraphEndCapture(void** ppGraphExec);
/* replaces omCudaGraphLaunch (cuh:524): replays the graph on the stream it was captured on
 * (its nodes use that stream's workspace), so that stream must still exist (omHipReleaseStream
 * refuses to release it while the graph lives). While any executable graph exists, workspaces
 * the library outgrows are kept allocated, so a replay never touches reused memory. */
int omHipGraphLaunch(void* pGraphExec);
/* replaces omCudaGraphDestroy (cuh:528): waits for the device (not for the capture stream, which
 * may be gone by then), then frees the graph */
int omHipGraphDestroy(void* pGraphExec);

/* ===== fills / copy (src/cuda/cuda_kernels.cuh:257-266; CPUBackend cpu_backend.ixx:65-77, :444-446) ===== */

int omHipFillZeros(float* pData, int nCount);                 /* omCudaFillZeros  cuh:257 */
int omHipFillOnes(float* pData, int nCount);                  /* omCudaFillOnes   cuh:260 */
int omHipFillValue(float* pData, int nCount, float fValue);   /* omCudaFillValue  cuh:263 */
int omHipCopy(const float* pSrc, float* pDst, int nCount);    /* omCudaCopy       cuh:266 */

/* ===== activations / bias (cuda_kernels.cuh:91-94, :249) ===== */

/* replaces omCudaReLU (cuh:91): out = x > 0 ? x : 0 (NaN -> 0, -0 -> +0), as cpu_backend.ixx:317-332 */
int omHipReLU(const float* pIn, float* pOut, int nCount);
/* replaces omCudaReLUBackward (cuh:94): gradIn = x > 0 ? gradOut : 0, as cpu_backend.ixx:337-346 */
int omHipReLUBackward(const float* pIn, const float* pGradOut, float* pGradIn, int nCount);
/* replaces omCudaAddBias (cuh:249): out[n,c,hw] = data[n,c,hw] + bias[c].
 * CPUBackend::addBias(A, bias, out, batch, cols) (cpu_backend.ixx:433-440) is
 * the case nN=batch, nC=cols, nHW=1. */
int omHipAddBias(const float* pData, const float* pBias, float* pOut, int nN, int nC, int nHW);

/* ===== softmax, cross-entropy, bias gradient (cuda_kernels.cuh:122, :288, :348, :399) ===== */

/* replaces omCudaSoftmax (cuh:122); CPUBackend::softmax cpu_backend.ixx:352-370: per row of
 * [nBatch, nClasses], exp(x - max) / sum. The row maximum is the reference's scan (NaN
 * elements skipped, a NaN first element kept); exp is the device expf and the sum's order is
 * fixed but not sequential, so elements agree with CPUBackend to a few ulp, not bitwise. */
int omHipSoftmax(const float* pIn, float* pOut, int nBatch, int nClasses);
/* replaces omCudaCrossEntropy (cuh:399) with CPUBackend::crossEntropy's rule
 * (cpu_backend.ixx:375-388; omCudaCrossEntropy's log(p + eps) differs): pResult[0] (device) =
 * -sum of log(max(p, 1e-7)) over the elements whose target exceeds 0.5, divided by nBatch */
int omHipCrossEntropy(const float* pSoftmax, const float* pTarget, float* pResult, int nBatch, int nClasses);
/* replaces omCudaSoftmaxCrossEntropyBackward (cuh:288); CPUBackend::crossEntropySoftmaxBackward
 * cpu_backend.ixx:393-410: grad = (softmax - target) * (1 / nBatch), bit-identical */
int omHipSoftmaxCrossEntropyBackward(const float* pSoftmax, const float* pTarget, float* pGradLogits,
                                     int nBatch, int nClasses);
/* NEW: omHipSoftmax -> omHipCrossEntropy -> omHipSoftmaxCrossEntropyBackward in one launch, each
 * output bit-identical to those calls' (tensorSoftmaxCrossEntropy tensor_ops.ixx:583-633 and
 * SoftmaxCrossEntropyBackward autograd.ixx:440-488 with a loss gradient of 1). pSoftmax, pLoss
 * and pGradLogits may each be NULL (not written). One workgroup: meant for class scores. */
int omHipSoftmaxCrossEntropy(const float* pLogits, const float* pTarget, float* pSoftmax, float* pLoss,
                             float* pGradLogits, int nBatch, int nClasses);
/* replaces omCudaAddBiasBackward (cuh:348): gradBias[c] = sum over n and hw of gradOut[n,c,hw].
 * AddBiasBackward (autograd.ixx:399-433) is the case nN = batch, nC = cols, nHW = 1; for it the
 * rows are added in order from 0, bit-identical to the reference loop, up to 4096 rows (more
 * rows: 16 ordered parts). nHW > 1: a fixed-order reduction per channel. */
int omHipAddBiasBackward(const float* pGradOut, float* pGradBias, int nN, int nC, int nHW);

/* ===== global reductions (cuda_kernels.cuh:127-130) ===== */

/* replaces omCudaSum (cuh:127; CUDABackend::sum om.hal.cuda_backend.ixx:732, called by
 * tensorSum tensor_ops.ixx:409-440): pResult[0] (device) = sum of pData[0..nCount). The
 * order is fixed (contiguous chunks, then the chunk sums), so repeated calls agree bit for
 * bit; against CPUBackend::sum's sequential loop (cpu_backend.ixx:290-294) the difference is
 * rounding only. nCount <= 0 writes 0. */
int omHipSum(const float* pData, float* pResult, int nCount);
/* replaces omCudaMean (cuh:130): the sum of omHipSum multiplied by 1.0f / nCount
 * (cuda_kernels.cu:1506-1513); nCount <= 0 writes 0. */
int omHipMean(const float* pData, float* pResult, int nCount);

/* ===== ViT attention, fp32 (cuda_kernels.cuh:488-495) ===== */

/* replaces omCudaQkvSplitHeads (cuh:488; CUDABackend::qkvSplitHeads om.hal.cuda_backend.ixx:967):
 * pQkv [nBatch*nSeqLen, 3*D] (D = nHeads*nHeadDim, each token's row Q | K | V) ->
 * pQ, pK, pV [nBatch*nHeads, nSeqLen, nHeadDim] with Q multiplied by fScale — the index maps
 * of MultiHeadAttention::forward's CPU branch (vit.ixx:196-212), bit-identical. */
int omHipQkvSplitHeads(const float* pQkv, float* pQ, float* pK, float* pV, int nBatch, int nSeqLen, int nHeads,
                       int nHeadDim, float fScale);
/* replaces omCudaMergeHeads (cuh:493; CUDABackend::mergeHeads om.hal.cuda_backend.ixx:977):
 * pIn [nBatch*nHeads, nSeqLen, nHeadDim] -> pOut [nBatch*nSeqLen, nHeads*nHeadDim]
 * (vit.ixx:220-232), bit-identical. */
int omHipMergeHeads(const float* pIn, float* pOut, int nBatch, int nSeqLen, int nHeads, int nHeadDim);
/* NEW: the attention core of MultiHeadAttention::forward's GPU branch on fp32 data
 * (vit.ixx:163-187): qkvSplitHeads (Q times fScale), tensorTranspose2dBatched +
 * tensorBatchedMatmul (Q K^T), tensorSoftmaxLastDim, tensorBatchedMatmul (P V),
 * mergeHeads. pQKV [nBatch*nSeq, 3*D] -> pOut [nBatch*nSeq, D], both fp32. Q is scaled as
 * qkvSplitHeads scales it; the products read the heads where they lie (no transpose or split
 * copy) and accumulate in fp32; the softmax is omHipSoftmax's. Intermediates use the
 * stream's staging workspace. */
int omHipAttention(const float* pQKV, float* pOut, int nBatch, int nSeq, int nHeads, int nHeadDim, float fScale);

/* ===== fp32 GEMM (cuda_kernels.cuh:109-117) ===== */

/* replaces omCudaMatmul (cuh:109): C[M,N] = A[M,K] * B[K,N] (CPUBackend::matmul cpu_backend.ixx:239-286) */
int omHipMatmul(const float* pA, const float* pB, float* pC, int nM, int nK, int nN);
/* NEW: C[M,N] = A[M,K] * B[N,K]^T  (Linear-weight layout). Reference composition:
 * transpose2d(B, Bt, N, K); matmul(A, Bt, C, M, K, N)  (cpu_backend.ixx:1535-1539, :239-286;
 * used by MatMulBackward autograd.ixx:261-273) */
int omHipMatmulTransB(const float* pA, const float* pB, float* pC, int nM, int nK, int nN);
/* NEW: C[M,N] = A[K,M]^T * B[K,N]. Reference composition: transpose2d(A, At, K, M);
 * matmul(At, B, C, M, K, N)  (the dB half of MatMulBackward autograd.ixx:276-286) */
int omHipMatmulTransA(const float* pA, const float* pB, float* pC, int nM, int nK, int nN);
/* NEW: out[M,N] = act(A[M,K] * W[K,N] + bias[N]) in one pass (bias nullable; nAct 0
 * identity, 1 ReLU). Reference composition: Linear::forward's tensorMatmul +
 * tensorAddBias (linear.ixx:50-58, tensor_ops.ixx:305-349, :542-576) followed by
 * tensorReLU (tensor_ops.ixx:511-536); each element is the unfused chain's value:
 * the same sum, then + bias, then x > 0 ? x : 0. */
int omHipLinearBiasAct(const float* pA, const float* pW, const float* pBias, float* pOut, int nM, int nK, int nN,
                       int nAct);
/* NEW: a Linear layer's backward in one launch. From X [nBatch, nIn] (the layer's input),
 * G [nBatch, nOut] (the gradient of its output) and W [nIn, nOut]:
 *   pGradWeight [nIn, nOut] = X^T G            (MatMulBackward's dB half, autograd.ixx:276-286)
 *   pGradBias   [nOut]      = column sums of G (AddBiasBackward, autograd.ixx:399-433; nullable)
 *   pGradInput  [nBatch, nIn] = G W^T          (MatMulBackward's dA half, autograd.ixx:261-273; nullable)
 * and, when pGate (the previous layer's ReLU output [nBatch, nIn]) is given, pGradInput is
 * gated as omHipReLUBackward(pGate, G W^T) would gate it (cpu_backend.ixx:337-346): the
 * ReLU backward of the layer below fused into the product. Every element equals the separate
 * entries' value whenever their products do not split K (each output tile here sums K in
 * one pass, in the same order). */
int omHipLinearBackward(const float* pInput, const float* pGradOut, const float* pWeight, const float* pGate,
                        float* pGradWeight, float* pGradBias, float* pGradInput, int nBatch, int nIn, int nOut);
/* NEW: the classifier head of a training step in one launch — Linear (tensorMatmul + addBias,
 * linear.ixx:50-58) -> tensorSoftmaxCrossEntropy (tensor_ops.ixx:583-633) -> their backward
 * (SoftmaxCrossEntropyBackward autograd.ixx:440-488, AddBiasBackward :399-433, MatMulBackward
 * :261-286) and, when pGate is given, the ReLU backward of the layer below. From X [nBatch, nIn],
 * W [nIn, nClasses], b [nClasses] (nullable) and one-hot targets T [nBatch, nClasses]:
 *   logits = X W + b, p = softmax(logits), loss = mean -log(max(p_target, 1e-7)),
 *   g = (p - T) / nBatch, gW = X^T g, gb = column sums of g, gX = g W^T (kept where pGate > 0).
 * pLogits, pLoss, pGradLogits, pGradBias, pGradInput and pGate may be NULL. Heads of at most
 * 64 classes run one kernel: the whole batch in one workgroup when its padded operands fit
 * 128 KB of LDS (the 784-256-128-10 MLP's 128 x 128 x 10 head), otherwise a workgroup per block
 * of 64, 32 or 16 rows whose weight-gradient parts the last one to finish adds in block order
 * (nBatch * (nClasses + 1) floats within 128 KB). The products' summation order differs from
 * omHipLinearBiasAct / omHipLinearBackward (within the fp32 bar); the softmax adds a row's
 * exponentials in class order as the reference's loops (omHipSoftmaxCrossEntropy reduces a row
 * across a wave: p agrees within a few ulp); gb and the loss add the rows in order from 0.
 * Larger heads run those three entries. Calls on one stream run in order; this entry shares
 * the library's workspace and arrival counters with the other entries. */
int omHipLinearSoftmaxCrossEntropyStep(const float* pInput, const float* pWeight, const float* pBias,
                                       const float* pTarget, const float* pGate, float* pLogits, float* pLoss,
                                       float* pGradLogits, float* pGradWeight, float* pGradBias, float* pGradInput,
                                       int nBatch, int nIn, int nClasses);
/* replaces omCudaBatchedMatmul (cuh:112): C[b] = A[b] * B[b], strides M*K, K*N, M*N
 * (CPUBackend::batchedMatmul cpu_backend.ixx:1520-1532) */
int omHipBatchedMatmul(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN);
/* NEW: C[b] = A[b] * B[b]^T with B[b] stored [N,K]; reference composition:
 * tensorTranspose2dBatched + batchedMatmul (tensor_ops.ixx:1588-1625, :1561-1582; vit.ixx:175-176) */
int omHipBatchedMatmulTransB(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN);
/* NEW: general strided-batched fp32 GEMM. transA/transB select A[K,M] / B[N,K]
 * storage; lda/ldb/ldc are row strides in elements; strides are per-batch element
 * offsets (0 shares an operand across the batch). */
int omHipGemmStridedBatched(int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                            const float* pA, long long nLda, long long nStrideA,
                            const float* pB, long long nLdb, long long nStrideB,
                            float* pC, long long nLdc, long long nStrideC);
/* NEW, no counterpart in the reference: omHipGemmStridedBatched for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and the same results, bit for bit; it calls no hipMalloc,
 * hipFree or allocating library routine: its split-K partial sums go to a fixed 32 MiB device
 * array that each GPU the library runs on holds until the process ends (every split plan of a
 * 256-CU device fits; a plan that would need more fails with -1 and a message). All calls on
 * one GPU share that array, so calls that overlap on one GPU (on different streams, or from
 * several threads) race: order them. */
int omHipGemmStridedBatchedNoAlloc(int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                                   const float* pA, long long nLda, long long nStrideA,
                                   const float* pB, long long nLdb, long long nStrideB,
                                   float* pC, long long nLdc, long long nStrideC);
/* replaces omCudaTranspose (cuh:117): out[c,r] = in[r,c]; CPUBackend::transpose2d cpu_backend.ixx:1535-1539 */
int omHipTranspose(const float* pIn, float* pOut, int nRows, int nCols);

/* ===== conv2d / batchnorm (cuda_kernels.cuh:136-146, :165-170) =====
 * Size limits of the implicit-GEMM convolutions (forward, fused and gradient
 * entries): one image's input with its padding margin below 2^29 bytes, one
 * image's output at most 2^30 bytes, the weights at most 2^30 bytes,
 * KH, KW < 65536 and H + pad, W + pad < 65535. Larger batches are processed in
 * chunks internally; a call outside these limits returns -1 with a message. */

/* replaces omCudaConv2d (cuh:136): NCHW conv, symmetric stride/pad, dilation 1,
 * groups 1; pBias may be NULL. CPUBackend::conv2d cpu_backend.ixx:619-658 */
int omHipConv2d(const float* pInput, const float* pWeight, const float* pBias, float* pOutput,
                int nBatch, int nCin, int nH, int nW,
                int nCout, int nKH, int nKW, int nStride, int nPad);
/* replaces omCudaConv2dIm2col (cuh:142): same result as omHipConv2d via an explicit
 * im2col buffer followed by a shared-weight batched GEMM */
int omHipConv2dIm2col(const float* pInput, const float* pWeight, const float* pBias, float* pOutput,
                      int nBatch, int nCin, int nH, int nW,
                      int nCout, int nKH, int nKW, int nStride, int nPad);
/* NEW: conv2d + bias + BatchNorm(inference) + activation in one kernel.
 * Reference composition: conv2d (cpu_backend.ixx:619-658) -> batchNorm2d(bTraining=false)
 * (cpu_backend.ixx:781-842, eval branch 823-840) -> relu (cpu_backend.ixx:317-332).
 * pBias may be NULL; pGamma/pBeta/pMean/pVar may all be NULL (no BN);
 * nAct: 0 = identity, 1 = ReLU. */
int omHipConv2dBiasBnAct(const float* pInput, const float* pWeight, const float* pBias,
                         const float* pGamma, const float* pBeta,
                         const float* pMean, const float* pVar, float fEps, int nAct,
                         float* pOutput,
                         int nBatch, int nCin, int nH, int nW,
                         int nCout, int nKH, int nKW, int nStride, int nPad);
/* NEW: im2col of one image, col[(c*KH+kh)*KW+kw, oh*Wout+ow]; CPUBackend::im2col cpu_backend.ixx:544-575 */
int omHipIm2col(const float* pInput, int nCin, int nH, int nW, int nKH, int nKW,
                int nPadH, int nPadW, int nStrideH, int nStrideW, float* pCol);
/* replaces omCudaBatchNorm2d (cuh:165); CPUBackend::batchNorm2d cpu_backend.ixx:781-842.
 * bTraining == 0: y = gamma*((x-runMean)*invStd)+beta, invStd = 1/sqrt(runVar+eps),
 * savedMean/savedInvStd (may be NULL) = runMean and invStd (:823-840).
 * bTraining != 0: batch mean and biased variance (two passes, :796-810), savedMean /
 * savedInvStd (may be NULL), runMean/runVar = (1-momentum)*run + momentum*batch (:818-821),
 * y normalised with the batch statistics. */
int omHipBatchNorm2d(const float* pInput, float* pOutput,
                     const float* pGamma, const float* pBeta,
                     float* pRunMean, float* pRunVar,
                     float* pSavedMean, float* pSavedInvStd,
                     int nBatch, int nChannels, int nH, int nW,
                     float fEps, float fMomentum, int bTraining);

/* ===== conv2d / batchnorm training (cuda_kernels.cuh:295-316) ===== */

/* replaces omCudaConv2dBackwardInput (cuh:295); CPUBackend::conv2dBackwardInput
 * cpu_backend.ixx:666-705. pGradInput [N,Cin,H,W] is overwritten. */
int omHipConv2dBackwardInput(const float* pGradOutput, const float* pWeight, float* pGradInput,
                             int nBatch, int nCin, int nH, int nW,
                             int nCout, int nKH, int nKW, int nStride, int nPad);
/* replaces omCudaConv2dBackwardWeight (cuh:301); CPUBackend::conv2dBackwardWeight
 * cpu_backend.ixx:710-772. pGradWeight [Cout,Cin,KH,KW] and pGradBias [Cout] (may be
 * NULL) are overwritten with the sums over the batch. */
int omHipConv2dBackwardWeight(const float* pInput, const float* pGradOutput,
                              float* pGradWeight, float* pGradBias,
                              int nBatch, int nCin, int nH, int nW,
                              int nCout, int nKH, int nKW, int nStride, int nPad);
/* replaces omCudaBatchNorm2dBackward (cuh:310); CPUBackend::batchNorm2dBackward
 * cpu_backend.ixx:847-890 with the saved mean / inverse std of the training forward.
 * pGradGamma / pGradBeta may be NULL. fEps is unused (pInvStd already holds it). */
int omHipBatchNorm2dBackward(const float* pGradOutput, const float* pInput,
                             const float* pMean, const float* pInvStd, const float* pGamma,
                             float* pGradInput, float* pGradGamma, float* pGradBeta,
                             int nBatch, int nChannels, int nH, int nW, float fEps);
/* NEW: the training forward of a conv block tail in one pass: y = act(BN_train(x)
 * [+ pResidual]) — the reference's batchNorm2d (training) then add then relu
 * (cpu_backend.ixx:796-840, :147-160, :317-332; BasicBlock resnet.ixx:55-79), each
 * rounded as there, so the result is bit-identical to the three calls. Statistics
 * and running averages as omHipBatchNorm2d in training mode; pResidual may be NULL,
 * nAct 0 identity / 1 ReLU. */
int omHipBatchNorm2dTrainAct(const float* pInput, float* pOutput, const float* pGamma, const float* pBeta,
                             float* pRunningMean, float* pRunningVar, float* pSavedMean, float* pSavedInvStd,
                             int nBatch, int nChannels, int nH, int nW, float fEps, float fMomentum,
                             const float* pResidual, int nAct);
/* NEW: omHipBatchNorm2dBackward of the gradient gated by a ReLU,
 * gradOut' = reluInput > 0 ? gradOut : 0 (cpu_backend.ixx:337-346) — bit-identical to
 * omHipReLUBackward followed by omHipBatchNorm2dBackward, without the gated tensor. */
int omHipBatchNorm2dBackwardRelu(const float* pGradOutput, const float* pReluInput, const float* pInput,
                                 const float* pMean, const float* pInvStd, const float* pGamma,
                                 float* pGradInput, float* pGradGamma, float* pGradBeta,
                                 int nBatch, int nChannels, int nH, int nW, float fEps);

/* ===== pooling and the residual sum (cuda_kernels.cuh:218-245, :74) ===== */

/* replaces omCudaMaxPool2d (cuh:218); CPUBackend::maxPool2d cpu_backend.ixx:897-934:
 * first maximum (strict >) in (kh, kw) order; pIndices (may be NULL) receives the flat
 * input index ((n*C+c)*H+ih)*W+iw, -1 for a window wholly in the padding (value -1e30). */
int omHipMaxPool2d(const float* pIn, float* pOut, int* pIndices,
                   int nN, int nC, int nH, int nW,
                   int nKH, int nKW, int nSH, int nSW, int nPH, int nPW);
/* replaces omCudaMaxPool2dBackward (cuh:224); CPUBackend::maxPool2dBackward
 * cpu_backend.ixx:937-955: pGradIn zeroed, then gradients scattered through the
 * indices. An input that is the maximum of several windows receives their
 * gradients in an unspecified order (atomic adds). */
int omHipMaxPool2dBackward(const float* pGradOut, const int* pIndices, float* pGradIn,
                           int nN, int nC, int nH, int nW, int nHout, int nWout);
/* NEW: as omHipMaxPool2dBackward with the window geometry given, computed as an
 * ordered gather: bit-identical to CPUBackend::maxPool2dBackward. */
int omHipMaxPool2dBackwardEx(const float* pGradOut, const int* pIndices, float* pGradIn,
                             int nN, int nC, int nH, int nW,
                             int nKH, int nKW, int nSH, int nSW, int nPH, int nPW);
/* replaces omCudaAvgPool2d (cuh:230); CPUBackend::avgPool2d cpu_backend.ixx:958-990
 * (sum of the valid taps / (KH*KW)) */
int omHipAvgPool2d(const float* pIn, float* pOut, int nN, int nC, int nH, int nW,
                   int nKH, int nKW, int nSH, int nSW, int nPH, int nPW);
/* replaces omCudaAvgPool2dBackward (cuh:236); CPUBackend::avgPool2dBackward
 * cpu_backend.ixx:994-1023; pGradIn [N,C,H,W] is overwritten */
int omHipAvgPool2dBackward(const float* pGradOut, float* pGradIn, int nN, int nC, int nH, int nW,
                           int nKH, int nKW, int nSH, int nSW, int nPH, int nPW);
/* replaces omCudaAdaptiveAvgPool2d (cuh:242); CPUBackend::adaptiveAvgPool2d
 * cpu_backend.ixx:1467-1488 (regions [floor(o*H/OH), floor((o+1)*H/OH))) */
int omHipAdaptiveAvgPool2d(const float* pIn, float* pOut, int nN, int nC, int nH, int nW,
                           int nOutH, int nOutW);
/* NEW: CPUBackend::adaptiveAvgPool2dBackward cpu_backend.ixx:1491-1510 */
int omHipAdaptiveAvgPool2dBackward(const float* pGradOut, float* pGradIn, int nN, int nC, int nH, int nW,
                                   int nOutH, int nOutW);
/* replaces omCudaAdd (cuh:74); CPUBackend::add cpu_backend.ixx:147-160 */
int omHipAdd(const float* pA, const float* pB, float* pC, int nCount);
/* NEW: out = a + (x > 0 ? gradOut : 0) — CPUBackend::add of a and reluBackward(x, gradOut)
 * (cpu_backend.ixx:147-160, :337-346) in one pass, bit-identical: the identity shortcut's
 * share of a residual block's backward. */
int omHipAddReluBackward(const float* pA, const float* pIn, const float* pGradOut, float* pOut, int nCount);
/* NEW: omHipConv2dBiasBnAct with the residual added after BN and before the
 * activation: out = act(BN(conv(x) + bias) + residual). Reference composition: the
 * BasicBlock / Bottleneck tail bn2(conv2(.)) + shortcut -> relu (resnet.ixx:55-79,
 * resnet50.ixx:57-83). pResidual [N,Cout,Ho,Wo] must not alias pOutput. */
int omHipConv2dBiasBnAddAct(const float* pInput, const float* pWeight, const float* pBias,
                            const float* pGamma, const float* pBeta,
                            const float* pMean, const float* pVar, float fEps,
                            const float* pResidual, int nAct, float* pOutput,
                            int nBatch, int nCin, int nH, int nW,
                            int nCout, int nKH, int nKW, int nStride, int nPad);

/* ===== fp16 / bf16 GEMM, fp32 accumulate (NEW; the reference has only the software
 * converter om.engine.fp16.ixx:36-164) ===== */

/* NEW: fp32 -> IEEE binary16 / bfloat16, round-to-nearest-even; and back */
int omHipConvertF32ToF16(const float* pIn, uint16_t* pOut, int nCount);
int omHipConvertF32ToBF16(const float* pIn, uint16_t* pOut, int nCount);
int omHipConvertF16ToF32(const uint16_t* pIn, float* pOut, int nCount);
int omHipConvertBF16ToF32(const uint16_t* pIn, float* pOut, int nCount);
/* NEW: C[M,N] (fp32) = A[M,K] * B[K,N], A/B binary16. Reference composition:
 * halfToFloat(A), halfToFloat(B), matmul (fp16.ixx:103-164, cpu_backend.ixx:239-286) */
int omHipMatmulF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN);
/* NEW: as omHipMatmulF16 with bfloat16 inputs */
int omHipMatmulBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN);
/* NEW: C = A * B^T with B stored [N,K] (Linear weight layout), fp16 / bf16 inputs */
int omHipMatmulTransBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN);
int omHipMatmulTransBBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN);
/* NEW: general strided-batched half-precision GEMM with fp32 output.
 * nDtype: 0 = binary16, 1 = bfloat16. Layout arguments as omHipGemmStridedBatched. */
int omHipGemmStridedBatchedHalf(int nDtype, int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                                const uint16_t* pA, long long nLda, long long nStrideA,
                                const uint16_t* pB, long long nLdb, long long nStrideB,
                                float* pC, long long nLdc, long long nStrideC);

/* NEW: half-precision Linear, out = act(x W + b) with fp32 accumulate (Linear::forward
 * linear.ixx:50-58: tensorMatmul then tensorAddBias, on halfToFloat inputs; ReLU after the
 * bias as omHipLinearBiasAct). pInput [nM, nK] and pWeight in nDtype (0 binary16, 1
 * bfloat16): [nK, nN] as Linear stores it (bTransW 0), or [nN, nK] (bTransW 1); pBias [nN]
 * fp32 or NULL; nAct 0 none, 1 ReLU; pOutput [nM, nN] fp32 (nOutHalf 0) or nDtype rounded to
 * nearest even (nOutHalf 1) — bit-identical to the fp32 output followed by
 * omHipConvertF32ToF16 / omHipConvertF32ToBF16 for finite values. */
int omHipLinearHalf(int nDtype, const uint16_t* pInput, const uint16_t* pWeight, int bTransW, const float* pBias,
                    int nAct, void* pOutput, int nOutHalf, int nM, int nK, int nN);
/* NEW: fused multi-head attention on half-precision inputs (QKV split with Q scaled,
 * Q x K^T, softmax over the keys, P x V, head merge). Reference composition:
 * MultiHeadAttention::forward vit.ixx:150-239 after the QKV projection —
 * qkvSplitHeads, tensorTranspose2dBatched + tensorBatchedMatmul, tensorSoftmaxLastDim
 * (CPUBackend::softmax cpu_backend.ixx:352-370), tensorBatchedMatmul, mergeHeads.
 * pQKV [nBatch*nSeq, 3*nHeads*nHeadDim] in nDtype (0 binary16, 1 bfloat16), 16-byte
 * aligned; pOut [nBatch*nSeq, nHeads*nHeadDim], fp32 (nOutHalf 0) or nDtype (1).
 * fScale multiplies the scores (1/sqrt(nHeadDim) for ViT). nHeadDim must be 64 and
 * nSeq <= 384. P is rounded to nDtype before P x V (fp32 accumulate). */
int omHipAttentionHalf(int nDtype, const uint16_t* pQKV, void* pOut, int nOutHalf,
                       int nBatch, int nSeq, int nHeads, int nHeadDim, float fScale);
/* NEW: MultiHeadAttention::forward (vit.ixx:150-239) on half-precision activations and
 * weights, fp32 accumulate: qkv = x Wqkv + bqkv; heads split with Q scaled by
 * 1/sqrt(nHeadDim); softmax(Q K^T) V; heads merged; out = ctx Wout + bout.
 * pX [nBatch*nSeq, nDim] in nDtype, nDim = nHeads*nHeadDim; pWqkv [nDim, 3*nDim] and pWout
 * [nDim, nDim] in nDtype, stored [in, out] as Linear (linear.ixx:31); pBqkv [3*nDim] and
 * pBout [nDim] fp32 or NULL; pOut [nBatch*nSeq, nDim] fp32 (nOutHalf 0) or nDtype (1).
 * nHeadDim 64 with nSeq <= 384 runs fused: the projection is rounded to nDtype, then
 * omHipAttentionHalf (P rounded to nDtype), its context rounded to nDtype. Other shapes
 * run the reference's unfused chain in fp32 (projection, Q scaled, Q K^T, softmax, P V,
 * merged heads) with the context rounded to nDtype for the output projection.
 * Intermediates use the library's per-stream workspace. */
int omHipMultiHeadAttentionHalf(int nDtype, const uint16_t* pX, const uint16_t* pWqkv, const float* pBqkv,
                                const uint16_t* pWout, const float* pBout, void* pOut, int nOutHalf,
                                int nBatch, int nSeq, int nHeads, int nHeadDim);

/* ===== device-resident inference (EngineBridge::inferBatch, EngineBridge.cpp:3525-3772) ===== */

/* NEW: a ResNet-18 classifier (torchvision layout, 3x224x224 input) resident on the device,
 * every conv with its BatchNorm (running statistics) and ReLU fused, the shortcut fused into
 * the second conv of each block. pParams (host) holds nParamFloats floats: for each conv in
 * network order — stem 7x7/2, then per BasicBlock conv1, conv2 and (first block of stages
 * 2-4) the 1x1/2 downsample — weight [Cout][Cin][K][K], BN gamma, beta, running mean,
 * running var [Cout]; then the FC weight [512][nClasses] and bias [nClasses]. Buffers are
 * sized for nMaxBatch images (at most 32, the reference's batch limit). */
int omHipResNet18Create(const float* pParams, long long nParamFloats, int nClasses, int nMaxBatch, void** ppNet);
/* NEW: waits for the net's work and frees it */
int omHipResNet18Destroy(void* pNet);
/* NEW: logits [nBatch, nClasses] (device) of nBatch normalised images (device) */
int omHipResNet18Forward(void* pNet, const float* pInput, float* pLogits, int nBatch);
/* NEW: the inferBatch pipeline: pImages (host) [nImages][nC][nH][nW] in batches of
 * nBatchSize (clamped to [1, 32]); each batch is staged in page-locked memory and uploaded
 * on the transfer stream while the previous batch computes; nNormPreset 1 applies the
 * ImageNet normalisation of normalizeImage (data_pipeline.ixx:744-803) on the device (0:
 * none). Per image, as the reference's classification branch: softmax of the logits,
 * pClasses = argmax (-1 when the top probability is below fConfThreshold), pConfidences =
 * top probability, pProbs [nImages][nClasses] (may be NULL). */
int omHipResNet18InferBatch(void* pNet, const float* pImages, int nImages, int nC, int nH, int nW, int nBatchSize,
                            int nNormPreset, float fConfThreshold, int* pClasses, float* pConfidences,
                            float* pProbs);

#ifdef __cplusplus
}
#endif

#endif /* OMHIP_H */
