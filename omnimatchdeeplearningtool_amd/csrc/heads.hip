// heads.hip — the fp32 pieces of the engine's ViT attention and of tensorSum:
//   * QKV split into heads with Q scaled, and the head merge
//     (CUDABackend::qkvSplitHeads / mergeHeads, src/hal/om.hal.cuda_backend.ixx:967-985,
//     omCudaQkvSplitHeads / omCudaMergeHeads src/cuda/cuda_kernels.cuh:488-495; the
//     CPU branch of MultiHeadAttention::forward, src/engine/om.engine.vit.ixx:196-233,
//     states the same index maps);
//   * the global sum and mean (CUDABackend::sum om.hal.cuda_backend.ixx:732,
//     omCudaSum / omCudaMean cuda_kernels.cuh:127-130) behind tensorSum
//     (src/engine/om.engine.tensor_ops.ixx:409-440);
//   * attention on an fp32 QKV projection (the GPU branch of
//     MultiHeadAttention::forward, vit.ixx:163-187) composed from the library's
//     strided GEMM and row softmax.
//
// The split and merge are pure permutations (plus one fp32 multiply for Q), so
// they are HBM streams: each thread moves 4 consecutive features of one token
// with 16-byte loads and stores when the head dimension and the pointers allow
// it; a token's 3D inputs are read contiguously and each head's d features are
// written as one contiguous run.
//
// The sum is two fixed-order stages (each workgroup adds a contiguous chunk:
// per-thread strided sums, a butterfly inside each wave, the waves in index
// order; then one workgroup adds the chunk sums the same way), so the result
// depends only on the input and the device's CU count, not on timing.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kSumThreads = 256;
constexpr int kSumPerBlock = 4096;   // elements per workgroup before the grid is capped

__device__ __forceinline__ float waveSum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum of the workgroup's per-thread values: butterfly per wave, then the
// waves in index order (thread 0 holds the result).
__device__ __forceinline__ float blockSum(float v, float* lds) {
    v = waveSum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    float t = 0.f;
    if (threadIdx.x == 0)
        for (int w = 0; w < kSumThreads / 64; ++w) t += lds[w];
    return t;
}

}  // namespace

// ---- QKV split / head merge ------------------------------------------------
// qkv [B*S, 3D] -> q, k, v [B*H, S, dh] (D = H*dh), q = qkv * scale.
// Work item i covers 4 features (VEC) or 1 feature of one token:
// token = i / D_, c = i % D_ in units of the item width.
template <bool VEC>
__global__ void qkv_split_kernel(const float* __restrict__ qkv, float* __restrict__ q, float* __restrict__ k,
                                 float* __restrict__ v, int tokens, int S, int H, int dh, float scale) {
    const int D = H * dh;
    const int W = VEC ? 4 : 1;
    const int perTok = D / W;
    const long long total = (long long)tokens * perTok;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int tok = (int)(i / perTok);
        const int c = (int)(i - (long long)tok * perTok) * W;
        const int h = c / dh, d = c - h * dh;
        const int n = tok / S, s = tok - n * S;
        const long long src = (long long)tok * 3 * D + c;
        const long long dst = (((long long)n * H + h) * S + s) * dh + d;
        if constexpr (VEC) {
            f4 a = *reinterpret_cast<const f4*>(qkv + src);
            const f4 b = *reinterpret_cast<const f4*>(qkv + src + D);
            const f4 e = *reinterpret_cast<const f4*>(qkv + src + 2 * D);
            a[0] = a[0] * scale; a[1] = a[1] * scale; a[2] = a[2] * scale; a[3] = a[3] * scale;
            *reinterpret_cast<f4*>(q + dst) = a;
            *reinterpret_cast<f4*>(k + dst) = b;
            *reinterpret_cast<f4*>(v + dst) = e;
        } else {
            q[dst] = qkv[src] * scale;
            k[dst] = qkv[src + D];
            v[dst] = qkv[src + 2 * D];
        }
    }
}

// in [B*H, S, dh] -> out [B*S, D]
template <bool VEC>
__global__ void merge_heads_kernel(const float* __restrict__ in, float* __restrict__ out, int tokens, int S, int H,
                                   int dh) {
    const int D = H * dh;
    const int W = VEC ? 4 : 1;
    const int perTok = D / W;
    const long long total = (long long)tokens * perTok;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int tok = (int)(i / perTok);
        const int c = (int)(i - (long long)tok * perTok) * W;
        const int h = c / dh, d = c - h * dh;
        const int n = tok / S, s = tok - n * S;
        const long long src = (((long long)n * H + h) * S + s) * dh + d;
        const long long dst = (long long)tok * D + c;
        if constexpr (VEC)
            *reinterpret_cast<f4*>(out + dst) = *reinterpret_cast<const f4*>(in + src);
        else
            out[dst] = in[src];
    }
}

// Multiplies x[r, c] (c < cols, row stride ld) by scale into y[r, c] (row stride cols).
__global__ void scale_copy_kernel(const float* __restrict__ x, float* __restrict__ y, int rows, int ld, int cols,
                                  float scale) {
    const long long total = (long long)rows * cols;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int r = (int)(i / cols);
        const int c = (int)(i - (long long)r * cols);
        y[i] = x[(long long)r * ld + c] * scale;
    }
}

// ---- global sum ------------------------------------------------------------
// Stage 1: workgroup b adds elements [b*chunk, min(n, (b+1)*chunk)).
template <bool VEC>
__global__ void __launch_bounds__(kSumThreads) sum_chunks_kernel(const float* __restrict__ x, long long n,
                                                                long long chunk, float* __restrict__ part,
                                                                float* __restrict__ result, float post) {
    __shared__ float lds[kSumThreads / 64];
    const long long lo = blockIdx.x * chunk;
    const long long hi = std::min(n, lo + chunk);
    float acc = 0.f;
    if constexpr (VEC) {   // chunk and x are 16-byte aligned multiples
        const long long hi4 = lo + (hi - lo) / 4 * 4;
        for (long long i = lo + 4 * (long long)threadIdx.x; i < hi4; i += 4 * kSumThreads) {
            const f4 v = *reinterpret_cast<const f4*>(x + i);
            acc += v[0];
            acc += v[1];
            acc += v[2];
            acc += v[3];
        }
        for (long long i = hi4 + threadIdx.x; i < hi; i += kSumThreads) acc += x[i];
    } else {
        for (long long i = lo + threadIdx.x; i < hi; i += kSumThreads) acc += x[i];
    }
    const float t = blockSum(acc, lds);
    if (threadIdx.x == 0) {
        if (result) result[0] = t * post;   // a single workgroup finishes the sum itself
        else part[blockIdx.x] = t;
    }
}

// Stage 2: one workgroup adds the chunk sums in the same fixed order.
__global__ void __launch_bounds__(kSumThreads) sum_parts_kernel(const float* __restrict__ part, int nPart,
                                                               float* __restrict__ result, float post) {
    __shared__ float lds[kSumThreads / 64];
    float acc = 0.f;
    for (int i = threadIdx.x; i < nPart; i += kSumThreads) acc += part[i];
    const float t = blockSum(acc, lds);
    if (threadIdx.x == 0) result[0] = t * post;
}

namespace {

int gridFor(long long items) {
    const long long cap = (long long)cuCount() * 16;
    return (int)std::max<long long>(1, std::min<long long>((items + 255) / 256, cap));
}

// result[0] = (sum of x[0..n)) * post, in two fixed-order stages.
int sumTo(const char* name, const float* x, float* result, int n, float post) {
    if (!result) return fail("%s: null result", name);
    if (n <= 0) return byteFill(result, 0, sizeof(float));
    if (!x) return fail("%s: null input", name);
    const long long N = n;
    const int maxParts = cuCount() * 4;
    long long parts = std::min<long long>((N + kSumPerBlock - 1) / kSumPerBlock, maxParts);
    long long chunk = (N + parts - 1) / parts;
    chunk = (chunk + 3) / 4 * 4;                    // chunks start on 16-byte boundaries
    parts = (N + chunk - 1) / chunk;
    const bool vec = al16(x);
    const hipStream_t s = stream();
    if (parts == 1) {
        if (vec)
            hipLaunchKernelGGL(sum_chunks_kernel<true>, dim3(1), dim3(kSumThreads), 0, s, x, N, chunk, nullptr, result,
                               post);
        else
            hipLaunchKernelGGL(sum_chunks_kernel<false>, dim3(1), dim3(kSumThreads), 0, s, x, N, chunk, nullptr,
                               result, post);
        OMHIP_CHECK_LAUNCH();
        return 0;
    }
    float* part = static_cast<float*>(workspace((size_t)parts * sizeof(float), kWsPartials));
    if (!part) return -1;   // workspace() recorded the cause
    if (vec)
        hipLaunchKernelGGL(sum_chunks_kernel<true>, dim3((unsigned)parts), dim3(kSumThreads), 0, s, x, N, chunk, part,
                           nullptr, 1.0f);
    else
        hipLaunchKernelGGL(sum_chunks_kernel<false>, dim3((unsigned)parts), dim3(kSumThreads), 0, s, x, N, chunk, part,
                           nullptr, 1.0f);
    OMHIP_CHECK_LAUNCH();
    hipLaunchKernelGGL(sum_parts_kernel, dim3(1), dim3(kSumThreads), 0, s, part, (int)parts, result, post);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int checkHeads(const char* name, int nBatch, int nSeq, int nHeads, int nHeadDim) {
    const long long total = (long long)nBatch * nSeq * nHeads * nHeadDim;
    if (total * 3 > 0x7fffffffLL)
        return fail("%s: %d x %d tokens x 3 x %d x %d features exceed the 2^31-element limit", name, nBatch, nSeq,
                    nHeads, nHeadDim);
    return 0;
}

constexpr size_t kAlign = 256;
size_t up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

}  // namespace

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipQkvSplitHeads(const float* pQkv, float* pQ, float* pK, float* pV, int nBatch, int nSeqLen, int nHeads,
                       int nHeadDim, float fScale) {
    const char* name = "omHipQkvSplitHeads";
    clearError();
    if (nBatch <= 0 || nSeqLen <= 0 || nHeads <= 0 || nHeadDim <= 0) return 0;
    if (!pQkv || !pQ || !pK || !pV) return fail("%s: null pointer", name);
    if (checkHeads(name, nBatch, nSeqLen, nHeads, nHeadDim)) return -1;
    const int tokens = nBatch * nSeqLen;
    const bool vec = nHeadDim % 4 == 0 && al16(pQkv) && al16(pQ) && al16(pK) && al16(pV);
    const long long items = (long long)tokens * nHeads * nHeadDim / (vec ? 4 : 1);
    if (vec)
        hipLaunchKernelGGL(qkv_split_kernel<true>, dim3(gridFor(items)), dim3(256), 0, stream(), pQkv, pQ, pK, pV,
                           tokens, nSeqLen, nHeads, nHeadDim, fScale);
    else
        hipLaunchKernelGGL(qkv_split_kernel<false>, dim3(gridFor(items)), dim3(256), 0, stream(), pQkv, pQ, pK, pV,
                           tokens, nSeqLen, nHeads, nHeadDim, fScale);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipMergeHeads(const float* pIn, float* pOut, int nBatch, int nSeqLen, int nHeads, int nHeadDim) {
    const char* name = "omHipMergeHeads";
    clearError();
    if (nBatch <= 0 || nSeqLen <= 0 || nHeads <= 0 || nHeadDim <= 0) return 0;
    if (!pIn || !pOut) return fail("%s: null pointer", name);
    if (checkHeads(name, nBatch, nSeqLen, nHeads, nHeadDim)) return -1;
    const int tokens = nBatch * nSeqLen;
    const bool vec = nHeadDim % 4 == 0 && al16(pIn) && al16(pOut);
    const long long items = (long long)tokens * nHeads * nHeadDim / (vec ? 4 : 1);
    if (vec)
        hipLaunchKernelGGL(merge_heads_kernel<true>, dim3(gridFor(items)), dim3(256), 0, stream(), pIn, pOut, tokens,
                           nSeqLen, nHeads, nHeadDim);
    else
        hipLaunchKernelGGL(merge_heads_kernel<false>, dim3(gridFor(items)), dim3(256), 0, stream(), pIn, pOut, tokens,
                           nSeqLen, nHeads, nHeadDim);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipSum(const float* pData, float* pResult, int nCount) {
    clearError();
    return sumTo("omHipSum", pData, pResult, nCount, 1.0f);
}

int omHipMean(const float* pData, float* pResult, int nCount) {
    clearError();
    // omCudaMean: the sum, then multiplied by 1 / count (cuda_kernels.cu:1506-1513)
    return sumTo("omHipMean", pData, pResult, nCount, nCount > 0 ? 1.0f / (float)nCount : 0.0f);
}

int omHipAttention(const float* pQKV, float* pOut, int nBatch, int nSeq, int nHeads, int nHeadDim, float fScale) {
    const char* name = "omHipAttention";
    clearError();
    if (nBatch <= 0 || nSeq <= 0 || nHeads <= 0 || nHeadDim <= 0) return 0;
    if (!pQKV || !pOut) return fail("%s: null pointer", name);
    if (checkHeads(name, nBatch, nSeq, nHeads, nHeadDim)) return -1;
    const long long S = nSeq, Dh = nHeadDim, D = (long long)nHeads * nHeadDim, T = (long long)nBatch * nSeq;
    // The outer loop runs over whichever of images / heads is fewer; each step
    // batches the other through one strided GEMM that reads K and V where they
    // lie in the projection and writes the context in the merged layout.
    const bool headsOuter = nHeads <= nBatch;
    const int outer = headsOuter ? nHeads : nBatch, inner = headsOuter ? nBatch : nHeads;
    if ((long long)inner * S * S > 0x7fffffffLL)
        return fail("%s: %d x %lld x %lld scores exceed the 2^31-element limit", name, inner, S, S);
    const size_t bQ = up((size_t)(T * D) * 4), bScores = up((size_t)inner * S * S * 4);
    char* base = static_cast<char*>(workspace(bQ + bScores, kWsStaging));
    if (!base) return -1;   // workspace() recorded the cause
    float* q = reinterpret_cast<float*>(base);
    float* scores = reinterpret_cast<float*>(base + bQ);
    const long long ldq = 3 * D;
    // Q * scale, as qkvSplitHeads scales it (one fp32 multiply), kept token-major [T, D]
    hipLaunchKernelGGL(scale_copy_kernel, dim3(gridFor(T * D)), dim3(256), 0, stream(), pQKV, q, (int)T, (int)ldq,
                       (int)D, fScale);
    OMHIP_CHECK_LAUNCH();
    const long long innerQ = headsOuter ? S * D : Dh;     // scaled Q: step between inner entries
    const long long innerKV = headsOuter ? S * ldq : Dh;  // K, V in the projection
    const long long innerC = headsOuter ? S * D : Dh;     // merged context
    for (int o = 0; o < outer; ++o) {
        const float* Q = q + (headsOuter ? o * Dh : o * S * D);
        const float* K = pQKV + (headsOuter ? o * Dh : o * S * ldq) + D;
        const float* V = K + D;
        float* C = pOut + (headsOuter ? o * Dh : o * S * D);
        if (omHipGemmStridedBatched(0, 1, inner, nSeq, nSeq, nHeadDim, Q, D, innerQ, K, ldq, innerKV, scores, S,
                                    S * S))
            return -1;
        if (omHipSoftmax(scores, scores, inner * nSeq, nSeq)) return -1;
        if (omHipGemmStridedBatched(0, 0, inner, nSeq, nHeadDim, nSeq, scores, S, S * S, V, ldq, innerKV, C, D,
                                    innerC))
            return -1;
    }
    return 0;
}

}  // extern "C"
