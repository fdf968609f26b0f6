// eltwise.hip — memory-bound HAL ops: fills, copy, ReLU (+backward), bias
// broadcast, transpose, BatchNorm inference, im2col, fp16/bf16 conversion.
//
// All are HBM-bound streams: each thread handles 4 consecutive floats with
// 128-bit loads/stores where the pointers allow, grid-stride over the array.
#include "omhip_internal.hpp"
#include "conv.hpp"
#include "../../include/omhip.h"

#include <algorithm>

namespace omhip {

typedef float f4 __attribute__((ext_vector_type(4)));

static inline int gridFor(long long nWork, int block = 256) {
    const long long cap = (long long)cuCount() * 16;
    return (int)std::max<long long>(1, std::min<long long>((nWork + block - 1) / block, cap));
}
static inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ReLU as the reference writes it: x > 0 ? x : 0 (NaN -> 0, -0 -> +0),
// cpu_backend.ixx:327 / simd.ixx:259 (max_ps(x, 0) returns the second operand
// for NaN and for a signed-zero tie).
__device__ __forceinline__ float relu1(float x) { return x > 0.f ? x : 0.f; }

// ---- fill / copy -----------------------------------------------------------
__global__ void fill_kernel(float* p, long long n, float v) {
    const long long n4 = n / 4;
    const long long stride = (long long)gridDim.x * blockDim.x;
    const f4 vv = {v, v, v, v};
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4; i += stride)
        reinterpret_cast<f4*>(p)[i] = vv;
    for (long long i = n4 * 4 + blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}
__global__ void fill_kernel_s(float* p, long long n, float v) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

int fillValue(float* p, long long n, float v) {
    if (n <= 0) return 0;
    if (!p) return fail("fill: null pointer");
    if (al16(p)) hipLaunchKernelGGL(fill_kernel, dim3(gridFor(n / 4 + 1)), dim3(256), 0, stream(), p, n, v);
    else hipLaunchKernelGGL(fill_kernel_s, dim3(gridFor(n)), dim3(256), 0, stream(), p, n, v);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// Byte fill (omHipMemset): 16-byte stores over the aligned body, bytes at the ends.
__global__ void byte_fill_kernel(unsigned char* p, long long n, unsigned int word) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    const long long head = (long long)((16 - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u);
    const long long h = head < n ? head : n;
    const long long body = (n - h) / 16;
    const uint4 w = {word, word, word, word};
    uint4* q = reinterpret_cast<uint4*>(p + h);
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < body; i += stride) q[i] = w;
    const unsigned char b = (unsigned char)(word & 0xffu);
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < h; i += stride) p[i] = b;
    for (long long i = h + body * 16 + blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) p[i] = b;
}

int byteFill(void* p, unsigned char value, size_t nBytes) {
    if (nBytes == 0) return 0;
    const unsigned int word = 0x01010101u * value;
    hipLaunchKernelGGL(byte_fill_kernel, dim3(gridFor((long long)(nBytes / 16) + 1)), dim3(256), 0, stream(),
                       static_cast<unsigned char*>(p), (long long)nBytes, word);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// ---- ReLU ------------------------------------------------------------------
__global__ void relu_kernel4(const float* __restrict__ in, float* __restrict__ out, long long n) {
    const long long n4 = n / 4;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4; i += stride) {
        f4 v = reinterpret_cast<const f4*>(in)[i];
        v[0] = relu1(v[0]); v[1] = relu1(v[1]); v[2] = relu1(v[2]); v[3] = relu1(v[3]);
        reinterpret_cast<f4*>(out)[i] = v;
    }
    for (long long i = n4 * 4 + blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = relu1(in[i]);
}
__global__ void relu_kernel1(const float* in, float* out, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) out[i] = relu1(in[i]);
}
__global__ void relu_bwd_kernel(const float* x, const float* g, float* gi, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        gi[i] = x[i] > 0.f ? g[i] : 0.f;
}

// out = a + (x > 0 ? g : 0): the reference's add(a, reluBackward(x, g)) in one pass.
__global__ void add_relu_bwd_kernel(const float* a, const float* x, const float* g, float* o, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        o[i] = a[i] + (x[i] > 0.f ? g[i] : 0.f);
}

// ---- bias broadcast: out[n,c,hw] = data[n,c,hw] + bias[c] -------------------
__global__ void add_bias_kernel(const float* __restrict__ d, const float* __restrict__ b, float* __restrict__ o,
                                long long total, int C, int HW) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int c = (int)((i / HW) % C);
        o[i] = d[i] + b[c];
    }
}

// ---- transpose: out[c, r] = in[r, c] through a padded LDS tile -------------
__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int rows, int cols) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
    for (int j = ty; j < 32; j += 8) {
        const int r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) tile[j][tx] = in[(long long)r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const int c = c0 + j, r = r0 + tx;
        if (r < rows && c < cols) out[(long long)c * rows + r] = tile[tx][j];
    }
}

// ---- BatchNorm inference -----------------------------------------------------
// y = gamma*((x-mean)*invStd)+beta with invStd = 1/sqrt(var+eps) in fp32,
// the exact expression of cpu_backend.ixx:832-838; the multiply-add is fused
// (the reference as compiled with clang contracts it to an fma).
__global__ void bn_stats_kernel(const float* mean, const float* var, float* savedMean, float* savedInvStd,
                                int C, float eps) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    if (savedMean) savedMean[c] = mean[c];
    if (savedInvStd) savedInvStd[c] = 1.0f / sqrtf(var[c] + eps);
}
__global__ void bn_eval_kernel(const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
                               const float* __restrict__ beta, const float* __restrict__ mean,
                               const float* __restrict__ var, int C, int HW, float eps, int plane0) {
    const int plane = plane0 + blockIdx.y;  // n*C + c
    const int c = plane % C;
    const float mu = mean[c];
    const float inv = 1.0f / sqrtf(var[c] + eps);
    const float g = gamma[c], b = beta[c];
    const long long base = (long long)plane * HW;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < HW; i += gridDim.x * blockDim.x)
        y[base + i] = __builtin_fmaf(g, (x[base + i] - mu) * inv, b);
}

// ---- im2col of one image: col[(c*KH+kh)*KW+kw][oh*Wo+ow] -------------------
__global__ void im2col_kernel(const float* __restrict__ x, float* __restrict__ col, int Cin, int H, int W,
                              int KH, int KW, int ph, int pw, int sh, int sw, int Ho, int Wo) {
    const long long HWo = (long long)Ho * Wo;
    const long long total = (long long)Cin * KH * KW * HWo;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const long long row = i / HWo;
        const int q = (int)(i - row * HWo);
        const int kw = (int)(row % KW);
        const int kh = (int)((row / KW) % KH);
        const int c = (int)(row / (KW * KH));
        const int oh = q / Wo, ow = q - (q / Wo) * Wo;
        const int ih = oh * sh - ph + kh, iw = ow * sw - pw + kw;
        float v = 0.f;
        if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) v = x[((long long)c * H + ih) * W + iw];
        col[i] = v;
    }
}

// batched im2col: col[n][(c*KH+kh)*KW+kw][q] for every image n
__global__ void im2col_batched_kernel(const float* __restrict__ x, float* __restrict__ col, int N, int Cin, int H,
                                      int W, int KH, int KW, int pad, int strd, int Ho, int Wo) {
    const long long HWo = (long long)Ho * Wo;
    const long long per = (long long)Cin * KH * KW * HWo;
    const long long total = per * N;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const long long n = i / per;
        const long long j = i - n * per;
        const long long row = j / HWo;
        const int q = (int)(j - row * HWo);
        const int kw = (int)(row % KW);
        const int kh = (int)((row / KW) % KH);
        const int c = (int)(row / (KW * KH));
        const int oh = q / Wo, ow = q - (q / Wo) * Wo;
        const int ih = oh * strd - pad + kh, iw = ow * strd - pad + kw;
        float v = 0.f;
        if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
            v = x[(((long long)n * Cin + c) * H + ih) * W + iw];
        col[i] = v;
    }
}

int im2colBatched(const float* x, float* col, int N, int Cin, int H, int W, int KH, int KW, int pad, int strd,
                  int Ho, int Wo) {
    const long long total = (long long)N * Cin * KH * KW * Ho * Wo;
    hipLaunchKernelGGL(im2col_batched_kernel, dim3(gridFor(total)), dim3(256), 0, stream(), x, col, N, Cin, H, W,
                       KH, KW, pad, strd, Ho, Wo);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// ---- fp32 <-> fp16 / bf16 ----------------------------------------------------
// fp16: hardware v_cvt_f16_f32 (IEEE round-to-nearest-even, subnormals kept).
// bf16: round-to-nearest-even on the bit pattern (add 0x7FFF plus the lsb of
// the kept half), NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(r >> 16);
}
__global__ void cvt_f32_f16_kernel(const float* in, uint16_t* out, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride) {
        const _Float16 h = (_Float16)in[i];
        out[i] = __builtin_bit_cast(uint16_t, h);
    }
}
__global__ void cvt_f32_bf16_kernel(const float* in, uint16_t* out, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = f32_to_bf16_rne(in[i]);
}
__global__ void cvt_f16_f32_kernel(const uint16_t* in, float* out, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (float)__builtin_bit_cast(_Float16, in[i]);
}
__global__ void cvt_bf16_f32_kernel(const uint16_t* in, float* out, long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = __builtin_bit_cast(float, (uint32_t)in[i] << 16);
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipFillZeros(float* pData, int nCount) { clearError(); return fillValue(pData, nCount, 0.f); }
int omHipFillOnes(float* pData, int nCount) { clearError(); return fillValue(pData, nCount, 1.f); }
int omHipFillValue(float* pData, int nCount, float fValue) { clearError(); return fillValue(pData, nCount, fValue); }

int omHipCopy(const float* pSrc, float* pDst, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pSrc || !pDst) return fail("omHipCopy: null pointer");
    OMHIP_CHECK(hipMemcpyAsync(pDst, pSrc, (size_t)nCount * sizeof(float), hipMemcpyDeviceToDevice, stream()));
    return 0;
}

int omHipReLU(const float* pIn, float* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipReLU: null pointer");
    if (al16(pIn) && al16(pOut))
        hipLaunchKernelGGL(relu_kernel4, dim3(gridFor(nCount / 4 + 1)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    else
        hipLaunchKernelGGL(relu_kernel1, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipReLUBackward(const float* pIn, const float* pGradOut, float* pGradIn, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pGradOut || !pGradIn) return fail("omHipReLUBackward: null pointer");
    hipLaunchKernelGGL(relu_bwd_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pGradOut, pGradIn,
                       (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAddReluBackward(const float* pA, const float* pIn, const float* pGradOut, float* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pA || !pIn || !pGradOut || !pOut) return fail("omHipAddReluBackward: null pointer");
    hipLaunchKernelGGL(add_relu_bwd_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pA, pIn, pGradOut, pOut,
                       (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAddBias(const float* pData, const float* pBias, float* pOut, int nN, int nC, int nHW) {
    clearError();
    if (nN <= 0 || nC <= 0 || nHW <= 0) return 0;
    if (!pData || !pBias || !pOut) return fail("omHipAddBias: null pointer");
    const long long total = (long long)nN * nC * nHW;
    hipLaunchKernelGGL(add_bias_kernel, dim3(gridFor(total)), dim3(256), 0, stream(), pData, pBias, pOut, total, nC,
                       nHW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipTranspose(const float* pIn, float* pOut, int nRows, int nCols) {
    clearError();
    if (nRows <= 0 || nCols <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipTranspose: null pointer");
    if ((nRows + 31) / 32 > 65535) return fail("omHipTranspose: %d rows exceed the grid limit", nRows);
    dim3 grid((nCols + 31) / 32, (nRows + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, stream(), pIn, pOut, nRows, nCols);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipBatchNorm2d(const float* pInput, float* pOutput, const float* pGamma, const float* pBeta,
                     float* pRunMean, float* pRunVar, float* pSavedMean, float* pSavedInvStd,
                     int nBatch, int nChannels, int nH, int nW, float fEps, float fMomentum, int bTraining) {
    clearError();
    if (nBatch <= 0 || nChannels <= 0 || nH <= 0 || nW <= 0) return 0;
    if (!pInput || !pOutput || !pGamma || !pBeta || !pRunMean || !pRunVar)
        return fail("omHipBatchNorm2d: null pointer");
    if (bTraining)
        return batchNorm2dTrain(pInput, pOutput, pGamma, pBeta, pRunMean, pRunVar, pSavedMean, pSavedInvStd, nBatch,
                                nChannels, nH, nW, fEps, fMomentum);
    if (pSavedMean || pSavedInvStd) {
        hipLaunchKernelGGL(bn_stats_kernel, dim3((nChannels + 255) / 256), dim3(256), 0, stream(), pRunMean, pRunVar,
                           pSavedMean, pSavedInvStd, nChannels, fEps);
        OMHIP_CHECK_LAUNCH();
    }
    const int HW = nH * nW;
    const int planes = nBatch * nChannels;
    const int bx = std::max(1, std::min((HW + 255) / 256, std::max(1, 4096 / std::max(1, planes))));
    for (int p0 = 0; p0 < planes; p0 += 65535) {   // grid.y is limited to 65535 planes per launch
        const int cnt = std::min(65535, planes - p0);
        hipLaunchKernelGGL(bn_eval_kernel, dim3(bx, cnt), dim3(256), 0, stream(), pInput, pOutput, pGamma, pBeta,
                           pRunMean, pRunVar, nChannels, HW, fEps, p0);
        OMHIP_CHECK_LAUNCH();
    }
    return 0;
}

int omHipIm2col(const float* pInput, int nCin, int nH, int nW, int nKH, int nKW, int nPadH, int nPadW,
                int nStrideH, int nStrideW, float* pCol) {
    clearError();
    if (nCin <= 0 || nH <= 0 || nW <= 0 || nKH <= 0 || nKW <= 0 || nStrideH <= 0 || nStrideW <= 0 || nPadH < 0 ||
        nPadW < 0)
        return fail("omHipIm2col: invalid geometry");
    if (!pInput || !pCol) return fail("omHipIm2col: null pointer");
    const int Ho = (nH + 2 * nPadH - nKH) / nStrideH + 1;
    const int Wo = (nW + 2 * nPadW - nKW) / nStrideW + 1;
    if (Ho <= 0 || Wo <= 0) return 0;
    const long long total = (long long)nCin * nKH * nKW * Ho * Wo;
    hipLaunchKernelGGL(im2col_kernel, dim3(gridFor(total)), dim3(256), 0, stream(), pInput, pCol, nCin, nH, nW, nKH,
                       nKW, nPadH, nPadW, nStrideH, nStrideW, Ho, Wo);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipConvertF32ToF16(const float* pIn, uint16_t* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipConvertF32ToF16: null pointer");
    hipLaunchKernelGGL(cvt_f32_f16_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}
int omHipConvertF32ToBF16(const float* pIn, uint16_t* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipConvertF32ToBF16: null pointer");
    hipLaunchKernelGGL(cvt_f32_bf16_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}
int omHipConvertF16ToF32(const uint16_t* pIn, float* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipConvertF16ToF32: null pointer");
    hipLaunchKernelGGL(cvt_f16_f32_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}
int omHipConvertBF16ToF32(const uint16_t* pIn, float* pOut, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pIn || !pOut) return fail("omHipConvertBF16ToF32: null pointer");
    hipLaunchKernelGGL(cvt_bf16_f32_kernel, dim3(gridFor(nCount)), dim3(256), 0, stream(), pIn, pOut, (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // extern "C"
