// conv.hip — NCHW conv2d as an implicit GEMM on fp32 MFMA, with the
// bias + BatchNorm(inference) + ReLU epilogue fused into the output write.
//
//   Out[co][q] = sum_kk W[co][kk] * X^[kk][q]
//   kk = (ci*KH + kh)*KW + kw    (the reference im2col row order, cpu_backend.ixx:554-557)
//   q  = (n*Ho + oh)*Wo + ow     (output pixel, batch folded into the GEMM N axis)
//   X^[kk][q] = x[n][ci][oh*s-p+kh][ow*s-p+kw], zero outside the image
//
// The reference lowers conv2d per image to im2col + matmul + bias
// (cpu_backend.ixx:619-658) and applies batchNorm2d / relu as separate passes
// (tensor_ops.ixx:672-833, :511-536). Here the im2col operand is never
// materialised: each thread gathers its pixels' taps straight into the LDS
// B slice, and the output passes through HBM once, already normalised.
//
// Split-K (for late layers whose Cout x pixels tile count cannot fill 256 CUs)
// writes fp32 partial tiles to a workspace and a second kernel sums the splits
// in a fixed order (deterministic) and applies the same epilogue.
#include "omhip_internal.hpp"
#include "mfma_f32_tile.hpp"
#include "gemm_f32.hpp"
#include "../../include/omhip.h"

#include <algorithm>

namespace omhip {

int im2colBatched(const float* x, float* col, int N, int Cin, int H, int W, int KH, int KW, int pad, int strd,
                  int Ho, int Wo);

struct ConvParams {
    const float* x;      // [N][Cin][H][W]
    const float* w;      // [Cout][Cin*KH*KW]
    const float* bias;   // [Cout] or null
    const float* gamma;  // BN (all four null = no BN)
    const float* beta;
    const float* mean;
    const float* var;
    float eps;
    int act;             // 0 identity, 1 relu
    float* out;          // [N][Cout][Ho][Wo]
    float* ws;           // split-K partials [splits][Cout][Nq]
    int N, Cin, H, W, Cout, KH, KW, stride, pad, Ho, Wo;
    int K;               // Cin*KH*KW
    int Nq;              // N*Ho*Wo
    int tilesM, tilesN;
    int splits, kChunk;  // split-K: k range [s*kChunk, min(K,(s+1)*kChunk))
};

// Implicit im2col loader. Thread t owns pixel column c = t % BN of the slice
// and rows g, g+TPC, g+2*TPC, ... (g = t / BN, TPC = NT/BN threads per column),
// so its tap sequence over the whole K walk advances by TPC every row and the
// (ci, kh, kw) decomposition is carried incrementally instead of divided out.
template <int BN, int BK, int NT>
struct ImplicitLoader {
    static constexpr int TPC = NT / BN;
    static constexpr int RPT = BK / TPC;   // rows per thread per slice
    static_assert(NT % BN == 0 && BK % TPC == 0, "implicit loader mapping");
    using Shape = LdsShape<false, BN, BK>;

    const float* xn;     // base of the pixel's image
    int ih0, iw0;        // top-left input coordinate of the pixel's window
    int pixoff;          // ih0*W + iw0 (negative at the top/left border; only used when the tap is inside)
    bool colValid;
    int H, W, HW, KH, KW, K;
    int kk, ci, kh, kw;  // current tap of this thread
    int koff;            // ci*HW + kh*W + kw
    float v[RPT];

    __device__ void init(const ConvParams& p, int q, int kStart, int tid) {
        H = p.H; W = p.W; HW = p.H * p.W; KH = p.KH; KW = p.KW; K = p.K;
        colValid = q < p.Nq;
        const int qq = colValid ? q : 0;
        const int HoWo = p.Ho * p.Wo;
        const int n = qq / HoWo;
        const int pix = qq - n * HoWo;
        const int oh = pix / p.Wo, ow = pix - (pix / p.Wo) * p.Wo;
        ih0 = oh * p.stride - p.pad;
        iw0 = ow * p.stride - p.pad;
        xn = p.x + (long long)n * p.Cin * HW;
        pixoff = ih0 * W + iw0;
        const int g = tid / BN;
        kk = kStart + g;
        const int khw = KH * KW;
        ci = kk / khw;
        const int rem = kk - ci * khw;
        kh = rem / KW;
        kw = rem - kh * KW;
        koff = ci * HW + kh * W + kw;
    }

    __device__ __forceinline__ void step() {
        kk += TPC;
#pragma unroll
        for (int s = 0; s < TPC; ++s) {
            ++kw; ++koff;
            if (kw == KW) {
                kw = 0; koff += W - KW; ++kh;
                if (kh == KH) { kh = 0; koff += HW - KH * W; ++ci; }
            }
        }
    }

    // Loads the next RPT taps (the slice's rows for this thread); kEnd bounds the split.
    __device__ void load(int kEnd) {
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int ih = ih0 + kh, iw = iw0 + kw;
            float val = 0.f;
            if (colValid && kk < kEnd && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                val = xn[koff + pixoff];
            v[j] = val;
            step();
        }
    }

    __device__ void store(float* s, int tid) const {
        const int c = tid % BN, g = tid / BN;
#pragma unroll
        for (int j = 0; j < RPT; ++j) s[(g + j * TPC) * Shape::LD + c] = v[j];
    }
};

template <class Cfg, bool VA>
__global__ __launch_bounds__(Cfg::NT) void conv_igemm_kernel(ConvParams p) {
    extern __shared__ float smem[];
    using SA = LdsShape<true, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<false, Cfg::BN, Cfg::BK>;
    constexpr int STAGE = SA::SIZE + SB::SIZE;
    float* sEpi = smem + 2 * STAGE;   // [5][BM]: bias, mean, invStd, gamma, beta

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N;
    const int wn = wave % Cfg::WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, p.tilesM * p.tilesN, p.tilesM, p.tilesN, 4, tm, tn);
    const int m0 = tm * Cfg::BM;
    const int n0 = tn * Cfg::BN;
    const int split = blockIdx.y;
    const int kBeg = split * p.kChunk;
    const int kEnd = min(p.K, kBeg + p.kChunk);

    DenseLoader<true, VA, Cfg::BM, Cfg::BK, Cfg::NT> la;
    la.p = p.w; la.ld = p.K; la.rows = p.Cout; la.K = kEnd; la.r0 = m0;
    ImplicitLoader<Cfg::BN, Cfg::BK, Cfg::NT> lb;
    lb.init(p, n0 + tid % Cfg::BN, kBeg, tid);

    const bool direct = p.splits == 1;
    if (direct && tid < Cfg::BM) {
        const int co = min(m0 + tid, p.Cout - 1);
        sEpi[tid] = p.bias ? p.bias[co] : 0.f;
        if (p.gamma) {
            sEpi[Cfg::BM + tid] = p.mean[co];
            sEpi[2 * Cfg::BM + tid] = 1.0f / sqrtf(p.var[co] + p.eps);
            sEpi[3 * Cfg::BM + tid] = p.gamma[co];
            sEpi[4 * Cfg::BM + tid] = p.beta[co];
        }
    }

    f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = (kEnd - kBeg + Cfg::BK - 1) / Cfg::BK;
    la.load(kBeg, tid);
    lb.load(kEnd);
    la.store(smem, tid);
    lb.store(smem + SA::SIZE, tid);
    __syncthreads();
    for (int t = 0; t < nk; ++t) {
        const int cur = t & 1;
        const bool more = (t + 1) < nk;
        if (more) {
            la.load(kBeg + (t + 1) * Cfg::BK, tid);
            lb.load(kEnd);
        }
        float* sCur = smem + cur * STAGE;
        float* sNxt = smem + (cur ^ 1) * STAGE;
        mma_slice<Cfg, true, false>(sCur, sCur + SA::SIZE, acc, wm, wn, lane);
        if (more) {
            la.store(sNxt, tid);
            lb.store(sNxt + SA::SIZE, tid);
        }
        __syncthreads();
    }

    const int li = lane & 31, h = lane >> 5;
    const int HoWo = p.Ho * p.Wo;
    if (!direct) {
        float* ws = p.ws + (long long)split * p.Cout * p.Nq;
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int q = n0 + wn * Cfg::WN + fn * 32 + li;
            if (q >= p.Nq) continue;
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int co = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (co < p.Cout) ws[(long long)co * p.Nq + q] = acc[fm][fn][r];
                }
        }
        return;
    }
#pragma unroll
    for (int fn = 0; fn < Cfg::FN; ++fn) {
        const int q = n0 + wn * Cfg::WN + fn * 32 + li;
        if (q >= p.Nq) continue;
        const int n = q / HoWo;
        const int pix = q - n * HoWo;
        float* o = p.out + (long long)n * p.Cout * HoWo + pix;
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rl = wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const int co = m0 + rl;
                if (co >= p.Cout) continue;
                float v = acc[fm][fn][r] + sEpi[rl];
                if (p.gamma)
                    v = __builtin_fmaf(sEpi[3 * Cfg::BM + rl], (v - sEpi[Cfg::BM + rl]) * sEpi[2 * Cfg::BM + rl],
                                       sEpi[4 * Cfg::BM + rl]);
                if (p.act == 1) v = v > 0.f ? v : 0.f;
                o[(long long)co * HoWo] = v;
            }
    }
}

// Sums split-K partials in split order and applies the epilogue; one thread
// per (co, q) with q fastest so reads and NCHW writes are both coalesced.
__global__ void conv_splitk_finish(ConvParams p) {
    const long long total = (long long)p.Cout * p.Nq;
    const int HoWo = p.Ho * p.Wo;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int co = (int)(i / p.Nq);
        const int q = (int)(i - (long long)co * p.Nq);
        float v = 0.f;
        for (int s = 0; s < p.splits; ++s) v += p.ws[(long long)s * total + i];
        if (p.bias) v += p.bias[co];
        if (p.gamma) {
            const float inv = 1.0f / sqrtf(p.var[co] + p.eps);
            v = __builtin_fmaf(p.gamma[co], (v - p.mean[co]) * inv, p.beta[co]);
        }
        if (p.act == 1) v = v > 0.f ? v : 0.f;
        const int n = q / HoWo;
        const int pix = q - n * HoWo;
        p.out[((long long)n * p.Cout + co) * HoWo + pix] = v;
    }
}

// ---- tile configurations -----------------------------------------------------
using ConvCfg64 = TileCfg<64, 256, 16, 64, 64>;     // Cout <= 64: 4 waves along pixels
using ConvCfg128 = TileCfg<128, 256, 16, 64, 128>;  // 2 x 2 waves

template <class Cfg>
static size_t convLds() {
    return (2 * (LdsShape<true, Cfg::BM, Cfg::BK>::SIZE + LdsShape<false, Cfg::BN, Cfg::BK>::SIZE) + 5 * Cfg::BM) *
           sizeof(float);
}

template <class Cfg, bool VA>
static int launchConvT(ConvParams& p) {
    auto kern = conv_igemm_kernel<Cfg, VA>;
    const size_t lds = convLds<Cfg>();
    static bool s_attr = false;
    if (!s_attr) {
        OMHIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        s_attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(p.tilesM * p.tilesN, p.splits), dim3(Cfg::NT), lds, stream(), p);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <class Cfg>
static int launchConvCfg(ConvParams& p, float* wsBuf) {
    p.tilesM = (p.Cout + Cfg::BM - 1) / Cfg::BM;
    p.tilesN = (p.Nq + Cfg::BN - 1) / Cfg::BN;
    const long long tiles = (long long)p.tilesM * p.tilesN;
    const long long cus = cuCount();
    // Split K while the grid is below one wave of CUs and each split keeps >= 256 taps.
    int splits = 1;
    while (wsBuf && tiles * splits * 2 <= cus * 2 && p.K / (splits * 2) >= 256 && splits < 16) splits *= 2;
    p.splits = splits;
    p.kChunk = (p.K + splits - 1) / splits;
    p.kChunk = (p.kChunk + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
    p.splits = (p.K + p.kChunk - 1) / p.kChunk;
    p.ws = wsBuf;
    const bool va = (p.K % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.w) & 15u) == 0);
    int rc = va ? launchConvT<Cfg, true>(p) : launchConvT<Cfg, false>(p);
    if (rc || p.splits == 1) return rc;
    const long long total = (long long)p.Cout * p.Nq;
    const int blocks = (int)std::min<long long>((total + 255) / 256, (long long)cus * 16);
    hipLaunchKernelGGL(conv_splitk_finish, dim3(blocks), dim3(256), 0, stream(), p);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

static int validateConv(const char* name, const float* x, const float* w, float* out, int N, int Cin, int H, int W,
                        int Cout, int KH, int KW, int stride, int pad, int& Ho, int& Wo) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0)
        return fail("%s: invalid geometry", name);
    if (!x || !w || !out) return fail("%s: null pointer", name);
    Ho = (H + 2 * pad - KH) / stride + 1;
    Wo = (W + 2 * pad - KW) / stride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("%s: kernel larger than the padded input", name);
    const long long K = (long long)Cin * KH * KW;
    const long long Nq = (long long)N * Ho * Wo;
    if (K > (1LL << 30) || Nq > (1LL << 30) || (long long)N * Cin * H * W > (1LL << 31) - 1 ||
        (long long)N * Cout * Ho * Wo > (1LL << 31) - 1 || (long long)Cin * H * W > (1LL << 30))
        return fail("%s: tensor exceeds the 32-bit index range of this kernel", name);
    return 0;
}

int conv2dFused(const char* name, const float* x, const float* w, const float* bias, const float* gamma,
                const float* beta, const float* mean, const float* var, float eps, int act, float* out, int N, int Cin,
                int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    clearError();
    int Ho, Wo;
    if (validateConv(name, x, w, out, N, Cin, H, W, Cout, KH, KW, stride, pad, Ho, Wo)) return -1;
    const bool anyBn = gamma || beta || mean || var;
    if (anyBn && !(gamma && beta && mean && var)) return fail("%s: BN needs gamma, beta, mean and var", name);
    if (act != 0 && act != 1) return fail("%s: unknown activation %d", name, act);
    ConvParams p{};
    p.x = x; p.w = w; p.bias = bias;
    p.gamma = anyBn ? gamma : nullptr; p.beta = beta; p.mean = mean; p.var = var;
    p.eps = eps; p.act = act; p.out = out;
    p.N = N; p.Cin = Cin; p.H = H; p.W = W; p.Cout = Cout; p.KH = KH; p.KW = KW;
    p.stride = stride; p.pad = pad; p.Ho = Ho; p.Wo = Wo;
    p.K = Cin * KH * KW;
    p.Nq = N * Ho * Wo;
    // Workspace large enough for up to 16 splits of the output.
    const size_t wsBytes = (size_t)16 * Cout * p.Nq * sizeof(float);
    float* ws = (wsBytes <= ((size_t)1 << 30)) ? static_cast<float*>(workspace(wsBytes)) : nullptr;
    if (Cout <= 64) return launchConvCfg<ConvCfg64>(p, ws);
    return launchConvCfg<ConvCfg128>(p, ws);
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipConv2d(const float* pInput, const float* pWeight, const float* pBias, float* pOutput, int nBatch, int nCin,
                int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    return conv2dFused("omHipConv2d", pInput, pWeight, pBias, nullptr, nullptr, nullptr, nullptr, 0.f, 0, pOutput,
                       nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad);
}

int omHipConv2dBiasBnAct(const float* pInput, const float* pWeight, const float* pBias, const float* pGamma,
                         const float* pBeta, const float* pMean, const float* pVar, float fEps, int nAct,
                         float* pOutput, int nBatch, int nCin, int nH, int nW, int nCout, int nKH, int nKW,
                         int nStride, int nPad) {
    return conv2dFused("omHipConv2dBiasBnAct", pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, nAct,
                       pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad);
}

// Explicit lowering: im2col of every image into one buffer, then a batched
// GEMM with the weight shared across the batch (A stride 0), then bias.
int omHipConv2dIm2col(const float* pInput, const float* pWeight, const float* pBias, float* pOutput, int nBatch,
                      int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    clearError();
    int Ho, Wo;
    if (validateConv("omHipConv2dIm2col", pInput, pWeight, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride,
                     nPad, Ho, Wo))
        return -1;
    const long long K = (long long)nCin * nKH * nKW;
    const long long HWo = (long long)Ho * Wo;
    void* col = nullptr;
    if (omHipMalloc(&col, (size_t)(nBatch * K * HWo) * sizeof(float))) return -1;
    int rc = im2colBatched(pInput, static_cast<float*>(col), nBatch, nCin, nH, nW, nKH, nKW, nPad, nStride, Ho, Wo);
    if (!rc)
        rc = gemmF32(false, false, nBatch, nCout, (int)HWo, (int)K, pWeight, K, 0, static_cast<const float*>(col), HWo,
                     K * HWo, pOutput, HWo, (long long)nCout * HWo);
    if (!rc && pBias) rc = omHipAddBias(pOutput, pBias, pOutput, nBatch, nCout, (int)HWo);
    (void)omHipFree(col);
    return rc;
}

}  // extern "C"
