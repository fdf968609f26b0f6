// gemm_f32.hip — fp32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Entry points: omHipMatmul / MatmulTransB / MatmulTransA / BatchedMatmul /
// BatchedMatmulTransB / GemmStridedBatched. They replace the reference's
// omCudaMatmul (src/cuda/cuda_kernels.cu:768-804) and omCudaBatchedMatmul
// (:843-878) and compute what CPUBackend::matmul / batchedMatmul compute
// (src/hal/om.hal.cpu_backend.ixx:239-286, :1520-1532); the transposed
// variants replace the reference's explicit transpose2d + matmul compositions
// (src/engine/om.engine.autograd.ixx:261-286).
#include "omhip_internal.hpp"
#include "mfma_f32_tile.hpp"
#include "gemm_f32.hpp"
#include "../../include/omhip.h"

#include <algorithm>

namespace omhip {

template <class Cfg, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void gemm_f32_kernel(GemmF32Params p) {
    extern __shared__ float smem[];
    constexpr bool A_KMAJOR = !TA;
    constexpr bool B_KMAJOR = TB;
    using SA = LdsShape<A_KMAJOR, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<B_KMAJOR, Cfg::BN, Cfg::BK>;
    constexpr int STAGE = SA::SIZE + SB::SIZE;   // floats per LDS buffer (A slice then B slice)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N;
    const int wn = wave % Cfg::WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, p.tilesM * p.tilesN, p.tilesM, p.tilesN, 8, tm, tn);
    const long long batch = blockIdx.z;
    const int split = blockIdx.y;
    const int m0 = tm * Cfg::BM;
    const int n0 = tn * Cfg::BN;
    // This split's K range; the loaders treat kEnd as the end of K.
    const int kBeg = split * p.kChunk;
    const int kEnd = min(p.K, kBeg + p.kChunk);

    DenseLoader<A_KMAJOR, VA, Cfg::BM, Cfg::BK, Cfg::NT> la;
    la.p = p.A + batch * p.sA; la.ld = p.lda; la.rows = p.M; la.K = kEnd; la.r0 = m0;
    DenseLoader<B_KMAJOR, VB, Cfg::BN, Cfg::BK, Cfg::NT> lb;
    lb.p = p.B + batch * p.sB; lb.ld = p.ldb; lb.rows = p.N; lb.K = kEnd; lb.r0 = n0;

    f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = (kEnd - kBeg + Cfg::BK - 1) / Cfg::BK;
    la.load(kBeg, tid);
    lb.load(kBeg, tid);
    la.store(smem, tid);
    lb.store(smem + SA::SIZE, tid);
    __syncthreads();
    for (int t = 0; t < nk; ++t) {
        const int cur = t & 1;
        const bool more = (t + 1) < nk;
        if (more) {
            la.load(kBeg + (t + 1) * Cfg::BK, tid);
            lb.load(kBeg + (t + 1) * Cfg::BK, tid);
        }
        float* sCur = smem + cur * STAGE;
        float* sNxt = smem + (cur ^ 1) * STAGE;
        mma_slice<Cfg, A_KMAJOR, B_KMAJOR>(sCur, sCur + SA::SIZE, acc, wm, wn, lane);
        if (more) {
            la.store(sNxt, tid);
            lb.store(sNxt + SA::SIZE, tid);
        }
        __syncthreads();
    }

    // Split-K / batch-reduce partials go densely to [split][batch][M][N].
    const bool partial = p.ws != nullptr;
    float* C = partial ? p.ws + ((long long)split * gridDim.z + batch) * p.M * p.N : p.C + batch * p.sC;
    const long long ldc = partial ? p.N : p.ldc;
    const int li = lane & 31, h = lane >> 5;
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = n0 + wn * Cfg::WN + fn * 32 + li;
            if (col >= p.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < p.M) C[(long long)row * ldc + col] = acc[fm][fn][r];
            }
        }
    }
}

// Sums the partials of every split in split order and writes C. Thread per element, columns fastest.
__global__ void gemm_splitk_finish(const float* ws, float* C, int splits, int batch, int M, int N, long long ldc,
                                   long long sC) {
    const long long plane = (long long)M * N;
    const long long total = plane * batch;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long b = i / plane, e = i - b * plane;
        const long long r = e / N, c = e - r * N;
        float v = 0.f;
        for (int s = 0; s < splits; ++s) v += ws[((long long)s * batch + b) * plane + e];
        C[b * sC + r * ldc + c] = v;
    }
}

template <class Cfg, bool TA, bool TB>
static size_t ldsBytesFor() {
    using SA = LdsShape<!TA, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<TB, Cfg::BN, Cfg::BK>;
    return 2 * (SA::SIZE + SB::SIZE) * sizeof(float);
}

template <class Cfg, bool TA, bool TB, bool VA, bool VB>
static int launchOne(const GemmF32Params& prm, int batch, int splits) {
    auto kern = gemm_f32_kernel<Cfg, TA, TB, VA, VB>;
    const size_t lds = ldsBytesFor<Cfg, TA, TB>();
    static bool s_attr = false;
    if (!s_attr) {
        OMHIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        s_attr = true;
    }
    dim3 grid(prm.tilesM * prm.tilesN, splits, batch);
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <class Cfg, bool TA, bool TB>
static int launchVec(GemmF32Params prm, int batch, int splits, bool va, bool vb) {
    prm.tilesM = (prm.M + Cfg::BM - 1) / Cfg::BM;
    prm.tilesN = (prm.N + Cfg::BN - 1) / Cfg::BN;
    if (va && vb) return launchOne<Cfg, TA, TB, true, true>(prm, batch, splits);
    if (va) return launchOne<Cfg, TA, TB, true, false>(prm, batch, splits);
    if (vb) return launchOne<Cfg, TA, TB, false, true>(prm, batch, splits);
    return launchOne<Cfg, TA, TB, false, false>(prm, batch, splits);
}

// Slice depth of the large tile is a build-time constant (LDS: 2 x (256x(BK+4) + BKx260) floats).
#ifndef OMHIP_GEMM_BK
#define OMHIP_GEMM_BK 16
#endif
using CfgL = TileCfg<256, 256, OMHIP_GEMM_BK, 128, 128>;
using CfgM = TileCfg<128, 128, 16, 64, 64>;
using CfgS = TileCfg<64, 64, 16, 32, 32>;

struct GemmPlan {
    int cfg;      // 0: 256x256, 1: 128x128, 2: 64x64
    int splits;   // K splits (1: none)
};

// Tile and split-K choice: the largest tile that gives every CU a workgroup.
// When even 64x64 tiles leave CUs idle and K is long (few rows or columns:
// 128 x 4096 x 4096, weight gradients), K is split: the smallest power of two
// (at most 64) that gives every CU a workgroup while each split keeps >= 256
// of K, over the 128x128 tile (64x64 when M or N is below 128). The partials
// cost one fp32 write and read of C per split. Measured on MI355X:
// 128 x 4096 x 4096 runs at 72 TFLOP/s split 8 ways against 34 unsplit;
// K = 512 problems run faster unsplit.
static GemmPlan planGemm(int M, int N, int K, int batch, bool wsOk) {
    const long long cus = cuCount();
    auto tiles = [&](int bm, int bn) { return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
    // TUNE-HOOK-GEMM
    if (tiles(256, 256) >= cus) return {0, 1};
    if (tiles(128, 128) >= cus) return {1, 1};
    if (tiles(64, 64) >= cus || !wsOk || K < 1024) return {2, 1};
    const int cfg = (M >= 128 && N >= 128) ? 1 : 2;
    const long long t = cfg == 1 ? tiles(128, 128) : tiles(64, 64);
    int s = 1;
    while (s < 64 && t * s < cus && K / (2 * s) >= 256) s *= 2;
    return {cfg, s};
}

template <bool TA, bool TB>
static int launchCfg(const GemmF32Params& prm, int batch, int splits, int cfg, bool va, bool vb) {
    if (cfg == 0) return launchVec<CfgL, TA, TB>(prm, batch, splits, va, vb);
    if (cfg == 1) return launchVec<CfgM, TA, TB>(prm, batch, splits, va, vb);
    return launchVec<CfgS, TA, TB>(prm, batch, splits, va, vb);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launches the GEMM (partials to ws when splits > 1) and, if needed, the
// finishing sum.
static int gemmF32Run(bool ta, bool tb, int batch, int M, int N, int K, const float* A, long long lda, long long sA,
                      const float* B, long long ldb, long long sB, float* C, long long ldc, long long sC,
                      GemmPlan plan) {
    GemmF32Params prm{};
    prm.A = A; prm.B = B; prm.C = C;
    prm.M = M; prm.N = N; prm.K = K;
    prm.lda = lda; prm.ldb = ldb; prm.ldc = ldc;
    prm.sA = sA; prm.sB = sB; prm.sC = sC;
    const int bk = 16;
    int splits = plan.splits;
    prm.kChunk = ((K + splits - 1) / splits + bk - 1) / bk * bk;
    splits = (K + prm.kChunk - 1) / prm.kChunk;
    const bool partial = splits > 1;
    if (partial) {
        prm.ws = static_cast<float*>(workspace((size_t)splits * batch * M * N * sizeof(float)));
        if (!prm.ws) return fail("gemm: no workspace for %d x %d partial products", splits * batch, M * N);
    }
    // A is K-contiguous unless transposed; the vector axis is K (A) or M (A^T).
    const bool va = aligned16(A) && lda % 4 == 0 && sA % 4 == 0 && (ta ? M % 4 == 0 : K % 4 == 0);
    const bool vb = aligned16(B) && ldb % 4 == 0 && sB % 4 == 0 && (tb ? K % 4 == 0 : N % 4 == 0);
    int rc;
    if (!ta && !tb) rc = launchCfg<false, false>(prm, batch, splits, plan.cfg, va, vb);
    else if (!ta && tb) rc = launchCfg<false, true>(prm, batch, splits, plan.cfg, va, vb);
    else if (ta && !tb) rc = launchCfg<true, false>(prm, batch, splits, plan.cfg, va, vb);
    else rc = launchCfg<true, true>(prm, batch, splits, plan.cfg, va, vb);
    if (rc || !partial) return rc;
    const long long total = (long long)M * N * batch;
    const int blocks = (int)std::min<long long>((total + 255) / 256, (long long)cuCount() * 16);
    hipLaunchKernelGGL(gemm_splitk_finish, dim3(blocks), dim3(256), 0, stream(), prm.ws, C, splits, batch, M, N, ldc,
                       sC);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// Split-K partials are kept to at most this many bytes of workspace.
constexpr size_t kMaxSplitWorkspace = (size_t)256 << 20;

int gemmF32(bool ta, bool tb, int batch, int M, int N, int K,
            const float* A, long long lda, long long sA,
            const float* B, long long ldb, long long sB,
            float* C, long long ldc, long long sC) {
    const bool wsOk = (size_t)64 * batch * M * N * sizeof(float) <= kMaxSplitWorkspace;
    const GemmPlan plan = planGemm(M, N, K, batch, wsOk);
    return gemmF32Run(ta, tb, batch, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, plan);
}

__global__ void zero_rows_kernel(float* C, int rows, int cols, long long ldc, long long sC) {
    const long long b = blockIdx.z;
    const long long n = (long long)rows * cols;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / cols, c = i % cols;
        C[b * sC + r * ldc + c] = 0.f;
    }
}

// Degenerate shapes: C is zeroed when its extent is valid (cpu_backend.ixx:246-251).
int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC) {
    if (!C || M <= 0 || N <= 0 || batch <= 0) return 0;
    const long long n = (long long)M * N;
    const int blocks = (int)std::min<long long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_rows_kernel, dim3(blocks, 1, batch), dim3(256), 0, stream(), C, M, N, ldc, sC);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int gemmF32Checked(const char* name, bool ta, bool tb, int batch, int M, int N, int K,
                   const float* A, long long lda, long long sA,
                   const float* B, long long ldb, long long sB,
                   float* C, long long ldc, long long sC) {
    clearError();
    if (batch <= 0 || M <= 0 || N <= 0) return 0;
    if (!C) return fail("%s: null output", name);
    if (!A || !B || K <= 0) return zeroOutput(C, batch, M, N, ldc, sC);
    if (batch > 65535) return fail("%s: batch %d exceeds 65535", name, batch);
    return gemmF32(ta, tb, batch, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC);
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipMatmul(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmul", false, false, 1, nM, nN, nK, pA, nK, 0, pB, nN, 0, pC, nN, 0);
}

int omHipMatmulTransB(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmulTransB", false, true, 1, nM, nN, nK, pA, nK, 0, pB, nK, 0, pC, nN, 0);
}

int omHipMatmulTransA(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmulTransA", true, false, 1, nM, nN, nK, pA, nM, 0, pB, nN, 0, pC, nN, 0);
}

int omHipBatchedMatmul(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
    return gemmF32Checked("omHipBatchedMatmul", false, false, nBatch, nM, nN, nK,
                          pA, nK, (long long)nM * nK, pB, nN, (long long)nK * nN, pC, nN, (long long)nM * nN);
}

int omHipBatchedMatmulTransB(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
    return gemmF32Checked("omHipBatchedMatmulTransB", false, true, nBatch, nM, nN, nK,
                          pA, nK, (long long)nM * nK, pB, nK, (long long)nN * nK, pC, nN, (long long)nM * nN);
}

int omHipGemmStridedBatched(int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                            const float* pA, long long nLda, long long nStrideA,
                            const float* pB, long long nLdb, long long nStrideB,
                            float* pC, long long nLdc, long long nStrideC) {
    clearError();
    if (nBatch > 0 && nM > 0 && nN > 0 && nK > 0) {
        if (nLda < (bTransA ? nM : nK) || nLdb < (bTransB ? nK : nN) || nLdc < nN)
            return fail("omHipGemmStridedBatched: leading dimension smaller than the row length");
        if (nStrideA < 0 || nStrideB < 0 || nStrideC < 0)
            return fail("omHipGemmStridedBatched: negative batch stride");
    }
    return gemmF32Checked("omHipGemmStridedBatched", bTransA != 0, bTransB != 0, nBatch, nM, nN, nK,
                          pA, nLda, nStrideA, pB, nLdb, nStrideB, pC, nLdc, nStrideC);
}

}  // extern "C"
