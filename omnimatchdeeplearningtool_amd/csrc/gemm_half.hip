// gemm_half.hip — fp16 / bf16 GEMM with fp32 accumulate on gfx950
// (v_mfma_f32_32x32x16_f16 / _bf16), fp32 output.
//
// The reference has no half-precision GEMM: its FP16Converter is a software
// converter (src/engine/om.engine.fp16.ixx:36-164) and every matmul runs in
// fp32 (cpu_backend.ixx:239-286). These entries compute what
// halfToFloat(A), halfToFloat(B), matmul would, with fp32 accumulation.
//
// Same block structure as the fp32 tile (double-buffered LDS slices, 32x32
// MFMA blocks per wave, the two lane halves reducing the two halves of a
// slice). Both operands are kept K-contiguous in LDS ([R][BK+8] halves) so a
// fragment (8 consecutive k of one row) is one ds_read_b128; an operand that is
// R-contiguous in HBM (B of A*B, A of A^T*B) is transposed on its way into LDS.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>

namespace omhip {

typedef float f32x16h __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct GemmHalfParams {
    const uint16_t* A;
    const uint16_t* B;
    float* C;
    int M, N, K;
    long long lda, ldb, ldc, sA, sB, sC;
    int tilesM, tilesN;
};

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct HCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int WAVES_N = BN / WN;
    static constexpr int NT = (BM / WM) * (BN / WN) * 64;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static constexpr int KH = BK / 2;
    static constexpr int LD = BK + 8;   // halves per LDS row
    static_assert(BK % 16 == 0, "BK multiple of 16");
};

// Loads an R x BK slice of an operand into LDS [R][LD] (k contiguous).
// KMAJOR: element (r,k) at P[r*ld+k]; otherwise at P[k*ld+r] (transposed on store).
template <bool KMAJOR, bool VEC, int R, int BK, int LD, int NT>
struct HalfLoader {
    static constexpr int ELEMS = R * BK;
    static constexpr int PER_T = VEC ? ELEMS / 8 / NT : ELEMS / NT;
    static_assert(ELEMS % (NT * (VEC ? 8 : 1)) == 0, "slice must split evenly");
    const uint16_t* p;
    long long ld;
    int rows, K, r0;
    u16x8 v8[VEC ? PER_T : 1];
    uint16_t v1[VEC ? 1 : PER_T];

    __device__ void coords(int e, int& r, int& k) const {
        if constexpr (VEC) {
            if constexpr (KMAJOR) { r = e / (BK / 8); k = (e % (BK / 8)) * 8; }
            else { k = e / (R / 8); r = (e % (R / 8)) * 8; }
        } else {
            if constexpr (KMAJOR) { r = e / BK; k = e % BK; }
            else { k = e / R; r = e % R; }
        }
    }

    __device__ void load(int k0, int tid) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int r, k;
            coords(tid + i * NT, r, k);
            const int gr = r0 + r, gk = k0 + k;
            const bool ok = gr < rows && gk < K;
            const uint16_t* src = KMAJOR ? p + (long long)gr * ld + gk : p + (long long)gk * ld + gr;
            if constexpr (VEC) {
                u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
                if (ok) v = *reinterpret_cast<const u16x8*>(src);
                v8[i] = v;
            } else {
                v1[i] = ok ? *src : (uint16_t)0;
            }
        }
    }

    __device__ void store(uint16_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int r, k;
            coords(tid + i * NT, r, k);
            if constexpr (VEC) {
                if constexpr (KMAJOR) {
                    *reinterpret_cast<u16x8*>(s + r * LD + k) = v8[i];
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) s[(r + e) * LD + k] = v8[i][e];
                }
            } else {
                s[r * LD + k] = v1[i];
            }
        }
    }
};

template <bool BF16>
__device__ __forceinline__ f32x16h mfma16(const u16x8& a, const u16x8& b, const f32x16h& c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
}

__device__ __forceinline__ void tileCoordsH(int bid, int total, int tilesM, int tilesN, int& tm, int& tn) {
    constexpr int XCDS = 8, GROUP_M = 8;
    int t = bid;
    if (total >= XCDS) {
        const int q = total / XCDS, rem = total % XCDS;
        const int xcd = bid % XCDS, idx = bid / XCDS;
        t = (xcd < rem) ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
    }
    const int perGroup = GROUP_M * tilesN;
    const int g = t / perGroup;
    const int firstM = g * GROUP_M;
    const int gsz = min(tilesM - firstM, GROUP_M);
    const int inG = t - g * perGroup;
    tm = firstM + inG % gsz;
    tn = inG / gsz;
}

template <class Cfg, bool BF16, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void gemm_half_kernel(GemmHalfParams p) {
    extern __shared__ uint16_t hsmem[];
    constexpr int SA = Cfg::BM * Cfg::LD, SB = Cfg::BN * Cfg::LD, STAGE = SA + SB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;
    int tm, tn;
    tileCoordsH(blockIdx.x, p.tilesM * p.tilesN, p.tilesM, p.tilesN, tm, tn);
    const long long batch = blockIdx.z;
    const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;

    HalfLoader<!TA, VA, Cfg::BM, Cfg::BK, Cfg::LD, Cfg::NT> la;
    la.p = p.A + batch * p.sA; la.ld = p.lda; la.rows = p.M; la.K = p.K; la.r0 = m0;
    HalfLoader<TB, VB, Cfg::BN, Cfg::BK, Cfg::LD, Cfg::NT> lb;
    lb.p = p.B + batch * p.sB; lb.ld = p.ldb; lb.rows = p.N; lb.K = p.K; lb.r0 = n0;

    f32x16h acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int li = lane & 31, h = lane >> 5;
    const int nk = (p.K + Cfg::BK - 1) / Cfg::BK;
    la.load(0, tid);
    lb.load(0, tid);
    la.store(hsmem, tid);
    lb.store(hsmem + SA, tid);
    __syncthreads();
    for (int t = 0; t < nk; ++t) {
        const int cur = t & 1;
        const bool more = (t + 1) < nk;
        if (more) {
            la.load((t + 1) * Cfg::BK, tid);
            lb.load((t + 1) * Cfg::BK, tid);
        }
        const uint16_t* sA = hsmem + cur * STAGE;
        const uint16_t* sB = sA + SA;
#pragma unroll
        for (int s = 0; s < Cfg::KH / 8; ++s) {
            const int kc = h * Cfg::KH + 8 * s;
            u16x8 a[Cfg::FM], b[Cfg::FN];
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
                a[fm] = *reinterpret_cast<const u16x8*>(sA + (wm * Cfg::WM + fm * 32 + li) * Cfg::LD + kc);
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn)
                b[fn] = *reinterpret_cast<const u16x8*>(sB + (wn * Cfg::WN + fn * 32 + li) * Cfg::LD + kc);
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn) acc[fm][fn] = mfma16<BF16>(a[fm], b[fn], acc[fm][fn]);
        }
        if (more) {
            uint16_t* nxt = hsmem + (cur ^ 1) * STAGE;
            la.store(nxt, tid);
            lb.store(nxt + SA, tid);
        }
        __syncthreads();
    }

    float* C = p.C + batch * p.sC;
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = n0 + wn * Cfg::WN + fn * 32 + li;
            if (col >= p.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < p.M) C[(long long)row * p.ldc + col] = acc[fm][fn][r];
            }
        }
}

using HCfgL = HCfg<256, 256, 32, 128, 128>;
using HCfgM = HCfg<128, 128, 32, 64, 64>;
using HCfgS = HCfg<64, 64, 32, 32, 32>;

template <class Cfg, bool BF16, bool TA, bool TB, bool VA, bool VB>
static int launchH(GemmHalfParams prm, int batch) {
    auto kern = gemm_half_kernel<Cfg, BF16, TA, TB, VA, VB>;
    const size_t lds = 2 * (size_t)(Cfg::BM + Cfg::BN) * Cfg::LD * sizeof(uint16_t);
    static bool s_attr = false;
    if (!s_attr) {
        OMHIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        s_attr = true;
    }
    prm.tilesM = (prm.M + Cfg::BM - 1) / Cfg::BM;
    prm.tilesN = (prm.N + Cfg::BN - 1) / Cfg::BN;
    hipLaunchKernelGGL(kern, dim3(prm.tilesM * prm.tilesN, 1, batch), dim3(Cfg::NT), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <class Cfg, bool BF16, bool TA, bool TB>
static int launchHV(const GemmHalfParams& prm, int batch, bool va, bool vb) {
    if (va && vb) return launchH<Cfg, BF16, TA, TB, true, true>(prm, batch);
    if (va) return launchH<Cfg, BF16, TA, TB, true, false>(prm, batch);
    if (vb) return launchH<Cfg, BF16, TA, TB, false, true>(prm, batch);
    return launchH<Cfg, BF16, TA, TB, false, false>(prm, batch);
}

template <bool BF16, bool TA, bool TB>
static int launchHC(const GemmHalfParams& prm, int batch, bool va, bool vb) {
    const long long cus = cuCount();
    auto tiles = [&](int bm, int bn) {
        return (long long)((prm.M + bm - 1) / bm) * ((prm.N + bn - 1) / bn) * batch;
    };
    // the 256x256 tile is only register-clean with 128-bit loads on both operands
    if (va && vb && tiles(256, 256) >= cus) return launchHV<HCfgL, BF16, TA, TB>(prm, batch, va, vb);
    if (tiles(128, 128) >= cus) return launchHV<HCfgM, BF16, TA, TB>(prm, batch, va, vb);
    return launchHV<HCfgS, BF16, TA, TB>(prm, batch, va, vb);
}

template <bool BF16>
static int dispatchH(bool ta, bool tb, const GemmHalfParams& prm, int batch, bool va, bool vb) {
    if (!ta && !tb) return launchHC<BF16, false, false>(prm, batch, va, vb);
    if (!ta && tb) return launchHC<BF16, false, true>(prm, batch, va, vb);
    if (ta && !tb) return launchHC<BF16, true, false>(prm, batch, va, vb);
    return launchHC<BF16, true, true>(prm, batch, va, vb);
}

int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC);

static int gemmHalf(const char* name, int dtype, bool ta, bool tb, int batch, int M, int N, int K,
                    const uint16_t* A, long long lda, long long sA, const uint16_t* B, long long ldb, long long sB,
                    float* C, long long ldc, long long sC) {
    clearError();
    if (batch <= 0 || M <= 0 || N <= 0) return 0;
    if (!C) return fail("%s: null output", name);
    if (!A || !B || K <= 0) return zeroOutput(C, batch, M, N, ldc, sC);
    if (batch > 65535) return fail("%s: batch %d exceeds 65535", name, batch);
    if (dtype != 0 && dtype != 1) return fail("%s: dtype must be 0 (fp16) or 1 (bf16)", name);
    GemmHalfParams prm{};
    prm.A = A; prm.B = B; prm.C = C; prm.M = M; prm.N = N; prm.K = K;
    prm.lda = lda; prm.ldb = ldb; prm.ldc = ldc; prm.sA = sA; prm.sB = sB; prm.sC = sC;
    auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    const bool va = al(A) && lda % 8 == 0 && sA % 8 == 0 && (ta ? M % 8 == 0 : K % 8 == 0);
    const bool vb = al(B) && ldb % 8 == 0 && sB % 8 == 0 && (tb ? K % 8 == 0 : N % 8 == 0);
    return dtype == 1 ? dispatchH<true>(ta, tb, prm, batch, va, vb) : dispatchH<false>(ta, tb, prm, batch, va, vb);
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipMatmulF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
    return gemmHalf("omHipMatmulF16", 0, false, false, 1, nM, nN, nK, pA, nK, 0, pB, nN, 0, pC, nN, 0);
}
int omHipMatmulBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
    return gemmHalf("omHipMatmulBF16", 1, false, false, 1, nM, nN, nK, pA, nK, 0, pB, nN, 0, pC, nN, 0);
}
int omHipMatmulTransBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
    return gemmHalf("omHipMatmulTransBF16", 0, false, true, 1, nM, nN, nK, pA, nK, 0, pB, nK, 0, pC, nN, 0);
}
int omHipMatmulTransBBF16(const uint16_t* pA, const uint16_t* pB, float* pC, int nM, int nK, int nN) {
    return gemmHalf("omHipMatmulTransBBF16", 1, false, true, 1, nM, nN, nK, pA, nK, 0, pB, nK, 0, pC, nN, 0);
}
int omHipGemmStridedBatchedHalf(int nDtype, int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                                const uint16_t* pA, long long nLda, long long nStrideA, const uint16_t* pB,
                                long long nLdb, long long nStrideB, float* pC, long long nLdc, long long nStrideC) {
    clearError();
    if (nBatch > 0 && nM > 0 && nN > 0 && nK > 0) {
        if (nLda < (bTransA ? nM : nK) || nLdb < (bTransB ? nK : nN) || nLdc < nN)
            return fail("omHipGemmStridedBatchedHalf: leading dimension smaller than the row length");
        if (nStrideA < 0 || nStrideB < 0 || nStrideC < 0)
            return fail("omHipGemmStridedBatchedHalf: negative batch stride");
    }
    return gemmHalf("omHipGemmStridedBatchedHalf", nDtype, bTransA != 0, bTransB != 0, nBatch, nM, nN, nK, pA, nLda,
                    nStrideA, pB, nLdb, nStrideB, pC, nLdc, nStrideC);
}

}  // extern "C"
