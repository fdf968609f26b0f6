// gemm_half.hip — fp16 / bf16 GEMM with fp32 accumulate on gfx950
// (v_mfma_f32_32x32x16_f16 / _bf16); output fp32, or rounded to nearest even
// into the input type, optionally after a per-column fp32 bias and ReLU (a
// Linear layer's x W + b in one pass).
//
// The reference has no half-precision GEMM: its FP16Converter is a software
// converter (src/engine/om.engine.fp16.ixx:36-164) and every matmul runs in
// fp32 (cpu_backend.ixx:239-286). These entries compute what
// halfToFloat(A), halfToFloat(B), matmul would, with fp32 accumulation.
//
// Two kernels:
//  * gemm_half_fast: R-major operands whose contiguous axis, leading dimension
//    and base are multiples of 8 halves, and K-major operands of any alignment
//    (every layout the networks produce). Slices are fetched with raw buffer
//    loads whose per-lane offset is fixed for the whole K walk (the slice
//    start rides in the scalar offset; rows past the matrix fall outside the
//    buffer range and read 0), so the mainloop spends almost no VALU on
//    addressing. A 16-byte-aligned K-major operand goes straight from the
//    buffer into LDS (buffer_load ... lds) in a swizzled unpadded [R][BK]
//    layout, and an MFMA fragment (8 consecutive k of one row) is one
//    ds_read_b128; one that is only 2-byte aligned (odd K or leading
//    dimension) is fetched 16 bytes at a time from the dword boundary below,
//    funnel-shifted into place in registers and stored to padded rows. An
//    operand that is R-contiguous in HBM (B of A*B, A of A^T*B) also goes
//    straight into LDS, in its own [BK][R] layout, and is transposed by the
//    fragment read (two ds_read_b64_tr_b16 per fragment). The MFMA takes the
//    B fragment as its first operand, so each lane ends up holding 4
//    consecutive output columns and the tile leaves in 128-bit stores (half
//    output and one-round fp32 grids: staged through LDS and written as whole
//    128-byte lines with streaming stores).
//  * gemm_half_generic: any other layout (element loads with bounds checks).
//
// Within a 16-deep MFMA step the two 32-lane halves supply k = 0..7 and
// k = 8..15 of the step; the sum over k is order-free, so this only changes
// rounding order.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace omhip {

typedef float f32x16h __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4h __attribute__((ext_vector_type(4)));

// Output: C (element offsets; fp32, or halves of the input type when outHalf)
// = act(A * B + bias) with bias [N] fp32 or null, act 0 identity, 1 ReLU.
struct GemmHalfParams {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    int M, N, K;
    long long lda, ldb, ldc, sA, sB, sC;
    int tilesM, tilesN;
    const float* bias;
    int act, outHalf;
};

template <bool BF16>
__device__ __forceinline__ uint16_t halfBits(float v) {   // round to nearest even
    if constexpr (BF16)
        return __builtin_bit_cast(uint16_t, (__bf16)v);
    else
        return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Epilogue of one output element: the bias add and ReLU in fp32 (in the
// order of tensorAddBias then relu), then the store in the output type.
template <bool BF16, class P>
__device__ __forceinline__ void storeOne(const P& p, long long off, int n, float v) {
    if (p.bias) v += p.bias[n];
    if (p.act == 1) v = v > 0.f ? v : 0.f;
    if (p.outHalf)
        static_cast<uint16_t*>(p.C)[off] = halfBits<BF16>(v);
    else
        static_cast<float*>(p.C)[off] = v;
}

// Four consecutive columns n .. n+3 of one row (n % 4 == 0, the element
// offset a multiple of 4 and the base 16-byte (fp32) / 8-byte (half) aligned).
template <bool BF16, class P>
__device__ __forceinline__ void storeFour(const P& p, long long off, int n, float v0, float v1, float v2, float v3) {
    if (p.bias) {
        v0 += p.bias[n]; v1 += p.bias[n + 1]; v2 += p.bias[n + 2]; v3 += p.bias[n + 3];
    }
    if (p.act == 1) {
        v0 = v0 > 0.f ? v0 : 0.f; v1 = v1 > 0.f ? v1 : 0.f; v2 = v2 > 0.f ? v2 : 0.f; v3 = v3 > 0.f ? v3 : 0.f;
    }
    if (p.outHalf) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 w = {(uint32_t)halfBits<BF16>(v0) | ((uint32_t)halfBits<BF16>(v1) << 16),
                         (uint32_t)halfBits<BF16>(v2) | ((uint32_t)halfBits<BF16>(v3) << 16)};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + off) = w;
    } else {
        typedef float f32x4e __attribute__((ext_vector_type(4)));
        const f32x4e w = {v0, v1, v2, v3};
        *reinterpret_cast<f32x4e*>(static_cast<float*>(p.C) + off) = w;
    }
}

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

// Workgroup id -> logical index such that each XCD (ids bid % 8) runs one
// contiguous range of the logical order: neighbouring tiles, which share
// operand rows or columns, then share one L2.
__device__ __forceinline__ int xcdRemap(int bid, int total) {
    constexpr int XCDS = 8;
    if (total < XCDS) return bid;
    const int q = total / XCDS, rem = total % XCDS;
    const int xcd = bid % XCDS, idx = bid / XCDS;
    return (xcd < rem) ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
}

// Logical tile index t -> (tm, tn): groups of 8 tile rows walked column by column.
__device__ __forceinline__ void groupCoords(int t, int tilesM, int tilesN, int& tm, int& tn) {
    constexpr int GROUP_M = 8;
    const int perGroup = GROUP_M * tilesN;
    const int g = t / perGroup;
    const int firstM = g * GROUP_M;
    const int gsz = min(tilesM - firstM, GROUP_M);
    const int inG = t - g * perGroup;
    tm = firstM + inG % gsz;
    tn = inG / gsz;
}

__device__ __forceinline__ void tileCoordsH(int bid, int total, int tilesM, int tilesN, int& tm, int& tn) {
    groupCoords(xcdRemap(bid, total), tilesM, tilesN, tm, tn);
}

template <class Cfg, bool BF16, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void gemm_half_generic(GemmHalfParams p) {
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

#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = n0 + wn * Cfg::WN + fn * 32 + li;
            if (col >= p.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < p.M) storeOne<BF16>(p, batch * p.sC + (long long)row * p.ldc + col, col, acc[fm][fn][r]);
            }
        }
}

using HCfgM = HCfg<128, 128, 32, 64, 64>;
using HCfgS = HCfg<64, 64, 32, 32, 32>;

template <class Cfg, bool BF16, bool TA, bool TB, bool VA, bool VB>
static int launchGeneric(GemmHalfParams prm, int batch) {
    auto kern = gemm_half_generic<Cfg, BF16, TA, TB, VA, VB>;
    const size_t lds = 2 * (size_t)(Cfg::BM + Cfg::BN) * Cfg::LD * sizeof(uint16_t);
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    prm.tilesM = (prm.M + Cfg::BM - 1) / Cfg::BM;
    prm.tilesN = (prm.N + Cfg::BN - 1) / Cfg::BN;
    hipLaunchKernelGGL(kern, dim3(prm.tilesM * prm.tilesN, 1, batch), dim3(Cfg::NT), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <class Cfg, bool BF16, bool TA, bool TB>
static int launchGenericV(const GemmHalfParams& prm, int batch, bool va, bool vb) {
    if (va && vb) return launchGeneric<Cfg, BF16, TA, TB, true, true>(prm, batch);
    if (va) return launchGeneric<Cfg, BF16, TA, TB, true, false>(prm, batch);
    if (vb) return launchGeneric<Cfg, BF16, TA, TB, false, true>(prm, batch);
    return launchGeneric<Cfg, BF16, TA, TB, false, false>(prm, batch);
}

template <bool BF16, bool TA, bool TB>
static int launchGenericC(const GemmHalfParams& prm, int batch, bool va, bool vb) {
    const long long tiles = (long long)((prm.M + 127) / 128) * ((prm.N + 127) / 128) * batch;
    if (tiles >= cuCount()) return launchGenericV<HCfgM, BF16, TA, TB>(prm, batch, va, vb);
    return launchGenericV<HCfgS, BF16, TA, TB>(prm, batch, va, vb);
}

// ---- fast kernel -------------------------------------------------------------

// Offsets at or above this byte count are outside every buffer view used by the
// fast kernel (views are limited to 2^30 bytes), so two such terms never wrap.
constexpr uint32_t kOOBH = 0x40000000u;
constexpr long long kMaxViewBytes = 0x40000000LL;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t halfRsrc(const void* base, uint32_t bytes) {
    // raw buffer, stride 0, range-checked against `bytes`
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

struct HalfFastParams {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    int M, N, K;
    int lda, ldb;        // < 2^21
    long long ldc, sA, sB, sC;
    int tilesM, tilesN;
    const float* bias;   // output as GemmHalfParams
    int act, outHalf;
    int batch;
    int flat;      // grid x runs over (batch, tile) pairs (else x = tile, z = batch)
    int compact;   // one tile holds a batch's whole C, stored through LDS (gemm_half_fast)
    int staged;    // SWAP tiles leave through LDS as whole-line streaming stores (storeStaged)
};

// K-major operand whose rows start at any half (an odd leading dimension,
// base or batch stride, e.g. P of P x V with 197 keys), through registers into
// padded LDS rows ([R][BK+8] halves). An R x BK slice is R*BK/8 chunks of 8
// halves; chunk e is (row e / (BK/8), k 8*(e % (BK/8))), so 8 consecutive lanes
// cover one row's 128 bytes. A chunk that starts at half h is fetched as the 16 bytes at
// the dword boundary below it plus the next dword, and shifted down by 16 bits
// when h is odd. The view starts at the dword holding the tile's first element
// and ends at the dword holding row rowsValid-1's K-th element (the 2 bytes
// after it, inside that same dword, are read but belong to no output that is
// kept: they fall past K, where the last slice zeroes every half, or in a row
// past the matrix). K-contiguous halves past K are zeroed explicitly on the
// last slice: there the next row's data lies, not the end of the view.
template <int R, int BK, int NT>
struct KMajorRaggedSlice {
    static constexpr bool DMA = false, SWZ = false, TR = false;
    static constexpr int CH = BK / 8;
    static constexpr int PER_T = R * CH / NT;
    static_assert(R * CH % NT == 0, "slice must split evenly");
    static constexpr int NLOADS = 2 * PER_T, NSTORES = PER_T;   // per thread and slice
    struct Regs {
        u32x4 v[PER_T];
    };
    __amdgpu_buffer_rsrc_t r;
    uint32_t voff[PER_T];   // byte offset of the dword holding the chunk's first half
    uint32_t sh[PER_T];     // 16 when that half is the dword's upper one, else 0

    __device__ void init(const uint16_t* base, int ld, int rowsValid, int K, int tid) {
        const int rv = rowsValid < R ? rowsValid : R;
        const uint32_t lead = (uint32_t)(reinterpret_cast<uintptr_t>(base) & 2u) >> 1;   // halves below base in its dword
        const uint16_t* b4 = base - lead;
        const uint32_t endHalves = (uint32_t)(rv - 1) * (uint32_t)ld + (uint32_t)K + lead;
        r = halfRsrc(b4, ((endHalves * 2u) + 3u) & ~3u);
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT;
            const uint32_t h = (uint32_t)(e / CH) * (uint32_t)ld + (uint32_t)(e % CH) * 8u + lead;
            voff[i] = (h * 2u) & ~3u;
            sh[i] = (h & 1u) * 16u;
        }
    }
    // FULL: the slice lies inside K. The slice start k0 is a multiple of BK, so
    // the scalar offset 2*k0 keeps the dword alignment.
    template <bool FULL>
    __device__ void load(int k0, int K, int tid, Regs& g) const {
        const uint32_t soff = (uint32_t)k0 * 2u;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const u32x4 lo = ld128(r, voff[i], soff);
            const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(r, voff[i] + 16u, soff, 0);
            u32x4 v = {__builtin_amdgcn_alignbit(lo[1], lo[0], sh[i]), __builtin_amdgcn_alignbit(lo[2], lo[1], sh[i]),
                       __builtin_amdgcn_alignbit(lo[3], lo[2], sh[i]), __builtin_amdgcn_alignbit(hi, lo[3], sh[i])};
            if (!FULL && k0 + BK > K) {
                const int n = K - (k0 + ((tid + i * NT) % CH) * 8);   // halves of this chunk inside K
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[j] &= (2 * j < n ? 0x0000ffffu : 0u) | (2 * j + 1 < n ? 0xffff0000u : 0u);
            }
            g.v[i] = v;
        }
    }
    template <int LD>
    __device__ void store(uint16_t* s, int tid, const Regs& g) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT;
            *reinterpret_cast<u32x4*>(s + (e / CH) * LD + (e % CH) * 8) = g.v[i];
        }
    }
};

// K-major operand in 16-byte chunks, loaded straight into LDS
// (buffer_load_dwordx4 ... lds): one instruction writes 64 lanes x 16 bytes
// contiguously at the LDS address in m0, lane L at +16L, so 8 rows of 64 halves
// per instruction, with no VGPR staging and no ds_write. The LDS rows are
// unpadded (BK = 64 halves) and the 16-byte chunk c of row r sits in slot
// c ^ ((r >> 1) & 7): the 16 lanes of a fragment read (rows r0 .. r0+15, one
// chunk) then hit 16 distinct 16-byte bank groups. Lane L of the instruction
// that fills rows 8j .. 8j+7 therefore fetches chunk (L % 8) ^ ((r >> 1) & 7) of
// row r = 8j + L / 8. Lanes past the matrix rows or past K use an offset
// outside the buffer view, for which the load writes zeros.
typedef __attribute__((address_space(3))) void* LdsPtr;

template <int R, int BK, int NT>
struct KMajorDmaSlice {
    static_assert(BK == 64, "8 chunks of 8 halves per row");
    static constexpr bool DMA = true, SWZ = true, TR = false;
    static constexpr int NW = NT / 64;
    static constexpr int INSTR = R / 8 / NW;   // instructions per wave and slice
    static_assert(R % (8 * NW) == 0, "rows must split evenly over the waves");
    static constexpr int NLOADS = INSTR, NSTORES = 0;
    struct Regs {};
    __amdgpu_buffer_rsrc_t r;
    uint32_t voff[INSTR];
    uint32_t kc[INSTR];   // k offset (halves) of the lane's chunk within the slice
    int wave;

    __device__ void init(const uint16_t* base, int ld, int rowsValid, int K, int tid) {
        const int rv = rowsValid < R ? rowsValid : R;
        r = halfRsrc(base, ((uint32_t)(rv - 1) * (uint32_t)ld + (uint32_t)K) * 2u);
        wave = tid >> 6;
        const int lane = tid & 63;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int row = 8 * (wave + i * NW) + lane / 8;
            const int c = (lane & 7) ^ ((row >> 1) & 7);
            kc[i] = (uint32_t)c * 8u;
            voff[i] = row < rv ? ((uint32_t)row * (uint32_t)ld + (uint32_t)c * 8u) * 2u : kOOBH;
        }
    }
    // Writes the slice starting at k0 into dst (this operand's region of an LDS stage).
    template <bool FULL>
    __device__ void dma(int k0, int K, uint16_t* dst) const {
        const uint32_t soff = (uint32_t)k0 * 2u;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const uint32_t vo = (FULL || k0 + (int)kc[i] < K) ? voff[i] : kOOBH;   // K % 8 == 0: whole chunks
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)(dst + (wave + i * NW) * 8 * BK), 16, vo, soff, 0, 0);
        }
    }
    template <bool FULL>
    __device__ void load(int, int, int, Regs&) const {}
    template <int LD>
    __device__ void store(uint16_t*, int, const Regs&) const {}
};

template <bool RAG, int R, int BK, int NT>
using KMajorFor = std::conditional_t<RAG, KMajorRaggedSlice<R, BK, NT>, KMajorDmaSlice<R, BK, NT>>;

// LDS layout of one operand's slice: padded rows (register path) or
// unpadded swizzled rows (DMA path); offset (halves) of chunk c of row r.
template <bool SWZ, int LDP, int BK>
__device__ __forceinline__ int ldsChunk(int r, int c) {
    if constexpr (SWZ)
        return r * BK + ((c ^ ((r >> 1) & 7)) << 3);
    else
        return r * LDP + (c << 3);
}

// 16 bytes per lane from the buffer straight into LDS at dst + 16 * lane.
__device__ __forceinline__ void dmaLoad16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)dst, 16, voff, soff, 0, 0);
}

template <int R, int BK, int NT>
struct RMajorDmaSlice {
    static constexpr bool DMA = true, SWZ = false, TR = true;
    static constexpr int NW = NT / 64;
    static constexpr int CH = R / 8;              // chunks per k row
    static constexpr int ROWS_PER_I = 64 / CH;    // k rows per DMA instruction
    static constexpr int INSTR = BK / ROWS_PER_I / NW;
    static_assert(CH >= 8 && CH <= 64 && BK % (ROWS_PER_I * NW) == 0, "k rows must split evenly over the waves");
    static constexpr int NLOADS = INSTR, NSTORES = 0;
    struct Regs {};
    __amdgpu_buffer_rsrc_t r;
    uint32_t voff[INSTR];
    uint32_t ld2;
    int wave;

    static __device__ __forceinline__ int swz(int k) { return ((k & 1) * 10 + ((k >> 1) & 1) * 4) & (CH - 1); }

    __device__ void init(const uint16_t* base, int ld, int colsValid, int K, int tid) {
        ld2 = (uint32_t)ld * 2u;
        const int cv = colsValid < R ? colsValid : R;
        r = halfRsrc(base, (uint32_t)(K - 1) * ld2 + (uint32_t)cv * 2u);
        wave = tid >> 6;
        const int lane = tid & 63;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int k = (wave + i * NW) * ROWS_PER_I + lane / CH;
            const int c = (lane % CH) ^ swz(k);
            voff[i] = (c * 8 < cv) ? (uint32_t)k * ld2 + (uint32_t)c * 16u : kOOBH;   // cols % 8 == 0
        }
    }
    template <bool FULL>   // rows past K read 0 either way
    __device__ void dma(int k0, int /*K*/, uint16_t* dst) const {
        const uint32_t soff = (uint32_t)k0 * ld2;
#pragma unroll
        for (int i = 0; i < INSTR; ++i)
            dmaLoad16(r, dst + (wave + i * NW) * 512, voff[i], soff);
    }
    template <bool FULL>
    __device__ void load(int, int, int, Regs&) const {}
    template <int LD>
    __device__ void store(uint16_t*, int, const Regs&) const {}
};

// Per-lane LDS offsets of an R-major operand's F fragments (rows base + 32j
// .. +31, k = 16s + 8h .. +7 of step s). ds_read_b64_tr_b16 returns to lane i
// of each 16-lane group the 4 halves E[4j + i/4][i%4], j = 0..3, where E[q] is
// what lane q of the group addressed; so lane q addresses k row 8h + q/4 (+4
// for the second read) at column 16g + 4(q%4) (g = lane bit 4), and lane l
// then holds rows base + 32j + l%32, k = 8h + 0..7: the MFMA operand layout.
//
// The reads are issued as inline assembly: the compiler treats the
// ds_read_tr builtin as possibly aliasing the in-flight LDS DMA of the next
// slice (which writes the other stage) and waits for every global load before
// the first one, which serialises the load latency with the slice's MFMAs.
// The compiler does not count these reads, so wait() (lgkmcnt 0, with the
// fragments passed through so their MFMAs stay behind it) must precede any
// use; the compiler's own LDS waits stay correct because LDS reads complete
// in issue order and extra reads in between only make its counts stricter.
typedef uint32_t u32x2t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t ldsAddr(const uint16_t* p) { return (uint32_t)(uintptr_t)(LdsPtr)(p); }

template <int I, int N, class F>
__device__ __forceinline__ void staticFor(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        staticFor<I + 1, N>(f);
    }
}

template <int R, int F>
struct TrFrags {
    uint32_t off[F];   // bytes from the operand's stage base, step 0, first read
    __device__ void init(int base, int lane) {
        const int q = lane & 15, g = (lane >> 4) & 1, h = lane >> 5;
        const int k = 8 * h + (q >> 2);
        const int sw = RMajorDmaSlice<R, 64, 64>::swz(k);
#pragma unroll
        for (int j = 0; j < F; ++j) {
            const int c = (base + 32 * j) / 8 + 2 * g + ((q & 3) >> 1);
            off[j] = 2u * (uint32_t)(k * R + ((c ^ sw) << 3) + 4 * (q & 1));
        }
    }
    // One read (half HH of fragment J at step STEP) from the stage base b (LDS bytes).
    template <int STEP, int J, int HH>
    __device__ __forceinline__ u32x2t half(uint32_t b) const {
        u32x2t r;
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(b + off[J]), "i"(STEP * 32 * R + HH * 8 * R));
        return r;
    }
    template <int STEP>
    __device__ __forceinline__ void issue(const uint16_t* s, u32x4 (&dst)[F]) const {
        const uint32_t b = ldsAddr(s);
        staticFor<0, F>([&](auto J) {
            const u32x2t lo = half<STEP, decltype(J)::value, 0>(b), hi = half<STEP, decltype(J)::value, 1>(b);
            dst[J] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        });
    }
    static __device__ __forceinline__ void wait(u32x4 (&f)[F]) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int j = 0; j < F; ++j) asm volatile("" : "+v"(f[j]));
    }
};

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct FCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int WAVES_N = BN / WN;
    static constexpr int NT = (BM / WM) * (BN / WN) * 64;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static constexpr int LD = BK + 8;   // halves per LDS row
    static constexpr int SA = BM * LD, SB = BN * LD, STAGE = SA + SB;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(uint16_t);
    static_assert(BK % 16 == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
};

template <bool BF16>
__device__ __forceinline__ f32x16h mfma16u(const u32x4& a, const u32x4& b, const f32x16h& c) {
    return mfma16<BF16>(__builtin_bit_cast(u16x8, a), __builtin_bit_cast(u16x8, b), c);
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSgMfma = 0x008, kSgVmemRead = 0x020, kSgDsRead = 0x100, kSgDsWrite = 0x200;

// Fragments of 16-deep MFMA step s: 8 consecutive k (lane half h: k = 16s+8h ..)
// of rows li of each 32-row block of the wave's sub-tile.
// K-major operands' fragments of step s; an R-major operand (TR) is issued
// through its TrFrags instead.
template <class Cfg, class LA, class LB, int S, bool KONLY = false>
__device__ __forceinline__ void readFrags(const uint16_t* sA, const uint16_t* sB, u32x4 (&a)[Cfg::FM],
                                          u32x4 (&b)[Cfg::FN], int wm, int wn, int li, int h,
                                          const TrFrags<Cfg::BM, Cfg::FM>& tra, const TrFrags<Cfg::BN, Cfg::FN>& trb) {
    const int c = S * 2 + h;   // chunk of 8 k
    if constexpr (LA::TR) {
        if constexpr (!KONLY) tra.template issue<S>(sA, a);
    } else {
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm)
            a[fm] = *reinterpret_cast<const u32x4*>(sA + ldsChunk<LA::SWZ, Cfg::LD, Cfg::BK>(wm * Cfg::WM + fm * 32 + li, c));
    }
    if constexpr (LB::TR) {
        if constexpr (!KONLY) trb.template issue<S>(sB, b);
    } else {
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn)
            b[fn] = *reinterpret_cast<const u32x4*>(sB + ldsChunk<LB::SWZ, Cfg::LD, Cfg::BK>(wn * Cfg::WN + fn * 32 + li, c));
    }
}

// Loader types and LDS footprint of the fast kernel for a layout.
template <class Cfg, bool TA, bool TB, bool RAG>
struct HalfOps {
    using LA = std::conditional_t<TA, RMajorDmaSlice<Cfg::BM, Cfg::BK, Cfg::NT>, KMajorFor<RAG, Cfg::BM, Cfg::BK, Cfg::NT>>;
    using LB = std::conditional_t<TB, KMajorFor<RAG, Cfg::BN, Cfg::BK, Cfg::NT>, RMajorDmaSlice<Cfg::BN, Cfg::BK, Cfg::NT>>;
    static constexpr int SA = Cfg::BM * (LA::SWZ || LA::TR ? Cfg::BK : Cfg::LD);
    static constexpr int SB = Cfg::BN * (LB::SWZ || LB::TR ? Cfg::BK : Cfg::LD);
    static constexpr int STAGE = SA + SB;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(uint16_t);
    static constexpr bool ANY_DMA = LA::DMA || LB::DMA;
};

template <class Cfg, bool BF16, bool SWAP>
__device__ __forceinline__ void mfmaStep(const u32x4 (&a)[Cfg::FM], const u32x4 (&b)[Cfg::FN],
                                         f32x16h (&acc)[Cfg::FM][Cfg::FN]) {
    // SWAP: B first, so the 32x32 result has n along its rows and m along lanes.
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn)
            acc[fm][fn] = SWAP ? mfma16u<BF16>(b[fn], a[fm], acc[fm][fn]) : mfma16u<BF16>(a[fm], b[fn], acc[fm][fn]);
}

// The MFMAs of one step with the next step's R-major (TR) fragment reads
// issued one before each MFMA (the rest after the last), each pair closed by
// a scheduling barrier: left alone, the scheduler moves the MFMAs around the
// read asm freely (it does not see LDS reads in it) and bunches the reads.
template <class Cfg, bool BF16, bool SWAP, class LA, class LB, int SN>
__device__ __forceinline__ void mfmaStepTr(const u32x4 (&a)[Cfg::FM], const u32x4 (&b)[Cfg::FN], u32x4 (&an)[Cfg::FM],
                                           u32x4 (&bn)[Cfg::FN], f32x16h (&acc)[Cfg::FM][Cfg::FN], const uint16_t* sA,
                                           const uint16_t* sB, const TrFrags<Cfg::BM, Cfg::FM>& tra,
                                           const TrFrags<Cfg::BN, Cfg::FN>& trb) {
    constexpr int RA = LA::TR ? 2 * Cfg::FM : 0, RB = LB::TR ? 2 * Cfg::FN : 0, NM = Cfg::FM * Cfg::FN;
    u32x2t pa[2 * Cfg::FM], pb[2 * Cfg::FN];
    const uint32_t baseA = ldsAddr(sA), baseB = ldsAddr(sB);
    auto rd = [&](auto R) {
        constexpr int r = decltype(R)::value;
        if constexpr (r < RA) pa[r] = tra.template half<SN, r / 2, r % 2>(baseA);
        else pb[r - RA] = trb.template half<SN, (r - RA) / 2, (r - RA) % 2>(baseB);
    };
    staticFor<0, NM>([&](auto I) {
        constexpr int m = decltype(I)::value, fm = m / Cfg::FN, fn = m % Cfg::FN;
        if constexpr (m < RA + RB) rd(I);
        acc[fm][fn] = SWAP ? mfma16u<BF16>(b[fn], a[fm], acc[fm][fn]) : mfma16u<BF16>(a[fm], b[fn], acc[fm][fn]);
        __builtin_amdgcn_sched_barrier(0);
    });
    staticFor<NM, RA + RB>(rd);
    if constexpr (LA::TR)
#pragma unroll
        for (int j = 0; j < Cfg::FM; ++j) an[j] = u32x4{pa[2 * j][0], pa[2 * j][1], pa[2 * j + 1][0], pa[2 * j + 1][1]};
    if constexpr (LB::TR)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j) bn[j] = u32x4{pb[2 * j][0], pb[2 * j][1], pb[2 * j + 1][0], pb[2 * j + 1][1]};
}

// Interleaves NMEM memory instructions of kind MASK with NMFMA MFMAs (spread
// evenly), so LDS traffic overlaps matrix-core execution.
template <int MASK, int NMEM, int NMFMA, int I = 0, int LEFT = NMFMA>
__device__ __forceinline__ void interleave() {
    if constexpr (I < NMEM) {
        constexpr int m = (LEFT + (NMEM - I) - 1) / (NMEM - I);
        __builtin_amdgcn_sched_group_barrier(MASK, 1, 0);
        if constexpr (m > 0) __builtin_amdgcn_sched_group_barrier(kSgMfma, m, 0);
        interleave<MASK, NMEM, NMFMA, I + 1, LEFT - m>();
    } else if constexpr (LEFT > 0) {
        __builtin_amdgcn_sched_group_barrier(kSgMfma, LEFT, 0);
    }
}

// Compact store (fp32 C, no bias or activation, one tile covering all M x N,
// ldc == N, 16-byte aligned base): the batch's C is one contiguous run of
// M*N floats whose rows need not start on a 16-byte boundary (e.g. 197 x 197
// blocks of a batched product with K > 64; one-slice products such as the
// attention scores take 64x64 tiles instead). Element stores of such rows leave partly written cache
// lines behind each store instruction; here the finished tile goes to LDS in
// C's own layout, a group of wave rows at a time, and the workgroup writes
// the run with aligned 16-byte streaming (nt) stores (a scalar head and tail). LDS element
// pre + j holds C element cb + r0*N + j, where pre = cb mod 4 and r0*N is a
// multiple of 4, so the 16-byte LDS reads are aligned exactly when the
// global stores are.
template <class Cfg, size_t LDS_BYTES>
__device__ __forceinline__ void storeCompact(const HalfFastParams& p, const f32x16h (&acc)[Cfg::FM][Cfg::FN],
                                             uint16_t* hsm, long long cb, int wm, int wn, int li, int h, int tid) {
    constexpr int WR = Cfg::BM / Cfg::WM;                   // wave rows of the tile
    constexpr int LDSF = (int)(LDS_BYTES / sizeof(float));
    static_assert(Cfg::WM * Cfg::BN + 4 <= LDSF, "one wave row of the tile fits in LDS");
    float* cs = reinterpret_cast<float*>(hsm);
    float* C = static_cast<float*>(p.C);
    const int pre = (int)(cb & 3);
    const int g = min(WR, (LDSF - 4) / (Cfg::WM * p.N));   // wave rows per pass (>= 1: N <= BN)
    for (int w0 = 0; w0 < WR; w0 += g) {
        const int r0 = w0 * Cfg::WM;
        if (r0 >= p.M) break;
        const int r1 = min(p.M, (w0 + g) * Cfg::WM);
        __syncthreads();   // LDS free: the mainloop's or the previous pass's reads are done
        if (wm >= w0 && wm < w0 + g) {
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn) {
                const int n = wn * Cfg::WN + fn * 32 + li;
#pragma unroll
                for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (m < p.M && n < p.N) cs[pre + (m - r0) * p.N + n] = acc[fm][fn][r];
                    }
            }
        }
        __syncthreads();
        const long long gb = cb + (long long)r0 * p.N;   // C element of LDS element pre
        const int cnt = (r1 - r0) * p.N;
        const int head = min(cnt, (int)((4 - (gb & 3)) & 3));   // elements before the first aligned one
        const int nvec = (cnt - head) >> 2;
        for (int j = tid; j < head; j += Cfg::NT) C[gb + j] = cs[pre + j];
        for (int v = tid; v < nvec; v += Cfg::NT) {
            const int j = head + 4 * v;
            __builtin_nontemporal_store(*reinterpret_cast<const f32x4h*>(cs + pre + j), reinterpret_cast<f32x4h*>(C + gb + j));
        }
        for (int j = head + 4 * nvec + tid; j < cnt; j += Cfg::NT) C[gb + j] = cs[pre + j];
    }
}

// Staged store of a SWAP tile, for half output and for fp32 grids of one
// round (tiles <= CUs). In the SWAP layout a store instruction of a wave
// covers 32 rows with 32 bytes each. Here each wave parks 32 rows of its own
// WM x WN sub-tile at a time in a private LDS region and writes them back row
// by row, 4 columns per lane, so an instruction writes whole 128-byte lines,
// and writes them as streaming (nt) stores: they leave L2 as they arrive
// instead of remaining dirty in it until the write-back at the end of the
// launch. Measured on MI355X against the register stores (fp16, 12608-row
// ViT-B/16 projections): half output 2-5 % faster on every shape (QKV 60.9 ->
// 58.5 us, fc2 74.7 -> 71.1), fp32 output of one-round grids 6-8 % faster
// (fc2 76.7 -> 71.9 us); fp32 grids of several rounds were 2-4 % slower with
// it and keep the register stores. LDS is wave-private after the block
// barrier that ends the mainloop, and a wave's LDS accesses complete in order.
// Compiled into the 256 x 256 tile (8 waves) only, where it was measured: in
// the small tiles the extra path cost the register path its allocation
// (batched P.V, 64 x 64 tiles: 28.8 -> 31.8 us).
template <class Cfg>
struct StagedStore {
    static constexpr bool USED = Cfg::NT == 512;
    static constexpr int PF = Cfg::WN + 4;   // floats per staged row (bank offset 4 from row to row)
    static constexpr size_t LDS_BYTES = (size_t)(Cfg::NT / 64) * 32 * PF * sizeof(float);
};

// Orders a wave's own LDS accesses across lanes: the writes before it are
// complete and visible to every lane of the wave before the reads after it
// (and the reads before it before the writes after it). No instruction is
// needed on gfx950 beyond keeping the compiler from moving accesses across it.
__device__ __forceinline__ void waveLdsOrder() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <class Cfg>
__device__ __forceinline__ void stagedBias(const HalfFastParams& p, int n0, int wn, int lane, float (&bz)[4]) {
    constexpr int LPR = Cfg::WN / 4;
    const int n = n0 + wn * Cfg::WN + 4 * (lane % LPR);   // as storeStaged's columns
#pragma unroll
    for (int j = 0; j < 4; ++j) bz[j] = 0.f;
    if (p.bias && n < p.N) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bz[j] = p.bias[n + j];
    }
}

// bz: the lane's four bias values (stagedBias, loaded before the main loop so that
// their latency is hidden by it).
template <class Cfg, bool BF16>
__device__ __forceinline__ void storeStaged(const HalfFastParams& p, const f32x16h (&acc)[Cfg::FM][Cfg::FN],
                                            uint16_t* hsm, long long cb, int m0, int n0, int wm, int wn, int li,
                                            int h, int lane, int wave, const float (&bz)[4]) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    constexpr int PF = StagedStore<Cfg>::PF;
    constexpr int LPR = Cfg::WN / 4;        // lanes per row
    constexpr int RPI = 64 / LPR;           // rows per store instruction
    float* st = reinterpret_cast<float*>(hsm) + wave * 32 * PF;
    const int lr = lane / LPR, lc = 4 * (lane % LPR);
    const int n = n0 + wn * Cfg::WN + lc;   // the lane's four columns n .. n+3 (N % 4 == 0: all in or all out)
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm) {
        // lane (li, h) holds row li, columns fn*32 + 8g + 4h .. +3 of block (fm, fn)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<f32x4h*>(st + li * PF + fn * 32 + 8 * g + 4 * h) =
                    f32x4h{acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2], acc[fm][fn][4 * g + 3]};
        waveLdsOrder();   // rows written by one lane are read by others
        const int mb = m0 + wm * Cfg::WM + fm * 32;   // first row of the 32-row block
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i) {
            const int r = i * RPI + lr;
            f32x4h v = *reinterpret_cast<const f32x4h*>(st + r * PF + lc);
            const int m = mb + r;
            if (m < p.M && n < p.N) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {   // as storeFour: bias, then ReLU
                    if (p.bias) v[j] += bz[j];
                    if (p.act == 1) v[j] = v[j] > 0.f ? v[j] : 0.f;
                }
                const long long off = cb + (long long)m * p.ldc + n;
                if (p.outHalf)
                    __builtin_nontemporal_store(
                        u32x2{(uint32_t)halfBits<BF16>(v[0]) | ((uint32_t)halfBits<BF16>(v[1]) << 16),
                              (uint32_t)halfBits<BF16>(v[2]) | ((uint32_t)halfBits<BF16>(v[3]) << 16)},
                        reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + off));
                else
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4h*>(static_cast<float*>(p.C) + off));
            }
        }
        waveLdsOrder();   // every lane has read this block before the next block's writes
    }
}

// SWAP (C rows allow 4-column stores: N, ldc, batch stride multiples of 4 and
// the base 16-byte aligned for fp32, 8-byte for half output) puts the B
// fragment first so each lane holds 4 consecutive columns; otherwise lanes run
// along n for coalesced element stores.
// RAG: the K-major operands' rows may start at any half (KMajorRaggedSlice).
template <class Cfg, bool BF16, bool TA, bool TB, bool SWAP, bool RAG>
__global__ __launch_bounds__(Cfg::NT) void gemm_half_fast(HalfFastParams p) {
    extern __shared__ uint16_t hsm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;
    const int li = lane & 31, h = lane >> 5;
    int tm, tn;
    long long batch;
    if (p.flat) {   // the tiles of one batch run on one XCD and share its L2
        const int tiles = p.tilesM * p.tilesN;
        const int t = xcdRemap(blockIdx.x, tiles * p.batch);
        batch = t / tiles;
        groupCoords(t - (int)batch * tiles, p.tilesM, p.tilesN, tm, tn);
    } else {
        tileCoordsH(blockIdx.x, p.tilesM * p.tilesN, p.tilesM, p.tilesN, tm, tn);
        batch = blockIdx.z;
    }
    const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
    const uint16_t* Ab = p.A + batch * p.sA;
    const uint16_t* Bb = p.B + batch * p.sB;
    float bzPre[4] = {0.f, 0.f, 0.f, 0.f};   // the staged store's bias, loaded ahead of the main loop
    if constexpr (SWAP && StagedStore<Cfg>::USED) {
        if (p.staged) stagedBias<Cfg>(p, n0, wn, lane, bzPre);
    }

    // A's rows are m: K-major unless transposed. B's rows are n: K-major when transposed.
    using Ops = HalfOps<Cfg, TA, TB, RAG>;
    using LA = typename Ops::LA;
    using LB = typename Ops::LB;
    constexpr int SA = Ops::SA, STAGE = Ops::STAGE;
    LA la;
    LB lb;
    la.init(TA ? Ab + m0 : Ab + (long long)m0 * p.lda, p.lda, p.M - m0, p.K, tid);
    lb.init(TB ? Bb + (long long)n0 * p.ldb : Bb + n0, p.ldb, p.N - n0, p.K, tid);
    typename LA::Regs ra;
    typename LB::Regs rb;

    f32x16h acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = (p.K + Cfg::BK - 1) / Cfg::BK;
    const int nFull = p.K / Cfg::BK;   // slices entirely inside K
    // first slice into stage 0 (a DMA operand writes LDS itself)
    if constexpr (LA::DMA) la.template dma<false>(0, p.K, hsm);
    else la.template load<false>(0, p.K, tid, ra);
    if constexpr (LB::DMA) lb.template dma<false>(0, p.K, hsm + SA);
    else lb.template load<false>(0, p.K, tid, rb);
    if constexpr (!LA::DMA) la.template store<Cfg::LD>(hsm, tid, ra);
    if constexpr (!LB::DMA) lb.template store<Cfg::LD>(hsm + SA, tid, rb);
    if constexpr (Ops::ANY_DMA) __builtin_amdgcn_s_waitcnt(0);   // LDS writes of the DMA loads done
    __syncthreads();
    // One slice per trip: fetch slice t+1 into registers, run slice t from LDS
    // stage t&1, park slice t+1 in the other stage. (Unrolling two slices to
    // make the stage offset a constant lets the scheduler interleave both
    // bodies and run out of VGPRs.)
    constexpr int STEPS = Cfg::BK / 16;
    constexpr int NFRAG = (LA::TR ? 0 : Cfg::FM) + (LB::TR ? 0 : Cfg::FN);   // compiler-issued LDS reads per step
    TrFrags<Cfg::BM, Cfg::FM> tra;
    TrFrags<Cfg::BN, Cfg::FN> trb;
    if constexpr (LA::TR) tra.init(wm * Cfg::WM, lane);
    if constexpr (LB::TR) trb.init(wn * Cfg::WN, lane);
    // Runs slice t from LDS stage t&1 as a software pipeline: the fragments of
    // step s+1 are read while the MFMAs of step s run, and the next slice's
    // registers (fetched at the top) are written to the other stage during the
    // last step. The group barriers pin that interleave.
    auto runSlice = [&](int t, bool more) {
        const uint16_t* sA = hsm + (t & 1) * STAGE;
        const uint16_t* sB = sA + SA;
        uint16_t* nxt = hsm + ((t & 1) ^ 1) * STAGE;
        u32x4 fa[2][Cfg::FM], fb[2][Cfg::FN];
        readFrags<Cfg, LA, LB, 0>(sA, sB, fa[0], fb[0], wm, wn, li, h, tra, trb);
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, NFRAG, 0);
        staticFor<0, STEPS>([&](auto I) {
            constexpr int st = decltype(I)::value;
            if constexpr (LA::TR || LB::TR) {   // this step's fragments landed (and nothing else is read yet)
                if constexpr (LA::TR) TrFrags<Cfg::BM, Cfg::FM>::wait(fa[st & 1]);
                if constexpr (LB::TR) TrFrags<Cfg::BN, Cfg::FN>::wait(fb[st & 1]);
            }
            if constexpr (st + 1 < STEPS) {
                readFrags<Cfg, LA, LB, st + 1, true>(sA, sB, fa[(st + 1) & 1], fb[(st + 1) & 1], wm, wn, li, h, tra, trb);
                if constexpr (LA::TR || LB::TR)
                    mfmaStepTr<Cfg, BF16, SWAP, LA, LB, st + 1>(fa[st & 1], fb[st & 1], fa[(st + 1) & 1], fb[(st + 1) & 1],
                                                             acc, sA, sB, tra, trb);
                else
                    mfmaStep<Cfg, BF16, SWAP>(fa[st & 1], fb[st & 1], acc);
                if constexpr (!(LA::TR || LB::TR)) interleave<kSgDsRead, NFRAG, Cfg::FM * Cfg::FN>();
            } else {
                if (more) {
                    if constexpr (!LA::DMA) la.template store<Cfg::LD>(nxt, tid, ra);
                    if constexpr (!LB::DMA) lb.template store<Cfg::LD>(nxt + SA, tid, rb);
                }
                mfmaStep<Cfg, BF16, SWAP>(fa[st & 1], fb[st & 1], acc);
                interleave<kSgDsWrite, LA::NSTORES + LB::NSTORES, Cfg::FM * Cfg::FN>();
            }
        });
    };
    auto step = [&](int t, auto fullTag) {
        constexpr bool FULL = decltype(fullTag)::value;
        // stage (t+1)&1 was last read in slice t-1, which every wave finished before the barrier
        uint16_t* nxt = hsm + ((t & 1) ^ 1) * STAGE;
        if constexpr (LA::DMA) la.template dma<FULL>((t + 1) * Cfg::BK, p.K, nxt);
        else la.template load<FULL>((t + 1) * Cfg::BK, p.K, tid, ra);
        if constexpr (LB::DMA) lb.template dma<FULL>((t + 1) * Cfg::BK, p.K, nxt + SA);
        else lb.template load<FULL>((t + 1) * Cfg::BK, p.K, tid, rb);
        __builtin_amdgcn_sched_group_barrier(kSgVmemRead, LA::NLOADS + LB::NLOADS, 0);
        runSlice(t, true);
        if constexpr (Ops::ANY_DMA) __builtin_amdgcn_s_waitcnt(0);   // this wave's DMA writes landed
        __syncthreads();
    };
    int t = 0;
    for (; t + 1 < nFull; ++t) step(t, std::true_type{});
    if (t + 1 < nk) step(t++, std::false_type{});   // the one partial slice at the end of K
    runSlice(t, false);

    const long long cb = batch * p.sC;
    if constexpr (SWAP) {
        if constexpr (StagedStore<Cfg>::USED) {
            if (p.staged) {
                __syncthreads();   // every wave is done reading the stages
                storeStaged<Cfg, BF16>(p, acc, hsm, cb, m0, n0, wm, wn, li, h, lane, wave, bzPre);
                return;
            }
        }
        // Lane (li, h) holds, for block (fm, fn), C[m][n .. n+3] at
        // m = mBase + li, n = nBase + 8*g + 4*h (registers 4g .. 4g+3).
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm) {
            const int m = m0 + wm * Cfg::WM + fm * 32 + li;
            if (m >= p.M) continue;
            const long long crow = cb + (long long)m * p.ldc;
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = n0 + wn * Cfg::WN + fn * 32 + 8 * g + 4 * h;
                    if (n < p.N)   // N % 4 == 0
                        storeFour<BF16>(p, crow + n, n, acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1],
                                        acc[fm][fn][4 * g + 2], acc[fm][fn][4 * g + 3]);
                }
        }
    } else {
        // Lane (li, h) holds C[m][n] at n = nBase + li,
        // m = mBase + 8*(r/4) + 4*h + (r%4): 32 lanes store one row's 128 bytes.
        if (p.compact) {
            storeCompact<Cfg, Ops::LDS_BYTES>(p, acc, hsm, cb, wm, wn, li, h, tid);
            return;
        }
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int n = n0 + wn * Cfg::WN + fn * 32 + li;
            if (n >= p.N) continue;
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < p.M) storeOne<BF16>(p, cb + (long long)m * p.ldc + n, n, acc[fm][fn][r]);
                }
        }
    }
}

// 256 x 256 x 64 with 8 waves of 64 x 128 (one workgroup per CU, two waves
// per SIMD) for large problems: measured on MI355X it beats 4 waves of
// 128 x 128 (one wave per SIMD cannot hide its own LDS and barrier latency)
// and BK = 32 (twice the barriers). 128 x 128 x 64 (4 waves of 64 x 64, two
// workgroups per CU) and 64 x 64 x 64 (4 waves of 32 x 32) serve problems
// whose large-tile count would leave CUs idle. 192 x 256 x 64 (8 waves of
// 96 x 64) fills more CUs than 256 x 256 when a problem is one round of
// large tiles on part of the chip (12608 x 768: 198 tiles instead of 150);
// its A rows are K-major (192 rows are not a power-of-two run of 16-byte
// chunks for the R-major loader).
#ifndef OMHIP_HALF_L
#define OMHIP_HALF_L 256, 256, 64, 64, 128
#endif
#ifndef OMHIP_HALF_R_RATE
#define OMHIP_HALF_R_RATE 0.95
#endif
using FCfgL = FCfg<OMHIP_HALF_L>;
using FCfgR = FCfg<192, 256, 64, 96, 64>;
using FCfgM = FCfg<128, 128, 64, 64, 64>;
using FCfgS = FCfg<64, 64, 64, 32, 32>;

template <class Cfg, bool BF16, bool TA, bool TB, bool SWAP, bool RAG>
static int launchFast(HalfFastParams prm, int batch) {
    auto kern = gemm_half_fast<Cfg, BF16, TA, TB, SWAP, RAG>;
    constexpr bool stageable = SWAP && StagedStore<Cfg>::USED;
    constexpr size_t lds = stageable ? std::max(HalfOps<Cfg, TA, TB, RAG>::LDS_BYTES, StagedStore<Cfg>::LDS_BYTES)
                                     : HalfOps<Cfg, TA, TB, RAG>::LDS_BYTES;
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    prm.tilesM = (prm.M + Cfg::BM - 1) / Cfg::BM;
    prm.tilesN = (prm.N + Cfg::BN - 1) / Cfg::BN;
    const long long tiles = (long long)prm.tilesM * prm.tilesN;
    prm.batch = batch;
    prm.flat = batch > 1 && tiles * batch * Cfg::NT < (1LL << 31);
    prm.compact = !SWAP && prm.compact && tiles == 1;
    prm.staged = stageable && (prm.outHalf || tiles * batch <= cuCount());
    const dim3 grid = prm.flat ? dim3((unsigned)(tiles * batch)) : dim3((unsigned)tiles, 1, batch);
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// Tile choice from a model of the time per CU. A CU receives n = ceil(tiles /
// CUs) workgroups and runs up to `slots` of them at once (256x256: 1 per CU,
// 128x128: 2, 64x64: 4, by LDS); its time is n x tile area / throughput,
// where the throughput with j of the slots filled is rate x (j/slots)^0.6 (a
// lone workgroup gets more than its share of the CU). Rates 1, 0.75, 0.5
// were fitted to a sweep of all three tiles over the ViT-B/16 GEMMs, the
// batched attention products and square / tall-skinny problems on MI355X,
// where the model picks the fastest tile or one within 4 % of it: e.g.
// 12608 x 2304 x 768 and 4096^3 take 256x256, 2048 x 4096 x 4096 128x128,
// 768 x (197 x 64 x 197), 2048^3 and 1024^3 64x64.
// cost: the model's time per CU of the chosen tile, in elements of C per unit rate
// (a 256x256 tile on a CU of its own = 65536).
static int pickFastTile(int M, int N, int K, int batch, bool transA, double* cost = nullptr) {
    const long long cus = cuCount();
    struct T { int bm, bn, slots; double rate; };
    const T cand[4] = {{256, 256, 1, 1.0}, {128, 128, 2, 0.75}, {64, 64, 4, 0.5}, {192, 256, 1, OMHIP_HALF_R_RATE}};
    // A product of one K slice is bound by its C stores, not its MFMAs: many
    // small workgroups overlap one another's stores (batched Q.K^T 768 x 197
    // x 197 x 64: 64x64 42.3 us, 256x256 with the compact store 46.0 us,
    // 128x128 55.4 us).
    if (K <= 64) return 2;
    int best = 0;
    double bestCost = 0;
    for (int c = 0; c < (transA ? 3 : 4); ++c) {
        const long long tiles = (long long)((M + cand[c].bm - 1) / cand[c].bm) * ((N + cand[c].bn - 1) / cand[c].bn) * batch;
        const long long n = (tiles + cus - 1) / cus;
        const double fill = (double)std::min<long long>(n, cand[c].slots) / cand[c].slots;
        const double cst = (double)n * cand[c].bm * cand[c].bn / (cand[c].rate * std::pow(fill, 0.6));
        if (c == 0 || cst < bestCost) { best = c; bestCost = cst; }
    }
    if (cost) *cost = bestCost;
    return best;
}

// Row split of one large product on 256x256 tiles whose last round is short
// (12608 x 3072 x 768: 600 tiles, 2.34 rounds): the rows of the whole rounds
// run as one launch and the rest as a second launch on the tile the model
// picks for them (128x128, two workgroups per CU), when that model's time for
// the tail plus a launch's worth (0.15 of a tile) beats the partial round of
// 256x256 tiles. Each element is still one tile's whole-K sum. Returns the
// first launch's row count, or 0.
static int planRowSplit(int M, int N, int K, int batch, bool transA) {
    if (batch != 1 || pickFastTile(M, N, K, 1, transA) != 0) return 0;
    const long long U = cuCount();
    const int tm = (M + 255) / 256, tn = (N + 255) / 256;
    const long long rounds = ((long long)tm * tn + U - 1) / U;
    if (rounds < 2) return 0;
    const int headRows = (int)((rounds - 1) * U / tn);
    if (headRows <= 0 || headRows >= tm) return 0;
    const int M1 = headRows * 256;
    double tail = 0;
    pickFastTile(M - M1, N, K, 1, transA, &tail);
    const double head = (double)(((long long)headRows * tn + U - 1) / U);
    return head + tail / 65536.0 + 0.15 < (double)rounds ? M1 : 0;
}

template <bool BF16, bool TA, bool TB, bool SWAP, bool RAG>
static int launchFastT(const HalfFastParams& prm, int batch) {
    switch (pickFastTile(prm.M, prm.N, prm.K, batch, TA)) {
        case 0: return launchFast<FCfgL, BF16, TA, TB, SWAP, RAG>(prm, batch);
        case 1: return launchFast<FCfgM, BF16, TA, TB, SWAP, RAG>(prm, batch);
        case 3:
            if constexpr (!TA) return launchFast<FCfgR, BF16, TA, TB, SWAP, RAG>(prm, batch);
            [[fallthrough]];
        default: return launchFast<FCfgS, BF16, TA, TB, SWAP, RAG>(prm, batch);
    }
}

template <bool BF16, bool TA, bool TB, bool RAG>
static int launchFastC(const HalfFastParams& prm, int batch, bool vecC) {
    return vecC ? launchFastT<BF16, TA, TB, true, RAG>(prm, batch) : launchFastT<BF16, TA, TB, false, RAG>(prm, batch);
}

template <bool BF16, bool TA, bool TB>
static int launchFastR(const HalfFastParams& prm, int batch, bool vecC, bool rag) {
    if constexpr (TA && !TB) {
        return launchFastC<BF16, TA, TB, false>(prm, batch, vecC);   // no K-major operand
    } else {
        return rag ? launchFastC<BF16, TA, TB, true>(prm, batch, vecC) : launchFastC<BF16, TA, TB, false>(prm, batch, vecC);
    }
}

template <bool BF16>
static int dispatchH(bool ta, bool tb, const GemmHalfParams& prm, int batch, bool va, bool vb) {
    // The fast kernel needs every buffer view (a 256-row K-major tile, or all K
    // rows of an R-major operand) below 2^30 bytes and R-major operands in
    // 16-byte chunks; K-major operands whose rows are not 16-byte aligned (odd
    // K or leading dimension, e.g. P of P x V over 197 keys) take the ragged
    // loader.
    const bool ldOk = prm.lda < (1LL << 21) && prm.ldb < (1LL << 21);
    const long long viewA = ta ? (long long)prm.K * prm.lda * 2 : 256LL * prm.lda * 2 + 4;
    const long long viewB = tb ? 256LL * prm.ldb * 2 + 4 : (long long)prm.K * prm.ldb * 2;
    auto even = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 1u) == 0; };
    const bool aOk = ta ? va : (va || even(prm.A));
    const bool bOk = tb ? (vb || even(prm.B)) : vb;
    const bool rag = (!ta && !va) || (tb && !vb);
    if (aOk && bOk && ldOk && viewA < kMaxViewBytes && viewB < kMaxViewBytes) {
        HalfFastParams f{};
        f.A = prm.A; f.B = prm.B; f.C = prm.C; f.M = prm.M; f.N = prm.N; f.K = prm.K;
        f.lda = (int)prm.lda; f.ldb = (int)prm.ldb; f.ldc = prm.ldc; f.sA = prm.sA; f.sB = prm.sB; f.sC = prm.sC;
        f.bias = prm.bias; f.act = prm.act; f.outHalf = prm.outHalf;
        const uintptr_t cAlign = prm.outHalf ? 7u : 15u;
        const bool cAligned = (reinterpret_cast<uintptr_t>(prm.C) & cAlign) == 0;
        const bool vecC = (prm.N % 4 == 0) && (prm.ldc % 4 == 0) && (prm.sC % 4 == 0) && cAligned;
        f.compact = !prm.outHalf && !prm.bias && prm.act == 0 && prm.ldc == prm.N && cAligned;   // + one tile
        if (!ta && !tb) return launchFastR<BF16, false, false>(f, batch, vecC, rag);
        if (!ta && tb) return launchFastR<BF16, false, true>(f, batch, vecC, rag);
        if (ta && !tb) return launchFastR<BF16, true, false>(f, batch, vecC, rag);
        return launchFastR<BF16, true, true>(f, batch, vecC, rag);
    }
    if (!ta && !tb) return launchGenericC<BF16, false, false>(prm, batch, va, vb);
    if (!ta && tb) return launchGenericC<BF16, false, true>(prm, batch, va, vb);
    if (ta && !tb) return launchGenericC<BF16, true, false>(prm, batch, va, vb);
    return launchGenericC<BF16, true, true>(prm, batch, va, vb);
}

int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC);
int headScoresHalf(bool bf16, int batch, int M, int N, int K, const uint16_t* A, long long lda, long long sA,
                   const uint16_t* B, long long ldb, long long sB, float* C, long long ldc, long long sC);
int headContextHalf(bool bf16, int batch, int M, int N, int K, const uint16_t* A, long long lda, long long sA,
                    const uint16_t* B, long long ldb, long long sB, float* C, long long ldc, long long sC);

// C = act(op(A) op(B) + bias), fp32 or (outHalf) the input half type.
static int gemmHalf(const char* name, int dtype, bool ta, bool tb, int batch, int M, int N, int K,
                    const uint16_t* A, long long lda, long long sA, const uint16_t* B, long long ldb, long long sB,
                    void* C, long long ldc, long long sC, const float* bias = nullptr, int act = 0,
                    bool outHalf = false) {
    clearError();
    if (batch <= 0 || M <= 0 || N <= 0) return 0;
    if (!C) return fail("%s: null output", name);
    if (batch > 65535) return fail("%s: batch %d exceeds 65535", name, batch);
    if (dtype != 0 && dtype != 1) return fail("%s: dtype must be 0 (fp16) or 1 (bf16)", name);
    if (act != 0 && act != 1) return fail("%s: activation must be 0 (none) or 1 (ReLU)", name);
    const bool empty = !A || !B || K <= 0;   // a product with no terms: act(0 + bias)
    if (empty && !bias && !outHalf) return zeroOutput(static_cast<float*>(C), batch, M, N, ldc, sC);
    GemmHalfParams prm{};
    prm.A = empty ? nullptr : A; prm.B = empty ? nullptr : B; prm.C = C; prm.M = M; prm.N = N;
    prm.K = empty ? 0 : K;
    prm.lda = lda; prm.ldb = ldb; prm.ldc = ldc; prm.sA = sA; prm.sB = sB; prm.sC = sC;
    prm.bias = bias; prm.act = act; prm.outHalf = outHalf ? 1 : 0;
    if (empty) {   // the generic kernel's loads are all masked off when K is 0
        return dtype == 1 ? launchGenericC<true, false, false>(prm, batch, false, false)
                          : launchGenericC<false, false, false>(prm, batch, false, false);
    }
    if (!ta && tb && !outHalf && !bias && act == 0) {   // many small A . B^T: the attention scores
        const int rc = headScoresHalf(dtype == 1, batch, M, N, K, A, lda, sA, B, ldb, sB, static_cast<float*>(C), ldc,
                                      sC);
        if (rc <= 0) return rc;
    }
    if (!ta && !tb && !outHalf && !bias && act == 0) {   // many small A . B with 64 columns: the attention context
        const int rc = headContextHalf(dtype == 1, batch, M, N, K, A, lda, sA, B, ldb, sB, static_cast<float*>(C), ldc,
                                       sC);
        if (rc <= 0) return rc;
    }
    if (const int M1 = planRowSplit(M, N, K, batch, ta)) {
        const size_t es = outHalf ? 2 : 4;
        if (gemmHalf(name, dtype, ta, tb, 1, M1, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, bias, act, outHalf))
            return -1;
        return gemmHalf(name, dtype, ta, tb, 1, M - M1, N, K, A + (ta ? (long long)M1 : (long long)M1 * lda), lda, sA,
                        B, ldb, sB, static_cast<char*>(C) + (size_t)M1 * (size_t)ldc * es, ldc, sC, bias, act,
                        outHalf);
    }
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
int omHipLinearHalf(int nDtype, const uint16_t* pInput, const uint16_t* pWeight, int bTransW, const float* pBias,
                    int nAct, void* pOutput, int nOutHalf, int nM, int nK, int nN) {
    return gemmHalf("omHipLinearHalf", nDtype, false, bTransW != 0, 1, nM, nN, nK, pInput, nK, 0, pWeight,
                    bTransW ? nK : nN, 0, pOutput, nN, 0, pBias, nAct, nOutHalf != 0);
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
