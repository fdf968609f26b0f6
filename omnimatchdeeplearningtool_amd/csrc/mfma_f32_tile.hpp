// mfma_f32_tile.hpp — fp32 MFMA block-tile mainloop for gfx950 (CDNA4).
//
// One workgroup computes a BM x BN tile of C = A * B with K walked in BK
// slices. A and B slices are staged global -> VGPR -> LDS with two LDS buffers
// (one barrier per slice: while the MFMAs read slice t from buffer t&1, the
// loads of slice t+1 are in flight and land in buffer (t+1)&1).
//
// Every wave owns a WM x WN sub-tile built from 32x32 v_mfma_f32_32x32x2_f32
// blocks (16 accumulators per lane per block). The MFMA consumes per lane
//   A operand: A[i = lane%32][k],  B operand: B[k][j = lane%32]
// and the two 32-lane halves (h = lane/32) supply two different k. Within a
// slice the half h walks k = h*BK/2 + s for s = 0..BK/2-1, i.e. each half
// reduces one contiguous half of the slice; the sum over k is order-free, so
// this permutation only changes rounding order, and it lets an operand whose
// K is contiguous be read from LDS 4 k at a time (ds_read_b128).
//
// Operand storage in LDS is chosen by the operand's layout in HBM:
//   KMAJOR: element (r,k) at P[r*ld + k]   -> LDS [R][BK+4]   (b128 fragment reads)
//   RMAJOR: element (r,k) at P[k*ld + r]   -> LDS [BK][R+4]   (b32 fragment reads)
// where r is the M index for A and the N index for B.
//
// Accumulator layout of a 32x32 block (lane l, register i):
//   row = 8*(i/4) + 4*(l/32) + (i%4),  col = l%32.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace omhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
    static constexpr int NWAVES = WAVES_M * WAVES_N;
    static constexpr int NT = NWAVES * 64;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static constexpr int KH = BK / 2;   // k per lane half per slice
    static_assert(BM % WM == 0 && BN % WN == 0, "wave tiling");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "32x32 MFMA blocks");
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");
};

// LDS footprint (floats) of one buffer of an operand with R rows.
template <bool KMAJOR, int R, int BK>
struct LdsShape {
    static constexpr int LD = KMAJOR ? (BK + 4) : (R + 4);
    static constexpr int SIZE = KMAJOR ? R * (BK + 4) : BK * (R + 4);
};

// ---------------------------------------------------------------------------
// Dense operand loader: element (r,k) of a row-major matrix, KMAJOR or RMAJOR.
// VEC loads 4 consecutive floats along the contiguous axis; the host enables it
// only when that axis length, the leading dimension and the base are multiples
// of 4 floats, so a vector is either fully inside the matrix or fully outside.
// ---------------------------------------------------------------------------
template <bool KMAJOR, bool VEC, int R, int BK, int NT>
struct DenseLoader {
    static constexpr int ELEMS = R * BK;
    static constexpr int PER_T = VEC ? ELEMS / 4 / NT : ELEMS / NT;
    static_assert(ELEMS % (NT * (VEC ? 4 : 1)) == 0, "tile must split evenly over threads");
    using Shape = LdsShape<KMAJOR, R, BK>;

    const float* p;   // operand base (this batch)
    long long ld;
    int rows;         // valid extent along r
    int K;
    int r0;           // tile origin along r
    f32x4 v4[VEC ? PER_T : 1];
    float v1[VEC ? 1 : PER_T];

    __device__ void load(int k0, int tid) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT;
                int r, k;
                if constexpr (KMAJOR) { r = e / (BK / 4); k = (e % (BK / 4)) * 4; }
                else { k = e / (R / 4); r = (e % (R / 4)) * 4; }
                const int gr = r0 + r, gk = k0 + k;
                f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (gr < rows && gk < K) {
                    const float* src = KMAJOR ? p + (long long)gr * ld + gk : p + (long long)gk * ld + gr;
                    v = *reinterpret_cast<const f32x4*>(src);
                }
                v4[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT;
                int r, k;
                if constexpr (KMAJOR) { r = e / BK; k = e % BK; }
                else { k = e / R; r = e % R; }
                const int gr = r0 + r, gk = k0 + k;
                float v = 0.f;
                if (gr < rows && gk < K)
                    v = KMAJOR ? p[(long long)gr * ld + gk] : p[(long long)gk * ld + gr];
                v1[i] = v;
            }
        }
    }

    __device__ void store(float* s, int tid) const {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT;
                int r, k;
                if constexpr (KMAJOR) { r = e / (BK / 4); k = (e % (BK / 4)) * 4; }
                else { k = e / (R / 4); r = (e % (R / 4)) * 4; }
                float* dst = KMAJOR ? s + r * Shape::LD + k : s + k * Shape::LD + r;
                *reinterpret_cast<f32x4*>(dst) = v4[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT;
                int r, k;
                if constexpr (KMAJOR) { r = e / BK; k = e % BK; }
                else { k = e / R; r = e % R; }
                s[KMAJOR ? r * Shape::LD + k : k * Shape::LD + r] = v1[i];
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Fragment reads + MFMA over one LDS slice.
// ---------------------------------------------------------------------------
template <class Cfg, bool A_KMAJOR, bool B_KMAJOR>
__device__ __forceinline__ void mma_slice(const float* __restrict__ sA, const float* __restrict__ sB,
                                          f32x16 (&acc)[Cfg::FM][Cfg::FN],
                                          int wm, int wn, int lane) {
    using SA = LdsShape<A_KMAJOR, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<B_KMAJOR, Cfg::BN, Cfg::BK>;
    const int li = lane & 31;
    const int h = lane >> 5;
    const int kb = h * Cfg::KH;
#pragma unroll
    for (int u = 0; u < Cfg::KH / 4; ++u) {
        float a[Cfg::FM][4], b[Cfg::FN][4];
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm) {
            const int row = wm * Cfg::WM + fm * 32 + li;
            if constexpr (A_KMAJOR) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(sA + row * SA::LD + kb + 4 * u);
                a[fm][0] = v[0]; a[fm][1] = v[1]; a[fm][2] = v[2]; a[fm][3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) a[fm][s] = sA[(kb + 4 * u + s) * SA::LD + row];
            }
        }
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = wn * Cfg::WN + fn * 32 + li;
            if constexpr (B_KMAJOR) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(sB + col * SB::LD + kb + 4 * u);
                b[fn][0] = v[0]; b[fn][1] = v[1]; b[fn][2] = v[2]; b[fn][3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) b[fn][s] = sB[(kb + 4 * u + s) * SB::LD + col];
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn)
                    acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[fm][s], b[fn][s], acc[fm][fn], 0, 0, 0);
    }
}

// The MFMAs of one LDS slice with `mid` run between its first and second
// halves: every fragment of the slice is read first, then the first half of
// the k steps, mid() (the next slice's LDS stores), the second half. The
// schedule barriers keep that order, so the stores' LDS traffic overlaps the
// second half's MFMAs instead of sitting between the last MFMA and the block
// barrier.
template <class Cfg, bool A_KMAJOR, bool B_KMAJOR, class Mid>
__device__ __forceinline__ void mma_slice_split(const float* __restrict__ sA, const float* __restrict__ sB,
                                                f32x16 (&acc)[Cfg::FM][Cfg::FN], int wm, int wn, int lane,
                                                Mid&& mid) {
    using SA = LdsShape<A_KMAJOR, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<B_KMAJOR, Cfg::BN, Cfg::BK>;
    constexpr int U = Cfg::KH / 4;
    static_assert(U % 2 == 0, "two halves of k steps");
    const int li = lane & 31;
    const int h = lane >> 5;
    const int kb = h * Cfg::KH;
    float a[U][Cfg::FM][4], b[U][Cfg::FN][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm) {
            const int row = wm * Cfg::WM + fm * 32 + li;
            if constexpr (A_KMAJOR) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(sA + row * SA::LD + kb + 4 * u);
                a[u][fm][0] = v[0]; a[u][fm][1] = v[1]; a[u][fm][2] = v[2]; a[u][fm][3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) a[u][fm][s] = sA[(kb + 4 * u + s) * SA::LD + row];
            }
        }
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = wn * Cfg::WN + fn * 32 + li;
            if constexpr (B_KMAJOR) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(sB + col * SB::LD + kb + 4 * u);
                b[u][fn][0] = v[0]; b[u][fn][1] = v[1]; b[u][fn][2] = v[2]; b[u][fn][3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) b[u][fn][s] = sB[(kb + 4 * u + s) * SB::LD + col];
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U / 2; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn)
                    acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u][fm][s], b[u][fn][s], acc[fm][fn], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    mid();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = U / 2; u < U; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn)
                    acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u][fm][s], b[u][fn][s], acc[fm][fn], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------
// Block-tile -> (tm, tn) mapping. Workgroups are dispatched round-robin over
// the 8 XCDs (each with its own L2), so consecutive block ids land on
// different XCDs. The remap gives each XCD a contiguous range of logical tile
// ids, and the grouped ordering turns a contiguous range into a compact 2-D
// patch (GROUP_M tile rows wide), so tiles sharing A rows / B columns share an L2.
// ---------------------------------------------------------------------------
// Logical id of block `bid` among `total` blocks: XCD x (= bid % 8) gets the
// contiguous logical range x*q .. (spread evenly when total % 8 != 0).
__device__ __forceinline__ int xcd_remap(int bid, int total) {
    constexpr int XCDS = 8;
    if (total < XCDS) return bid;
    const int q = total / XCDS, rem = total % XCDS;
    const int xcd = bid % XCDS, idx = bid / XCDS;
    return (xcd < rem) ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
}

// Logical tile t -> (tm, tn) in the grouped ordering (groupM tile rows wide).
__host__ __device__ __forceinline__ void grouped_tile(int t, int tilesM, int tilesN, int groupM, int& tm, int& tn) {
    const int perGroup = groupM * tilesN;
    const int g = t / perGroup;
    const int firstM = g * groupM;
    const int gsz = (tilesM - firstM) < groupM ? (tilesM - firstM) : groupM;
    const int inG = t - g * perGroup;
    tm = firstM + inG % gsz;
    tn = inG / gsz;
}

__device__ __forceinline__ void tile_coords(int bid, int total, int tilesM, int tilesN, int groupM,
                                            int& tm, int& tn) {
    grouped_tile(xcd_remap(bid, total), tilesM, tilesN, groupM, tm, tn);
}

}  // namespace omhip
