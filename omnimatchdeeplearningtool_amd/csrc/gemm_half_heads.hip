// gemm_half_heads.hip — batched fp16 / bf16 products of many small matrices,
// one workgroup per batch entry: the attention score products Q . K^T of a
// transformer's heads (768 heads of 197 x 64 at ViT-B/16 batch 64; the
// reference forms them with tensorBatchedMatmul over the split heads,
// om.engine.vit.ixx:193-205, cpu_backend.ixx:1520-1532).
//
// C[b] = A[b] . B[b]^T, A [M][K] and B [N][K] half (K = 64, rows 16-byte
// aligned), C [M][ldc] fp32 with N <= 256. The general tiled kernel runs such
// a product as 16 workgroups of 64 x 64 per head, each paying its own
// prologue and epilogue for four MFMAs; here one workgroup holds the head's
// whole B (at most 256 rows x 128 bytes) in LDS and its four waves walk the
// head's 16-row blocks of A:
//  * B goes straight from memory into LDS (buffer_load ... lds), 8 rows of
//    64 halves per instruction, chunk c of row r in slot c ^ ((r >> 1) & 7)
//    (the 16 lanes of a fragment read then hit 16 distinct 16-byte bank
//    groups); rows past N read as zeros.
//  * A fragments (8 consecutive k of one row per lane) are loaded straight
//    from memory into registers, the next block's while this one computes.
//  * Each 16 x 16 output tile is C^T = B . A^T on v_mfma_f32_16x16x32 (B from
//    LDS as the first operand), so lane (l16, g4) holds C[row r0 + l16][col
//    16t + 4g4 .. +3]: four consecutive floats, stored with one 16-byte store
//    (columns past N in the last tile are stored one at a time).
// Within each MFMA the four 16-lane groups supply k = 8g4 .. 8g4+7 of the
// 32-deep step; the sum over k is order-free, so only rounding order differs
// from the tiled kernel.
//
// The context products P . V (C[b] = A[b] . B[b], A [M][K] half with rows at
// any half offset — the 197-key probabilities — B [K][64] half, K <= 256) run
// the same way with V (B) in LDS:
//  * C^T = V^T . P^T: the V^T fragment of d tile dt (16 d) and keys 32ks +
//    8g4 .. +7 comes from V's natural [key][d] rows through two
//    ds_read_b64_tr_b16 (lane i of a 16-lane group receives element
//    E[4j + i/4][i%4] of what the group addressed: addressing rows 8g4 + i/4
//    and 8g4 + 4 + i/4 at columns 16dt + 4(i%4) gives lane i the column
//    16dt + i of 8 consecutive keys). V row r (128 bytes) keeps its 16-byte
//    chunk c in slot c ^ 2((r >> 3) & 3) ^ 4((r >> 1) & 1): within a half-wave
//    the two 16-lane groups (8 rows apart) and the row pairs of one group
//    (2 rows apart) take different slots, so its 32 8-byte pieces cover every
//    bank evenly (the two-term form left the row pairs on the same slots:
//    half of the LDS cycles were bank conflicts).
//  * the P fragment (8 consecutive keys of one row per lane) is fetched as the
//    16 bytes from the dword boundary below it plus the next dword and
//    funnel-shifted into place; halves past K are zeroed on the last step
//    (the next row's data lies there).
//  * lane (l16, g4) ends with C[row r0 + l16][16dt + 4g4 .. +3] and stores
//    it with one 16-byte store.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <cstdint>

namespace omhip {

namespace {

typedef _Float16 f16x8s __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8s __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));
typedef float f32x4s __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2s __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* LdsPtrS;

constexpr uint32_t kOOBS = 0x40000000u;   // a byte offset past every view (views are below 2^30 bytes)
constexpr int kHeadK = 64;
constexpr int kHeadMaxN = 256;
constexpr int kHeadNT = 256;

struct HeadScoreArgs {
    const uint16_t* A;
    const uint16_t* B;
    float* C;
    int M, N;
    int lda, ldb;            // halves, multiples of 8
    long long ldc;           // floats
    long long sA, sB, sC;    // batch strides (elements)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrcS(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

template <bool BF16>
__device__ __forceinline__ f32x4s mfmaS(const u32x4s& a, const u32x4s& b, const f32x4s& c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8s, a), __builtin_bit_cast(bf16x8s, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8s, a), __builtin_bit_cast(f16x8s, b), c,
                                                      0, 0, 0);
}

__device__ __forceinline__ int slotS(int r, int c) { return c ^ ((r >> 1) & 7); }

template <bool BF16>
__global__ __launch_bounds__(kHeadNT) void head_scores_kernel(HeadScoreArgs p) {
    __shared__ __attribute__((aligned(16))) uint16_t sB[kHeadMaxN * kHeadK];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;
    const long long b = blockIdx.x;
    const int M = p.M, N = p.N;
    const int nTiles = (N + 15) >> 4;

    // B rows into LDS: instruction i writes rows 8i .. 8i+7 (1 KB, lane L at +16L).
    {
        const auto rb = rsrcS(p.B + b * p.sB, (uint32_t)((N - 1) * p.ldb + kHeadK) * 2u);
        const int rsub = lane >> 3, slot = lane & 7;
        for (int i = wave; i < 2 * nTiles; i += kHeadNT / 64) {
            const int r = 8 * i + rsub;
            const uint32_t vo = r < N ? (uint32_t)(r * p.ldb + 8 * slotS(r, slot)) * 2u : kOOBS;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (LdsPtrS)(sB + i * 8 * kHeadK), 16, vo, 0, 0, 0);
        }
    }

    // A fragments of row block rb: lane (l16, g4) holds A[16 rb + l16][32 ks + 8 g4 .. +7].
    const auto ra = rsrcS(p.A + b * p.sA, (uint32_t)((M - 1) * p.lda + kHeadK) * 2u);
    auto loadA = [&](int rb, u32x4s (&af)[2]) {
        const int r = 16 * rb + l16;
        const uint32_t vo = r < M ? (uint32_t)(r * p.lda + 8 * g4) * 2u : kOOBS;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            af[ks] = __builtin_bit_cast(u32x4s, __builtin_amdgcn_raw_buffer_load_b128(ra, vo, (uint32_t)ks * 64u, 0));
    };
    const int nBlocks = (M + 15) >> 4;
    u32x4s af[2], an[2] = {};
    if (wave < nBlocks) loadA(wave, af);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's LDS DMA (and first A fragments) landed
    __syncthreads();

    const auto rc = rsrcS(p.C + b * p.sC, (uint32_t)((long long)(M - 1) * p.ldc + N) * 4u);
    // per-lane LDS offsets (halves) of the B fragment of tile 0, steps 0 and 1
    uint32_t kOff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) kOff[ks] = (uint32_t)(l16 * kHeadK + 8 * slotS(l16, 4 * ks + g4));
    const int fullTiles = N >> 4;   // tiles whose 16 columns all lie inside N
    auto tile = [&](int t) {
        f32x4s acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // tile t's rows are 16t + l16: whole 16-row steps keep the slot swizzle
            const u32x4s kf = *reinterpret_cast<const u32x4s*>(sB + kOff[ks] + t * 16 * kHeadK);
            acc = mfmaS<BF16>(kf, af[ks], acc);
        }
        return acc;
    };
    for (int rb = wave; rb < nBlocks; rb += kHeadNT / 64) {
        if (rb + kHeadNT / 64 < nBlocks) loadA(rb + kHeadNT / 64, an);
        const int r = 16 * rb + l16;
        // rows past M store nothing (their offset lies outside the view)
        const uint32_t rowOff = r < M ? (uint32_t)((long long)r * p.ldc) * 4u + 16u * g4 : kOOBS;
        int t = 0;
        for (; t + 4 <= fullTiles; t += 4) {
            f32x4s acc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u] = tile(t + u);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4s, acc[u]), rc, rowOff,
                                                       (uint32_t)(t + u) * 64u, 0);
        }
        for (; t < fullTiles; ++t)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4s, tile(t)), rc, rowOff, (uint32_t)t * 64u,
                                                   0);
        if (t < nTiles) {   // the last tile, cut by N: one element at a time
            const f32x4s acc = tile(t);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool in = 16 * t + 4 * g4 + i < N;
                const float v = acc[i];   // a named scalar: bit_cast of a vector element would read element 0
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rc,
                                                      in ? rowOff + 4u * i : kOOBS, (uint32_t)t * 64u, 0);
            }
        }
        af[0] = an[0];
        af[1] = an[1];
    }
}

struct HeadContextArgs {
    const uint16_t* A;       // P: [M][lda], rows at any half offset
    const uint16_t* B;       // V: [K][ldb], 16-byte aligned rows of 64 halves
    float* C;                // [M][ldc], ldc % 4 == 0, 16-byte aligned
    int M, K;
    int lda, ldb;
    long long ldc;
    long long sA, sB, sC;
};

constexpr int kCtxN = 64;        // output columns (the head dimension)
constexpr int kCtxMaxK = 256;    // keys

__device__ __forceinline__ int vSlotS(int r, int c) { return c ^ (2 * ((r >> 3) & 3)) ^ (4 * ((r >> 1) & 1)); }

template <bool BF16>
__global__ __launch_bounds__(kHeadNT) void head_context_kernel(HeadContextArgs p) {
    __shared__ __attribute__((aligned(16))) uint16_t sV[kCtxMaxK * kCtxN];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;
    const long long b = blockIdx.x;
    const int M = p.M, K = p.K;
    const int nSteps = (K + 31) >> 5;

    // V rows into LDS (rows past K read as zeros): instruction i writes rows 8i .. 8i+7.
    {
        const auto rb = rsrcS(p.B + b * p.sB, (uint32_t)((K - 1) * p.ldb + kCtxN) * 2u);
        const int rsub = lane >> 3, slot = lane & 7;
        for (int i = wave; i < 4 * nSteps; i += kHeadNT / 64) {
            const int r = 8 * i + rsub;
            const uint32_t vo = r < K ? (uint32_t)(r * p.ldb + 8 * vSlotS(r, slot)) * 2u : kOOBS;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (LdsPtrS)(sV + i * 8 * kCtxN), 16, vo, 0, 0, 0);
        }
    }

    // P fragments of row block rb, step ks: halves 32ks + 8g4 .. +7 of row 16rb + l16. The view
    // starts at the dword holding the batch's first element and ends at the dword holding the last
    // row's K-th element; a fragment is the 16 bytes at the dword boundary below its first half and
    // the next dword, shifted down 16 bits when that half is odd.
    const uint16_t* a0 = p.A + b * p.sA;
    const uint32_t lead = (uint32_t)(reinterpret_cast<uintptr_t>(a0) & 2u) >> 1;
    const uint32_t endH = (uint32_t)(M - 1) * (uint32_t)p.lda + (uint32_t)K + lead;
    const auto ra = rsrcS(a0 - lead, (endH * 2u + 3u) & ~3u);
    auto loadP = [&](int rb, u32x4s (&lo)[kCtxMaxK / 32], uint32_t (&hi)[kCtxMaxK / 32], uint32_t& sh) {
        const int r = 16 * rb + l16;
        const uint32_t h = (uint32_t)r * (uint32_t)p.lda + 8u * g4 + lead;
        const uint32_t vo = r < M ? (h * 2u) & ~3u : kOOBS;
        sh = (h & 1u) * 16u;
#pragma unroll
        for (int ks = 0; ks < kCtxMaxK / 32; ++ks)
            if (ks < nSteps) {
                lo[ks] = __builtin_bit_cast(u32x4s, __builtin_amdgcn_raw_buffer_load_b128(ra, vo, 64u * ks, 0));
                hi[ks] = __builtin_amdgcn_raw_buffer_load_b32(ra, vo + 16u, 64u * ks, 0);
            }
    };
    const int nBlocks = (M + 15) >> 4;
    u32x4s plo[kCtxMaxK / 32], nlo[kCtxMaxK / 32];
    uint32_t phi[kCtxMaxK / 32], nhi[kCtxMaxK / 32], psh = 0, nsh = 0;
    if (wave < nBlocks) loadP(wave, plo, phi, psh);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's LDS DMA (and first P fragments) landed
    __syncthreads();

    // per-lane byte offsets of the two transposing reads of d tile dt at step 0
    uint32_t vOff[4][2];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int r = 8 * g4 + 4 * hh + (l16 >> 2);
            const int c = 2 * dt + ((l16 & 3) >> 1);
            vOff[dt][hh] = 2u * (uint32_t)(r * kCtxN + 8 * vSlotS(r, c) + 4 * (l16 & 1));
        }
    const uint32_t vBase = (uint32_t)(uintptr_t)(LdsPtrS)(sV);
    const auto rc = rsrcS(p.C + b * p.sC, (uint32_t)((long long)(M - 1) * p.ldc + kCtxN) * 4u);
    const int kLast = K - 32 * (nSteps - 1) - 8 * g4;   // halves of this lane's last-step fragment inside K

    for (int rb = wave; rb < nBlocks; rb += kHeadNT / 64) {
        if (rb + kHeadNT / 64 < nBlocks) loadP(rb + kHeadNT / 64, nlo, nhi, nsh);
        f32x4s acc[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4s{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < kCtxMaxK / 32; ++ks) {
            if (ks >= nSteps) break;
            u32x4s pf = {__builtin_amdgcn_alignbit(plo[ks][1], plo[ks][0], psh),
                         __builtin_amdgcn_alignbit(plo[ks][2], plo[ks][1], psh),
                         __builtin_amdgcn_alignbit(plo[ks][3], plo[ks][2], psh),
                         __builtin_amdgcn_alignbit(phi[ks], plo[ks][3], psh)};
            if (ks == nSteps - 1 && kLast < 8) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    pf[j] &= (2 * j < kLast ? 0x0000ffffu : 0u) | (2 * j + 1 < kLast ? 0xffff0000u : 0u);
            }
            u32x4s vf[4];
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                u32x2s lo, up;
                asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                             : "=v"(lo) : "v"(vBase + vOff[dt][0]), "i"(0) : "memory");
                asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                             : "=v"(up) : "v"(vBase + vOff[dt][1]), "i"(0) : "memory");
                vf[dt] = u32x4s{lo[0], lo[1], up[0], up[1]};
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                asm volatile("" : "+v"(vf[dt]));
                acc[dt] = mfmaS<BF16>(vf[dt], pf, acc[dt]);
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) vOff[dt][hh] += 32u * kCtxN * 2u;
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) vOff[dt][hh] -= (uint32_t)nSteps * 32u * kCtxN * 2u;
        const int r = 16 * rb + l16;
        const uint32_t rowOff = r < M ? (uint32_t)((long long)r * p.ldc) * 4u + 16u * g4 : kOOBS;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4s, acc[dt]), rc, rowOff, 64u * dt, 0);
#pragma unroll
        for (int ks = 0; ks < kCtxMaxK / 32; ++ks) {
            plo[ks] = nlo[ks];
            phi[ks] = nhi[ks];
        }
        psh = nsh;
    }
}

template <bool BF16>
int launchHeadContext(const HeadContextArgs& a, int batch) {
    hipLaunchKernelGGL(head_context_kernel<BF16>, dim3(batch), dim3(kHeadNT), 0, stream(), a);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <bool BF16>
int launchHeadScores(const HeadScoreArgs& a, int batch) {
    hipLaunchKernelGGL(head_scores_kernel<BF16>, dim3(batch), dim3(kHeadNT), 0, stream(), a);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // namespace

// Runs C[b] = A[b] . B[b]^T on the per-head kernel when the shape is one it
// takes (K = 64, N <= 256, M <= 1024, at least one entry per CU, 16-byte
// aligned rows, every view below 2^30 bytes) and returns 0, or -1 with the
// error recorded; returns 1, having done nothing, for any other shape.
int headScoresHalf(bool bf16, int batch, int M, int N, int K, const uint16_t* A, long long lda, long long sA,
                   const uint16_t* B, long long ldb, long long sB, float* C, long long ldc, long long sC) {
    auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    if (K != kHeadK || N > kHeadMaxN || M > 1024 || batch < cuCount() || !al16(A) || !al16(B) ||
        (reinterpret_cast<uintptr_t>(C) & 3u) != 0 || lda % 8 || ldb % 8 || sA % 8 || sB % 8 || lda >= (1 << 20) ||
        ldb >= (1 << 20))
        return 1;
    if ((long long)(M - 1) * ldc + N >= (1LL << 28) || (long long)(M - 1) * lda + K >= (1LL << 29) ||
        (long long)(N - 1) * ldb + K >= (1LL << 29))
        return 1;
    HeadScoreArgs a{A, B, C, M, N, (int)lda, (int)ldb, ldc, sA, sB, sC};
    return bf16 ? launchHeadScores<true>(a, batch) : launchHeadScores<false>(a, batch);
}

// Runs C[b] = A[b] . B[b] on the per-head kernel when the shape is one it
// takes (N = 64, K <= 256, M <= 1024, at least one entry per CU, B rows and
// C 16-byte aligned, every view below 2^30 bytes) and returns 0, or -1 with
// the error recorded; returns 1, having done nothing, for any other shape.
int headContextHalf(bool bf16, int batch, int M, int N, int K, const uint16_t* A, long long lda, long long sA,
                    const uint16_t* B, long long ldb, long long sB, float* C, long long ldc, long long sC) {
    auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    if (N != kCtxN || K > kCtxMaxK || M > 1024 || batch < cuCount() || !al16(B) || !al16(C) || ldb % 8 ||
        sB % 8 || ldc % 4 || sC % 4 || lda >= (1 << 20) || ldb >= (1 << 20))
        return 1;
    if ((long long)(M - 1) * ldc + N >= (1LL << 28) || (long long)(M - 1) * lda + K + 2 >= (1LL << 29) ||
        (long long)(K - 1) * ldb + N >= (1LL << 29))
        return 1;
    HeadContextArgs a{A, B, C, M, K, (int)lda, (int)ldb, ldc, sA, sB, sC};
    return bf16 ? launchHeadContext<true>(a, batch) : launchHeadContext<false>(a, batch);
}

}  // namespace omhip
