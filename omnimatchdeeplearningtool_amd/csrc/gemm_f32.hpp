// gemm_f32.hpp — host-side interface of the fp32 MFMA GEMM shared by the GEMM
// and conv entry points.
#pragma once

#include <cstddef>

namespace omhip {

struct GemmPlan {
    int cfg;      // 0: 256x256, 1: 128x128, 2: 64x64
    int splits;   // K splits (1: none)
};

// Tile and split-K choice on a device of `cus` compute units: the largest tile
// that gives every CU a workgroup. When even 64x64 tiles give fewer than two
// workgroups per CU and K is long (few rows or columns: 128 x 4096 x 4096,
// weight gradients), K is split over the 64x64 tile: the smallest power of two
// (at most 64) that gives every CU two workgroups while each split keeps >= 256
// of K. The partials cost one fp32 write and read of C per split. Measured on
// MI355X (TFLOP/s, against splitting the 128x128 tile until every CU had one
// workgroup): 128 x 4096 x 4096 86 (76), 64 x 4096 x 4096 69 (56),
// 128 x 1024 x 4096 47 (29), 512 x 1024 x 2048 72 (56), 256 x 4096 x 4096 96
// (75). With 512 <= K < 1024 only grids of at most CUs / 4 tiles split (pieces
// of >= 128 of K: 128 x 256 x 784, the MLP's first layer, 18.9 -> 11.5 us;
// 256 x 512 x 768 18.9 -> 12.8; 512^3 14.2 -> 11.7); shorter K runs faster
// unsplit. A split plan stops doubling once the grid holds 2 x CUs
// workgroups, so its partials cover fewer than 4 x CUs tiles of 64 x 64
// floats (16 MiB on 256 CUs). Host-only, so a CPU test checks that bound.
inline GemmPlan planGemmFor(int M, int N, int K, int batch, bool wsOk, long long cus) {
    auto tiles = [&](int bm, int bn) { return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
    if (tiles(256, 256) >= cus) return {0, 1};
    if (tiles(128, 128) >= cus) return {1, 1};
    const long long t = tiles(64, 64);
    if (t >= 2 * cus || !wsOk || K < 512 || (K < 1024 && t * 4 > cus)) return {2, 1};
    if (K < 1024) {   // very few tiles (at most CUs / 4): splits of >= 128 of K
        int s = 1;
        while (s < 64 && t * s < 2 * cus && K / (2 * s) >= 128) s *= 2;
        return {2, s};
    }
    // with one tile per CU already, a split must keep >= 1024 of K (1024^3
    // ran 79 TFLOP/s unsplit, 70 split in two)
    const int minK = t >= cus ? 1024 : 256;
    int s = 1;
    while (s < 64 && t * s < 2 * cus && K / (2 * s) >= minK) s *= 2;
    return {2, s};
}

// The K pieces a plan's launch actually uses: K in chunks of a whole number of
// 16-deep slices (the last chunk may be shorter), so fewer than plan.splits
// pieces when K is short.
inline int splitPieces(int K, int splits, int* kChunk = nullptr) {
    const int bk = 16;
    const int chunk = ((K + splits - 1) / splits + bk - 1) / bk * bk;
    if (kChunk) *kChunk = chunk;
    return (K + chunk - 1) / chunk;
}

// Bytes of the fixed device array behind omHipGemmStridedBatchedNoAlloc: twice
// the bound above for a 256-CU device. Its last kNoAllocCounterBytes hold the
// tiles' split-K arrival counters (zero at load, and every launch leaves them
// zero); the partials use the rest.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr size_t kNoAllocCounterBytes = (size_t)64 << 10;

struct GemmF32Params {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    long long lda, ldb, ldc;
    long long sA, sB, sC;   // per-batch element offsets (0 shares the operand)
    int tilesM, tilesN;
    int kChunk;             // split-K: split s covers k in [s*kChunk, min(K, (s+1)*kChunk))
    float* ws;              // split-K partials [split][batch][M][N] (null: write C directly)
    unsigned* ctr;          // split-K: per (batch, tile) arrival counters, zero at rest
    int splits;             // split-K: pieces of K (the last arrival of a tile sums them)
    const float* bias;      // [N] added to every row of C, or null
    int act;                // 0 identity, 1 ReLU (after the bias)
    const float* gate;      // Linear backward: C kept where gate > 0 (row stride ldg)
    long long ldg;
    float* colSum;          // Linear backward: B's column sums (the bias gradient)
};

// C[b] = op(A[b]) * op(B[b]); ta: A stored [K,M]; tb: B stored [N,K].
// Enqueues on the library stream; returns 0 or -1 (message via fail()).
// bias ([N], nullable) and act (0 identity, 1 ReLU) are applied to every
// element of C as it is written: C = act(op(A) * op(B) + bias).
int gemmF32(bool ta, bool tb, int batch, int M, int N, int K,
            const float* A, long long lda, long long sA,
            const float* B, long long ldb, long long sB,
            float* C, long long ldc, long long sC,
            const float* bias = nullptr, int act = 0);

// Zeroes C (batch x M x N, row stride ldc, batch stride sC) on the stream.
int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC);

}  // namespace omhip
