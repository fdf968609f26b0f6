// gemm_f32.hpp — host-side interface of the fp32 MFMA GEMM shared by the GEMM
// and conv entry points.
#pragma once

namespace omhip {

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
};

// C[b] = op(A[b]) * op(B[b]); ta: A stored [K,M]; tb: B stored [N,K].
// Enqueues on the library stream; returns 0 or -1 (message via fail()).
int gemmF32(bool ta, bool tb, int batch, int M, int N, int K,
            const float* A, long long lda, long long sA,
            const float* B, long long ldb, long long sB,
            float* C, long long ldc, long long sC);

// C (+)= sum over b of op(A[b]) * op(B[b]) (a batch-reduce GEMM: the batch
// is one more reduction axis). Partial products go to the library workspace
// and are summed in batch order onto 0 (or onto C's current value when
// accumulate is set), so the result is deterministic. Fails when the partials
// (batch x M x N floats) exceed 256 MiB: callers chunk the batch.
int gemmF32BatchReduce(bool ta, bool tb, int batch, int M, int N, int K,
                       const float* A, long long lda, long long sA,
                       const float* B, long long ldb, long long sB,
                       float* C, long long ldc, bool accumulate);

// Largest partial-product buffer gemmF32BatchReduce accepts, in bytes.
constexpr size_t kBatchReduceMaxBytes = (size_t)256 << 20;

// Zeroes C (batch x M x N, row stride ldc, batch stride sC) on the stream.
int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC);

}  // namespace omhip
