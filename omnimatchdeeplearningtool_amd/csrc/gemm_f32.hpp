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
