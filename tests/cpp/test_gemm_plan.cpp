// CPU test of the fp32 GEMM's tile / split-K plan (omhip::planGemmFor): the
// split-K partial sums of every plan fit the no-allocation entry's fixed array
// (kNoAllocScratchBytes less its arrival counters), the tiles' counters fit
// theirs (kNoAllocCounterBytes), and the partials stay below the stated bound of 4 x CUs tiles of
// 64 x 64 floats, over the GEMM sweep, the MLP and ResNet weight-gradient
// shapes, the shapes that reach the bound, and a dense grid of small M / N.
// Exit status 0 = all checks passed.
#include <cstdio>
#include <vector>

#include "../../omnimatchdeeplearningtool_amd/csrc/gemm_f32.hpp"

static int g_fail = 0;
static long long g_maxBytes = 0;

static void check(int M, int N, int K, int batch, long long cus) {
    // the wsOk rule of gemmF32: 64 splits of the batch's C within 256 MiB
    const bool wsOk = (long long)64 * batch * M * N * 4 <= (256LL << 20);
    const omhip::GemmPlan p = omhip::planGemmFor(M, N, K, batch, wsOk, cus);
    if (p.splits <= 1) return;
    const int pieces = omhip::splitPieces(K, p.splits);
    const long long tiles = (long long)((M + 63) / 64) * ((N + 63) / 64) * batch;
    const long long bytes = (long long)pieces * tiles * 64 * 64 * 4;   // partials in whole 64 x 64 tiles
    if (g_maxBytes < bytes && cus == 256) g_maxBytes = bytes;
    if (p.cfg != 2 || bytes > (long long)(omhip::kNoAllocScratchBytes - omhip::kNoAllocCounterBytes) ||
        tiles * 4 > (long long)omhip::kNoAllocCounterBytes || tiles * p.splits >= 4 * cus ||
        bytes > 4 * cus * 64LL * 64 * 4) {
        std::printf("FAIL M=%d N=%d K=%d batch=%d cus=%lld: cfg %d splits %d (%d pieces) %lld bytes\n", M, N, K, batch,
                    cus, p.cfg, p.splits, pieces, bytes);
        ++g_fail;
    }
}

int main() {
    const int sq[] = {512, 1024, 2048, 4096, 8192};
    for (int s : sq) check(s, s, s, 1, 256);
    check(128, 4096, 4096, 1, 256);
    check(8192, 256, 2048, 1, 256);
    check(448, 4672, 2048, 1, 256);   // 511 tiles split in two: the largest plan on 256 CUs
    check(128, 256, 784, 1, 256);     // MLP layers and their gradients
    check(784, 256, 128, 1, 256);
    check(256, 128, 128, 1, 256);
    check(64, 4096, 4096, 1, 256);
    // a dense grid of small outputs with long K, single and batched, on 256 and 304 CUs
    for (long long cus : {256LL, 304LL, 80LL})
        for (int b : {1, 2, 3, 8})
            for (int M = 16; M <= 1024; M += 48)
                for (int N = 16; N <= 5000; N += 112)
                    for (int K : {512, 784, 1000, 1024, 2048, 4096, 16384, 65536}) check(M, N, K, b, cus);
    std::printf("largest split plan on 256 CUs: %lld bytes\n", g_maxBytes);
    std::printf(g_fail ? "FAILED %d\n" : "ALL PASSED\n", g_fail);
    return g_fail ? 1 : 0;
}
