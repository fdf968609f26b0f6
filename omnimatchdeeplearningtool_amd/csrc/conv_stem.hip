// conv_stem.hip — the RGB stem convolution (3 input channels, 7x7 kernel,
// stride 2, padding 3: the first layer of the reference's ResNet-18 / -50,
// resnet.ixx / resnet50.ixx conv1) on 16x16x4 fp32 MFMA, with bias, BatchNorm
// (inference), residual and ReLU fused into the output write as in conv.hip.
//
// The general implicit-GEMM kernel gathers each im2col element with a buffer
// load plus two VALU operations (tap-mask bit, out-of-range shift); with 49
// taps per channel that is five VALU instructions per MFMA here, and gfx950
// issues them in the matrix cores' time. This kernel has none in its loop:
//
//  * A block computes output rows of one image for 64 output channels. Its
//    input window — 3 channels x the input rows x the whole row width, with
//    zero columns for the left / right padding and zero rows above / below the
//    image — is copied into LDS once, [ci][row][kStemRS floats], input column
//    x at LDS column x + 4.
//  * Each wave owns 16 output channels and all 7 16-pixel subtiles of the row
//    (seven independent accumulators). For v_mfma_f32_16x16x4_f32, lane l
//    supplies A[i = l%16][k = l/16] and B[k = l/16][j = l%16], so the four
//    k values of one instruction come from the lane's group g = l/16. The 147
//    taps (ci, kh, kw) are covered by 37 "quads": a base tap p plus one of five
//    shapes {G(0), .., G(3)}, lane group g taking tap p + G(g). The LDS offset
//    of tap t for output pixel j is 2j + 1 + off(t) with off linear in
//    (ci, kh, kw), so a lane's B address for quad q and subtile s is
//        [2j + 1 + off(G_shape(g))]  (a per-lane register per shape)
//      + off(p_q) + 32s              (a compile-time constant)
//    and every B operand is a ds_read_b32 with an immediate offset. The
//    weights work the same way in the flat tap index (ci*49 + kh*7 + kw): five
//    per-lane row bases, 37 buffer loads with immediate offsets, held in 37
//    registers for the whole block.
//  * Quads per channel plane: 7 horizontal 1x4 (kw 0-3 of every row), 3
//    vertical 4x1 (kh 0-3 of kw 4-6), one 2x2 square at (4,4) and one L at
//    (6,4)-(6,6)+(5,6); the tap (4,6) of the three planes forms one more quad
//    with a zero-weight fourth lane group: 37 x 4 = 148 k for 147 taps.
//
//  * A block takes up to 7 consecutive output rows of one image (rows * 2 + 5
//    input rows staged once, the 37 weight registers loaded once) and runs
//    them one after another, each row's stores draining under the next row's
//    MFMAs. The host picks the row count that evens out the rows per CU.
//
// Applies to Cin == 3, 7x7, stride 2, pad 3, W a multiple of 4 up to 224 (so
// Wo <= 112 = 7 subtiles), any H, any Cout and batch; conv.hip dispatches here
// for that geometry and to the general kernel otherwise.
#include "omhip_internal.hpp"
#include "buffer_io.hpp"
#include "mfma_f32_tile.hpp"
#include "conv.hpp"

#include <algorithm>

namespace omhip {

namespace {

constexpr int kStemRS = 232;             // LDS row stride in floats: cols 0-3 zero, x at col x+4, zero tail
constexpr int kStemRows = 7;             // output rows per block at most
constexpr int kStemInRows = 2 * kStemRows + 5;   // input rows they read per channel
constexpr int kStemPS = kStemInRows * kStemRS;   // one input channel's rows
constexpr int kStemLds = 3 * kStemPS;    // floats of input window
constexpr int kStemSub = 7;              // 16-pixel subtiles per output row
constexpr int kStemQuads = 37;
constexpr int kStemNT = 256;             // 4 waves x 16 channels = 64 channels per block

struct Tap {
    int ci, kh, kw;
};

// Lane-group offsets of the five quad shapes: H (1x4), V (4x1), S (2x2),
// L ((0,0) (0,1) (0,2) (-1,2)), C (across the three channels; the fourth
// group repeats the base tap with a zero weight).
constexpr Tap kShape[5][4] = {
    {{0, 0, 0}, {0, 0, 1}, {0, 0, 2}, {0, 0, 3}},
    {{0, 0, 0}, {0, 1, 0}, {0, 2, 0}, {0, 3, 0}},
    {{0, 0, 0}, {0, 0, 1}, {0, 1, 0}, {0, 1, 1}},
    {{0, 0, 0}, {0, 0, 1}, {0, 0, 2}, {0, -1, 2}},
    {{0, 0, 0}, {1, 0, 0}, {2, 0, 0}, {0, 0, 0}},
};
constexpr int kShapeC = 4;

__host__ __device__ constexpr int ldsOff(Tap t) { return t.ci * kStemPS + t.kh * kStemRS + t.kw; }
__host__ __device__ constexpr int tapIdx(Tap t) { return t.ci * 49 + t.kh * 7 + t.kw; }

__host__ __device__ constexpr int quadShape(int q) {
    if (q == 36) return kShapeC;
    const int t = q % 12;
    return t < 7 ? 0 : (t < 10 ? 1 : (t == 10 ? 2 : 3));
}
__host__ __device__ constexpr Tap quadBase(int q) {
    if (q == 36) return {0, 4, 6};
    const int ci = q / 12, t = q % 12;
    if (t < 7) return {ci, t, 0};
    if (t < 10) return {ci, 0, 4 + (t - 7)};
    if (t == 10) return {ci, 4, 4};
    return {ci, 6, 4};
}
// Smallest lane-group offset of a shape (LDS floats / flat taps): lane bases
// are rebased by it so that every per-lane register is non-negative.
__host__ __device__ constexpr int minLds(int s) {
    int m = 0;
    for (int g = 0; g < 4; ++g) m = ldsOff(kShape[s][g]) < m ? ldsOff(kShape[s][g]) : m;
    return m;
}
__host__ __device__ constexpr int minTap(int s) {
    int m = 0;
    for (int g = 0; g < 4; ++g) m = tapIdx(kShape[s][g]) < m ? tapIdx(kShape[s][g]) : m;
    return m;
}

// The quads cover every tap of the 3 x 7 x 7 window exactly once (the zero-weight
// lane of the cross-channel quad aside), and every LDS read stays inside the
// window for output columns below 112.
constexpr bool quadsCoverWindow() {
    int seen[147] = {};
    for (int q = 0; q < kStemQuads; ++q) {
        const Tap b = quadBase(q);
        const int s = quadShape(q);
        for (int g = 0; g < 4; ++g) {
            if (s == kShapeC && g == 3) continue;
            const Tap t{b.ci + kShape[s][g].ci, b.kh + kShape[s][g].kh, b.kw + kShape[s][g].kw};
            if (t.ci < 0 || t.ci > 2 || t.kh < 0 || t.kh > 6 || t.kw < 0 || t.kw > 6) return false;
            ++seen[tapIdx(t)];
        }
        // per-lane register (max 2*15+1 + shape span + the last row's 2*(rows-1) input rows)
        // + immediate (incl. 6 subtiles of 32)
        for (int g = 0; g < 4; ++g) {
            const int addr = 31 + ldsOff(kShape[s][g]) - minLds(s) + 2 * (kStemRows - 1) * kStemRS + ldsOff(b) +
                             minLds(s) + 32 * (kStemSub - 1);
            if (addr >= kStemLds || ldsOff(b) + minLds(s) < 0 || tapIdx(b) + minTap(s) < 0) return false;
        }
    }
    for (int i = 0; i < 147; ++i)
        if (seen[i] != 1) return false;
    return true;
}
static_assert(quadsCoverWindow(), "stem quads must tile the 3x7x7 window");

typedef float f32x4v __attribute__((ext_vector_type(4)));

struct StemArgs {
    const float* x;      // [N][3][H][W]
    const float* w;      // [Cout][147]
    const float* bias;   // [Cout] or null
    const float* gamma;  // BN (null = none)
    const float* beta;
    const float* mean;
    const float* var;
    float eps;
    const float* res;    // [N][Cout][Ho][Wo] or null
    float* out;          // [N][Cout][Ho][Wo]
    int N, H, W, Cout, Ho, Wo;
    int cBlocks;         // ceil(Cout / 64)
    int rows;            // output rows per block (<= kStemRows), consecutive rows of one image
    int rowBlocks;       // blocks per image: ceil(Ho / rows)
    uint32_t xBytes, wBytes, outBytes;
};

template <bool BN, bool RES, bool RELU>
__device__ __forceinline__ void stemStore(const StemArgs& p, const f32x4v (&acc)[kStemSub], const float* sEpi,
                                          int n, int oh, int cw, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const uint32_t HoWo = (uint32_t)(p.Ho * p.Wo);
    const auto ro = bufferRsrc(p.out, p.outBytes);
    const auto rr = bufferRsrc(RES ? p.res : p.out, p.outBytes);
    const int c = cw + 4 * g;   // first of the lane's four channels, relative to the block
    const int cAbs = blockIdx.y * 64 + c;
    const uint32_t base = ((uint32_t)(n * p.Cout + cAbs) * HoWo + (uint32_t)(oh * p.Wo + j)) * 4u;
    const f32x4v b = *reinterpret_cast<const f32x4v*>(sEpi + c);
    f32x4v mu{}, is{}, ga{}, be{};
    if constexpr (BN) {
        mu = *reinterpret_cast<const f32x4v*>(sEpi + 64 + c);
        is = *reinterpret_cast<const f32x4v*>(sEpi + 128 + c);
        ga = *reinterpret_cast<const f32x4v*>(sEpi + 192 + c);
        be = *reinterpret_cast<const f32x4v*>(sEpi + 256 + c);
    }
#pragma unroll
    for (int s = 0; s < kStemSub; ++s) {
        const bool colOk = 16 * s + j < p.Wo;
        float rv[4];
        uint32_t vo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            vo[r] = (colOk && cAbs + r < p.Cout) ? base + 64u * s : kOOB;
            if constexpr (RES) rv[r] = bufLoad1(rr, vo[r], (uint32_t)r * HoWo * 4u);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v = acc[s][r] + b[r];
            if constexpr (BN) v = __builtin_fmaf(ga[r], (v - mu[r]) * is[r], be[r]);
            if constexpr (RES) v += rv[r];
            if constexpr (RELU) v = v > 0.f ? v : 0.f;
            bufStore1Stream(ro, vo[r], (uint32_t)r * HoWo * 4u, v);
        }
    }
}

template <bool BN, bool RES, bool RELU>
__global__ __launch_bounds__(kStemNT) void conv_stem_kernel(StemArgs p) {
    __shared__ __attribute__((aligned(16))) float sIn[kStemLds];
    __shared__ __attribute__((aligned(16))) float sEpi[5 * 64];   // bias, mean, invStd, gamma, beta

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, j = lane & 15;
    // consecutive output rows of one image per block; an XCD takes a contiguous range of blocks
    // (neighbouring blocks share input rows in its L2)
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    const int n = blk / p.rowBlocks;
    const int oh0 = (blk - n * p.rowBlocks) * p.rows;
    const int nRows = min(p.rows, p.Ho - oh0);
    const int cw = wave * 16;
    const int cRow = blockIdx.y * 64 + cw + j;   // this lane's A row (output channel)

    // Weights: a[q] = W[cRow][tap(q, g)], via one row base per shape and the quad's flat tap as immediate.
    const auto rw = bufferRsrc(p.w, p.wBytes);
    uint32_t wb[5];
#pragma unroll
    for (int s = 0; s < 5; ++s) {
        int d = 0;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
            if (g == gg) d = tapIdx(kShape[s][gg]) - minTap(s);
        const bool zero = cRow >= p.Cout || (s == kShapeC && g == 3);
        wb[s] = zero ? kOOB : (uint32_t)(cRow * 147 + d) * 4u;
    }
    float a[kStemQuads];
#pragma unroll
    for (int q = 0; q < kStemQuads; ++q)
        a[q] = bufLoad1(rw, wb[quadShape(q)], (uint32_t)(tapIdx(quadBase(q)) + minTap(quadShape(q))) * 4u);

    // Epilogue vectors of the block's 64 channels.
    if (tid < 64) {
        const int co = min(blockIdx.y * 64 + tid, p.Cout - 1);
        sEpi[tid] = p.bias ? p.bias[co] : 0.f;
        if (p.gamma) {
            sEpi[64 + tid] = p.mean[co];
            sEpi[128 + tid] = 1.0f / sqrtf(p.var[co] + p.eps);
            sEpi[192 + tid] = p.gamma[co];
            sEpi[256 + tid] = p.beta[co];
        }
    }

    // Input window: 3 x kStemInRows rows (input rows 2*oh0-3 .. of each channel; rows past the
    // block's 2*nRows+5 or outside the image are zero) of 58 float4 columns: column quad 0 and quads
    // past the row are zero, quad c4 in [1, W/4] holds x[.., 4*(c4-1) ..]. Wave w copies rows
    // w, w+4, .. (the row arithmetic is wave-uniform), lane c4 < 58 one column quad of each, five
    // rows' loads in flight before their LDS writes.
    {
        const auto rx = bufferRsrc(p.x, p.xBytes);
        constexpr int Q = kStemRS / 4;   // 58 quads per row
        constexpr int ROWS = 3 * kStemInRows;
        constexpr int IT = (ROWS + 3) / 4;
        constexpr int CH = 5;
        const bool colOk = lane >= 1 && lane <= (p.W >> 2);
        const uint32_t colOff = (uint32_t)(4 * (lane - 1)) * 4u;
#pragma unroll
        for (int i0 = 0; i0 < IT; i0 += CH) {
            f32x4v v[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int rI = wave + 4 * (i0 + k);   // wave-uniform
                const int ci = rI / kStemInRows, kh = rI - ci * kStemInRows;
                const int y = 2 * oh0 - 3 + kh;
                const bool rowOk = rI < ROWS && kh < 2 * nRows + 5 && y >= 0 && y < p.H;
                const uint32_t rowOff = rowOk ? (uint32_t)(((n * 3 + ci) * p.H + y) * p.W) * 4u : 0u;
                v[k] = bufLoad4(rx, (rowOk && colOk) ? colOff : kOOB, rowOff);
            }
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int rI = wave + 4 * (i0 + k);
                if (rI < ROWS && lane < Q) *reinterpret_cast<f32x4v*>(sIn + rI * kStemRS + 4 * lane) = v[k];
            }
        }
    }
    __syncthreads();

    // Per-lane B bases (floats) per shape: 2j + 1 + off(G(g)) - min; row r adds 2r input rows.
    int bb[5];
#pragma unroll
    for (int s = 0; s < 5; ++s) {
        int d = 0;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
            if (g == gg) d = ldsOff(kShape[s][gg]) - minLds(s);
        bb[s] = 2 * j + 1 + d;
    }

    for (int r = 0; r < nRows; ++r) {
        // Quad q's seven B operands are read while quad q-1's MFMAs run.
        f32x4v acc[kStemSub];
#pragma unroll
        for (int s = 0; s < kStemSub; ++s) acc[s] = f32x4v{0.f, 0.f, 0.f, 0.f};
        float bq[2][kStemSub];
        auto readB = [&](int q, float (&dst)[kStemSub]) {
            const int sh = quadShape(q);
            const float* src = sIn + bb[sh] + (ldsOff(quadBase(q)) + minLds(sh));
#pragma unroll
            for (int s = 0; s < kStemSub; ++s) dst[s] = src[32 * s];
        };
        readB(0, bq[0]);
#pragma unroll
        for (int q = 0; q < kStemQuads; ++q) {
            if (q + 1 < kStemQuads) readB(q + 1, bq[(q + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < kStemSub; ++s)
                acc[s] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], bq[q & 1][s], acc[s], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        stemStore<BN, RES, RELU>(p, acc, sEpi, n, oh0 + r, cw, lane);
#pragma unroll
        for (int s = 0; s < 5; ++s) bb[s] += 2 * kStemRS;
    }
}

template <bool BN, bool RES, bool RELU>
int launchStem(const StemArgs& p) {
    hipLaunchKernelGGL((conv_stem_kernel<BN, RES, RELU>), dim3(p.N * p.rowBlocks, p.cBlocks), dim3(kStemNT), 0,
                       stream(), p);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // namespace

bool stemGeometry(int Cin, int W, int KH, int KW, int stride, int padH, int padW) {
    return Cin == 3 && KH == 7 && KW == 7 && stride == 2 && padH == 3 && padW == 3 && W % 4 == 0 && W <= 224;
}

int convStem(const float* x, const float* w, const float* bias, const float* gamma, const float* beta,
             const float* mean, const float* var, float eps, const float* res, int act, float* out, int N, int H,
             int W, int Cout, int Ho, int Wo) {
    StemArgs p{x, w, bias, gamma, beta, mean, var, eps, res, out, N, H, W, Cout, Ho, Wo, (Cout + 63) / 64, 1, Ho,
               0, 0, 0};
    // Rows per block: the busiest CU runs ceil(blocks / CUs) blocks of `rows` rows each, plus a
    // block's start-up (weights, input window) worth about a third of a row; fewer blocks win ties.
    {
        const long long U = cuCount();
        double best = 1e300;
        for (int r = 1; r <= kStemRows; ++r) {
            const long long rb = (Ho + r - 1) / r;
            const long long blocks = (long long)N * rb * p.cBlocks;
            const double cost = (double)((blocks + U - 1) / U) * (std::min(r, Ho) + 0.3);
            if (cost <= best) { best = cost; p.rows = r; p.rowBlocks = (int)rb; }
        }
    }
    const long long xBytes = (long long)N * 3 * H * W * 4, wBytes = (long long)Cout * 147 * 4;
    const long long oBytes = (long long)N * Cout * Ho * Wo * 4;
    if (xBytes > (long long)kMaxBufferBytes || wBytes > (long long)kMaxBufferBytes ||
        oBytes > (long long)kMaxBufferBytes || (long long)N * Ho >= (1LL << 31) || Wo > 16 * kStemSub || Ho <= 0)
        return fail("conv stem: tensor exceeds the 2^30-byte buffer range of this kernel");
    p.xBytes = (uint32_t)xBytes;
    p.wBytes = (uint32_t)wBytes;
    p.outBytes = (uint32_t)oBytes;
    switch ((gamma ? 1 : 0) | (res ? 2 : 0) | (act == 1 ? 4 : 0)) {
        case 0: return launchStem<false, false, false>(p);
        case 1: return launchStem<true, false, false>(p);
        case 2: return launchStem<false, true, false>(p);
        case 3: return launchStem<true, true, false>(p);
        case 4: return launchStem<false, false, true>(p);
        case 5: return launchStem<true, false, true>(p);
        case 6: return launchStem<false, true, true>(p);
        default: return launchStem<true, true, true>(p);
    }
}

}  // namespace omhip
