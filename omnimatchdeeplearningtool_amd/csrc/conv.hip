// conv.hip — NCHW conv2d as an implicit GEMM on fp32 MFMA, with the
// bias + BatchNorm(inference) + ReLU epilogue fused into the output write.
//
//   Out[co][q] = sum_kk W[co][kk] * X^[kk][q]
//   kk = (ci*KH + kh)*KW + kw    (the reference im2col row order, cpu_backend.ixx:554-557)
//   q  = (n*Ho + oh)*Wo + ow     (output pixel, batch folded into the GEMM N axis)
//   X^[kk][q] = x[n][ci][oh*s-p+kh][ow*s-p+kw], zero outside the image
//
// The reference lowers conv2d per image to im2col + matmul + bias
// (cpu_backend.ixx:619-658) and applies batchNorm2d / relu as separate passes
// (tensor_ops.ixx:672-833, :511-536). Here the im2col operand is never
// materialised: each thread gathers its pixels' taps straight into the LDS
// B slice, and the output passes through HBM once, already normalised.
//
// gfx950 does not overlap VALU work with MFMA execution, so every VALU
// instruction in the mainloop costs matrix-core time. Both operands are
// therefore fetched with raw buffer loads whose per-lane offset is fixed for
// the whole K walk and whose uniform part (slice start, tap offset) rides in
// the scalar soffset: a weight slice costs no VALU, a gathered im2col element
// costs two (a bit extract of the pixel's "tap outside the image" mask and a
// shift-or that pushes such a lane past the buffer end, where the hardware's
// range check returns 0). Tap offsets come from a per-geometry table read
// with scalar loads.
//
// Split-K (for late layers whose Cout x pixels tile count cannot fill 256 CUs)
// and the K pieces of remainder tiles write fp32 partial tiles to a
// workspace; the last block of a tile to finish (counted per tile) sums the
// parts in a fixed order (deterministic) and applies the same epilogue, so no
// second launch is needed.
#include "omhip_internal.hpp"
#include "mfma_f32_tile.hpp"
#include "buffer_io.hpp"
#include "fastdiv.hpp"
#include "gemm_f32.hpp"
#include "conv.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

namespace omhip {

struct ConvParams {
    const float* x;      // [N][Cin][H][W] (this batch chunk)
    const float* w;      // [Cout][Cin*KH*KW]
    const float* bias;   // [Cout] or null
    const float* gamma;  // BN (all four null = no BN)
    const float* beta;
    const float* mean;
    const float* var;
    float eps;
    int act;             // 0 identity, 1 relu
    const float* res;    // [N][Cout][Ho][Wo] added after BN, before the activation, or null
    float* out;          // [N][Cout][Ho][Wo]
    float* ws;           // split-K partials [splits][Cout][Nq]
    const uint2* tab;    // per K row: (byte offset of tap (ci,kh,kw), tap code); "outside" code past K
    int N, Cin, H, W, Cout, KH, KW, stride;
    int padH, padW;      // top / left padding; negative crops (the window starts inside the image)
    int Ho, Wo;          // output pixel grid of the GEMM
    // Output image: grid pixel (oh, ow) is written at (oh*oStride + oOffH, ow*oStride + oOffW) of an
    // oH x oW image (the plain conv: oStride 1, offsets 0, oH x oW = Ho x Wo).
    int oH, oW, oStride, oOffH, oOffW;
    int K;               // Cin*KH*KW
    int Nq;              // N*Ho*Wo
    int tilesM, tilesN;
    int splits, kChunk;  // split-K: k range [s*kChunk, min(K,(s+1)*kChunk))
    // splits == 1: tiles [0, fullTiles) of the grouped order run whole; the rest
    // run as remPieces K pieces of remChunk, partials in rws [piece][tile - fullTiles][BM][BN].
    int fullTiles, remPieces, remChunk;
    float* rws;
    unsigned* ctr;       // split-K / remainder tiles: per-tile arrival counters (zero at rest)
    int padOff;          // max(padH,0)*W + max(padW,0): the x buffer view starts this many floats before x
    uint32_t xBytes;     // range of the x buffer view
    FastDiv dHoWo, dWo;  // division by Ho*Wo and by Wo (grid pixel indices are below 2^30)
    uint64_t rowRep;     // bit rr*KW set for rr < KH (mask modes: KH*KW <= 63)
};

// Tap table: entry kk = (4*(ci*H*W + kh*W + kw), code), code = kh*KW+kw for
// the mask modes or (kh << 16) | kw for the coordinate-compare mode. Rows past
// K get offset 0 and a code that tests "outside" for every pixel (mask bit
// 31 / 63, or kh = kw = 0xffff with H + pad, W + pad < 65535), so a slice that
// runs past K gathers zeros through the voffset range check.
__global__ void build_tap_table(uint2* tab, int K, int Kpad, int KH, int KW, int H, int W, int mode) {
    const int kk = blockIdx.x * blockDim.x + threadIdx.x;
    if (kk >= Kpad) return;
    uint2 e;
    if (kk < K) {
        const int khw = KH * KW;
        const int ci = kk / khw;
        const int t = kk - ci * khw;
        const int kh = t / KW;
        const int kw = t - kh * KW;
        e.x = (uint32_t)(ci * H * W + kh * W + kw) * 4u;
        e.y = mode == 2 ? (uint32_t)((kh << 16) | kw) : (uint32_t)t;
    } else {
        e.x = 0;
        e.y = mode == 0 ? 31u : (mode == 1 ? 63u : 0xffffffffu);
    }
    tab[kk] = e;
}

// Weight slice loader: W[Cout][K] with K contiguous -> LDS [BM][BK+4].
// Each thread owns fixed (row, k) positions; its byte offsets are computed
// once and the slice start rides in soffset. Rows past Cout point past the
// buffer end (zero). The last slice of a K range is loaded with an explicit
// column test (it may end inside the slice).
template <int BM, int BK, int NT, bool VEC>
struct WeightLoader {
    static constexpr int PER_T = VEC ? BM * BK / 4 / NT : BM * BK / NT;
    static_assert(BM * BK % (NT * (VEC ? 4 : 1)) == 0, "slice must split evenly");
    using Shape = LdsShape<true, BM, BK>;
    __amdgpu_buffer_rsrc_t r;
    uint32_t voff[PER_T];
    f32x4 v4[VEC ? PER_T : 1];
    float v1[VEC ? 1 : PER_T];

    static __device__ __forceinline__ void coords(int e, int& row, int& k) {
        if constexpr (VEC) { row = e / (BK / 4); k = (e % (BK / 4)) * 4; }
        else { row = e / BK; k = e % BK; }
    }

    __device__ void init(const ConvParams& p, int m0, int tid) {
        r = bufferRsrc(p.w, (uint32_t)p.Cout * (uint32_t)p.K * 4u);
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int row, k;
            coords(tid + i * NT, row, k);
            voff[i] = (m0 + row < p.Cout) ? (uint32_t)((m0 + row) * p.K + k) * 4u : kOOB;
        }
    }

    // FULL: the slice lies inside [k0, kEnd) (no per-element test).
    template <bool FULL = false>
    __device__ void load(int k0, int kEnd, int tid) {
        const uint32_t soff = (uint32_t)k0 * 4u;
        if (FULL || k0 + BK <= kEnd) {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                if constexpr (VEC) v4[i] = bufLoad4(r, voff[i], soff);
                else v1[i] = bufLoad1(r, voff[i], soff);
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                int row, k;
                coords(tid + i * NT, row, k);
                const uint32_t vo = (k0 + k < kEnd) ? voff[i] : kOOB;   // VEC: K % 4 == 0, all-or-none
                if constexpr (VEC) v4[i] = bufLoad4(r, vo, soff);
                else v1[i] = bufLoad1(r, vo, soff);
            }
        }
    }

    __device__ void store(float* s, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int row, k;
            coords(tid + i * NT, row, k);
            if constexpr (VEC) *reinterpret_cast<f32x4*>(s + row * Shape::LD + k) = v4[i];
            else s[row * Shape::LD + k] = v1[i];
        }
    }
};

// Implicit im2col loader -> LDS [BN][BK+4] (K contiguous, like the weights,
// so both MFMA operands are read 4 k at a time). Thread t owns pixel column
// c = t % BN and the RPT consecutive rows g*RPT .. g*RPT+RPT-1 of each slice
// (g = t / BN, the same for all lanes of a wave since BN >= 64), so the rows'
// table entries are wave-uniform scalar loads and the thread's RPT values are
// contiguous in its pixel's LDS row (128-bit stores). Per pixel: one byte offset
// (into a buffer view that starts pad*W+pad floats before x, so it is never
// negative) and the mask of taps that fall outside the image.
//   MODE: gatherMode(KH*KW), or 3 for an unpadded 1x1 kernel whose taps all
//   lie inside the image: no mask, and in slices wholly inside K (FULL) no
//   per-element arithmetic at all (rows past K still read 0: their table
//   code is nonzero).
template <int BN, int BK, int NT, int MODE>
struct GatherLoader {
    static constexpr int TPC = NT / BN;
    static constexpr int RPT = BK / TPC;
    static_assert(NT % BN == 0 && BK % TPC == 0 && BN >= 64 && RPT % 4 == 0, "gather mapping");
    using Shape = LdsShape<true, BN, BK>;
    __amdgpu_buffer_rsrc_t r;
    uint32_t voffPix;
    uint32_t invLo, invHi;
    int ih0, iw0, H, W;
    int rowOff;   // (tid / BN) * RPT: wave-uniform, kept in a scalar register
    const uint2* tab;
    float v[RPT];

    __device__ void init(const ConvParams& p, int q, int tid) {
        rowOff = __builtin_amdgcn_readfirstlane((tid / BN) * RPT);
        r = bufferRsrc(p.x - p.padOff, p.xBytes);
        tab = p.tab;
        H = p.H; W = p.W;
        const bool colValid = q < p.Nq;
        const int qq = colValid ? q : 0;
        const int HoWo = p.Ho * p.Wo;
        const int n = (int)p.dHoWo.div((uint32_t)qq);
        const int pix = qq - n * HoWo;
        const int oh = (int)p.dWo.div((uint32_t)pix), ow = pix - oh * p.Wo;
        ih0 = colValid ? oh * p.stride - p.padH : -(1 << 29);   // a padding column matches no tap
        iw0 = ow * p.stride - p.padW;
        voffPix = (uint32_t)(n * p.Cin * p.H * p.W + (colValid ? ih0 : 0) * W + iw0 + p.padOff) * 4u;
        if constexpr (MODE == 3) {
            if (!colValid) voffPix = kOOB;   // a padding column reads zeros
            return;
        }
        uint64_t inside = 0;
        if constexpr (MODE != 2) {
            // Taps (kh, kw) inside the image: kw in [cl, ch), kh in [rl, rh).
            // colBits * rowRep repeats the column bits in every row's KW-bit
            // field (no carries: colBits < 2^KW); the row mask keeps [rl, rh).
            const int cl = min(max(-iw0, 0), p.KW), ch = max(min(p.KW, W - iw0), cl);
            const int rl = min(max(-ih0, 0), p.KH), rh = max(min(p.KH, H - ih0), rl);
            const uint64_t colBits = (1ull << ch) - (1ull << cl);
            inside = (colBits * p.rowRep) & ((1ull << (rh * p.KW)) - (1ull << (rl * p.KW)));
        }
        invLo = ~(uint32_t)inside;
        invHi = ~(uint32_t)(inside >> 32);
    }

    // Issues this thread's RPT loads of the slice starting at row kk0 (FULL:
    // the slice lies wholly inside K).
    template <bool FULL = false>
    __device__ void load(int kk0, int /*tid*/) {
        const int base = kk0 + rowOff;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const uint2 e = tab[base + j];
            uint32_t inv;
            if constexpr (MODE == 3) {
                if constexpr (FULL) {
                    v[j] = bufLoad1(r, voffPix, e.x);
                    continue;
                }
                inv = e.y != 0u;   // 0 for the single tap, 31 for rows past K
            } else if constexpr (MODE == 0) {
                inv = __builtin_amdgcn_ubfe(invLo, e.y, 1);
            } else if constexpr (MODE == 1) {
                inv = (uint32_t)((((uint64_t)invHi << 32) | invLo) >> e.y) & 1u;
            } else {
                const int kh = (int)(e.y >> 16), kw = (int)(e.y & 0xffffu);
                inv = ((unsigned)(ih0 + kh) >= (unsigned)H) | ((unsigned)(iw0 + kw) >= (unsigned)W);
            }
            v[j] = bufLoad1(r, (inv << 30) | voffPix, e.x);
        }
    }

    __device__ void store(float* s, int tid) const {
        const int c = tid % BN, g = tid / BN;
#pragma unroll
        for (int j = 0; j < RPT; j += 4) {
            const f32x4 q = {v[j], v[j + 1], v[j + 2], v[j + 3]};
            *reinterpret_cast<f32x4*>(s + c * Shape::LD + g * RPT + j) = q;
        }
    }
};

// Index within the output image of grid pixel pix = oh*Wo + ow.
__device__ __forceinline__ int outPixel(const ConvParams& p, int pix) {
    if (p.oStride == 1 && p.oOffH == 0 && p.oOffW == 0 && p.oW == p.Wo) return pix;
    const int oh = (int)p.dWo.div((uint32_t)pix), ow = pix - oh * p.Wo;
    return (oh * p.oStride + p.oOffH) * p.oW + ow * p.oStride + p.oOffW;
}

// Direct epilogue of one block's tile: bias, BN (inference), residual and
// ReLU applied to the finished sums and written to the NCHW output. The lane
// holding acc[fm][fn][r] owns tile row wm*WM + fm*32 + 8*(r/4) + 4*(lane/32) +
// r%4 and column wn*WN + fn*32 + lane%32, so rows r = 4j..4j+3 are four
// consecutive channels (one 16-byte read of each epilogue vector) and a row's
// byte offset past the lane's first row is the wave-uniform (8j + r%4) * row
// stride, carried in soffset. Columns past Nq and rows past Cout get an
// out-of-range voffset and store nothing. The output view (chunk images x
// Cout x oH x oW floats) is at most 2^30 bytes. The stores are streaming (nt):
// every block of a launch finishes at about the same time, and the output
// then drains to memory as it is written rather than in the L2 write-back at
// the end of the launch (ResNet-18 b32 stack -1 %).
template <class Cfg, bool BN, bool RES, bool RELU>
__device__ __forceinline__ void storeTile(const ConvParams& p, const f32x16 (&acc)[Cfg::FM][Cfg::FN],
                                          const float* sEpi, int m0, int n0, int wm, int wn, int lane) {
    const int li = lane & 31, h = lane >> 5;
    const int HoWo = p.Ho * p.Wo;
    const uint32_t oHW = (uint32_t)(p.oH * p.oW);
    const uint32_t viewBytes = (uint32_t)p.N * (uint32_t)p.Cout * oHW * 4u;
    const auto ro = bufferRsrc(p.out, viewBytes);
    const auto rr = bufferRsrc(RES ? p.res : p.out, viewBytes);   // read only when RES
    const bool fullM = m0 + Cfg::BM <= p.Cout;
#pragma unroll
    for (int fn = 0; fn < Cfg::FN; ++fn) {
        const int q = n0 + wn * Cfg::WN + fn * 32 + li;
        const bool colOk = q < p.Nq;
        const int qq = colOk ? q : 0;
        const int n = (int)p.dHoWo.div((uint32_t)qq);
        const int opix = outPixel(p, qq - n * HoWo);
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm) {
            const int rl0 = wm * Cfg::WM + fm * 32 + 4 * h;
            const uint32_t vbase = colOk ? ((uint32_t)(n * p.Cout + m0 + rl0) * oHW + (uint32_t)opix) * 4u : kOOB;
            const int rowsLeft = p.Cout - m0 - rl0;   // rows of this lane's column still inside Cout
            // one group of four channels at a time: its residuals, epilogue
            // vectors and results stay within a few registers
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rl = rl0 + 8 * j;
                uint32_t vo[4];
                float rv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    vo[i] = (fullM || 8 * j + i < rowsLeft) ? vbase : kOOB;
                    if constexpr (RES) rv[i] = bufLoad1(rr, vo[i], (8 * j + i) * oHW * 4u);
                }
                const f32x4 b = *reinterpret_cast<const f32x4*>(sEpi + rl);
                f32x4 mu, is, g, be;
                if constexpr (BN) {
                    mu = *reinterpret_cast<const f32x4*>(sEpi + Cfg::BM + rl);
                    is = *reinterpret_cast<const f32x4*>(sEpi + 2 * Cfg::BM + rl);
                    g = *reinterpret_cast<const f32x4*>(sEpi + 3 * Cfg::BM + rl);
                    be = *reinterpret_cast<const f32x4*>(sEpi + 4 * Cfg::BM + rl);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = acc[fm][fn][4 * j + i] + b[i];
                    if constexpr (BN) v = __builtin_fmaf(g[i], (v - mu[i]) * is[i], be[i]);
                    if constexpr (RES) v += rv[i];
                    if constexpr (RELU) v = v > 0.f ? v : 0.f;
                    bufStore1Stream(ro, vo[i], (8 * j + i) * oHW * 4u, v);
                }
                __builtin_amdgcn_sched_barrier(0);   // keeps one group's registers live at a time
            }
        }
    }
}

// Output epilogue by variant (BN, residual, ReLU chosen per launch).
template <class Cfg>
__device__ __forceinline__ void storeEpilogue(const ConvParams& p, const f32x16 (&acc)[Cfg::FM][Cfg::FN],
                                              const float* sEpi, int m0, int n0, int wm, int wn, int lane) {
    switch ((p.gamma ? 1 : 0) | (p.res ? 2 : 0) | (p.act == 1 ? 4 : 0)) {
        case 0: storeTile<Cfg, false, false, false>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 1: storeTile<Cfg, true, false, false>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 2: storeTile<Cfg, false, true, false>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 3: storeTile<Cfg, true, true, false>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 4: storeTile<Cfg, false, false, true>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 5: storeTile<Cfg, true, false, true>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        case 6: storeTile<Cfg, false, true, true>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
        default: storeTile<Cfg, true, true, true>(p, acc, sEpi, m0, n0, wm, wn, lane); break;
    }
}

// Writes one block's finished accumulators. A direct block applies the
// epilogue and writes the output. A K piece (remainder tiles) writes a compact
// partial tile, a split (split-K) its [Cout][Nq] partials (same row / column
// ownership and out-of-range handling as storeTile); then the block counts
// itself in at the tile's counter, and the block that arrives last adds every
// part's partials in part order (0 + part 0 + part 1 + ...), applies the
// epilogue, writes the output and returns the counter to zero. The order of
// the sum does not depend on which block arrives last, so the result is
// deterministic and equal to a separate finishing pass's. Partials are
// written and read with agent-coherent (sc1) accesses — the encoding of
// monotonic agent-scope atomic loads / stores in the gfx942 / gfx950 memory
// model, performed at the device coherence point past the per-XCD L2s; a
// block's stores have completed (s_waitcnt) before its thread 0 increments the
// counter, and the last block reads the partials only after seeing the final
// count. An acquire-release counter add would add an L2 write-back to every
// arrival and an L2 invalidate to each, which exist for non-coherent accesses
// (none cross between the blocks here): measured on MI355X, the ResNet-18 b32
// stack then ran 1134 -> 1361 us (layer-3 3x3 convs 71 -> 95 us).
template <class Cfg>
__device__ __forceinline__ void finishBlock(const ConvParams& p, f32x16 (&acc)[Cfg::FM][Cfg::FN], const float* sEpi,
                                            int* sFlag, int m0, int n0, int wm, int wn, int lane, int piece,
                                            int rtile, int split, bool direct, int ctrIdx) {
    const int li = lane & 31, h = lane >> 5;
    if (!direct) {
        const int tiles = p.tilesM * p.tilesN;
        const uint32_t nq = (uint32_t)p.Nq;
        const int nParts = piece >= 0 ? p.remPieces : p.splits;
        const long long pieceElems = (long long)(tiles - p.fullTiles) * (Cfg::BM * Cfg::BN);
        float* const rbase = p.rws + (long long)rtile * (Cfg::BM * Cfg::BN);
        // element (fm, fn, r) of part `part`: compact tile row / column, or [Cout][Nq] position
        auto rowOf = [&](int fm, int r) { return wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3); };
        if (piece >= 0) {
            const auto rp = bufferRsrc(rbase + piece * pieceElems, Cfg::BM * Cfg::BN * 4u);
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
                for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        bufStore1Agent(rp, (uint32_t)(rowOf(fm, r) * Cfg::BN + wn * Cfg::WN + fn * 32 + li) * 4u, 0u,
                                       acc[fm][fn][r]);
        } else {
            const auto rw = bufferRsrc(p.ws + (long long)split * p.Cout * p.Nq, (uint32_t)p.Cout * nq * 4u);
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn) {
                const int q = n0 + wn * Cfg::WN + fn * 32 + li;
#pragma unroll
                for (int fm = 0; fm < Cfg::FM; ++fm) {
                    const int rl0 = wm * Cfg::WM + fm * 32 + 4 * h;
                    const uint32_t vbase = q < p.Nq ? ((uint32_t)(m0 + rl0) * nq + (uint32_t)q) * 4u : kOOB;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int rowOff = 8 * (r >> 2) + (r & 3);
                        const uint32_t vo = m0 + rl0 + rowOff < p.Cout ? vbase : kOOB;
                        bufStore1Agent(rw, vo, (uint32_t)rowOff * nq * 4u, acc[fm][fn][r]);
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);   // this thread's partial stores have completed
        __syncthreads();
        if (threadIdx.x == 0)
            *sFlag = __hip_atomic_fetch_add(p.ctr + ctrIdx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(nParts - 1);
        __syncthreads();
        if (!*sFlag) return;
        // last arrival: acc = 0 + part 0 + part 1 + ...
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.f;
        for (int part = 0; part < nParts; ++part) {
            if (piece >= 0) {
                const auto rp = bufferRsrc(rbase + part * pieceElems, Cfg::BM * Cfg::BN * 4u);
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
                    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[fm][fn][r] += bufLoad1Agent(
                                rp, (uint32_t)(rowOf(fm, r) * Cfg::BN + wn * Cfg::WN + fn * 32 + li) * 4u, 0u);
            } else {
                const auto rw = bufferRsrc(p.ws + (long long)part * p.Cout * p.Nq, (uint32_t)p.Cout * nq * 4u);
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn) {
                    const int q = n0 + wn * Cfg::WN + fn * 32 + li;
#pragma unroll
                    for (int fm = 0; fm < Cfg::FM; ++fm) {
                        const int rl0 = wm * Cfg::WM + fm * 32 + 4 * h;
                        const uint32_t vbase = q < p.Nq ? ((uint32_t)(m0 + rl0) * nq + (uint32_t)q) * 4u : kOOB;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int rowOff = 8 * (r >> 2) + (r & 3);
                            const uint32_t vo = m0 + rl0 + rowOff < p.Cout ? vbase : kOOB;
                            acc[fm][fn][r] += bufLoad1Agent(rw, vo, (uint32_t)rowOff * nq * 4u);
                        }
                    }
                }
            }
        }
        if (threadIdx.x == 0)   // ready for the next launch
            __hip_atomic_store(p.ctr + ctrIdx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    storeEpilogue<Cfg>(p, acc, sEpi, m0, n0, wm, wn, lane);
}

// Stages the epilogue vectors of output channels m0 .. m0+BM-1 in LDS (bias,
// mean, invStd, gamma, beta); threads tid < BM each take one channel.
template <int BM>
__device__ __forceinline__ void stageEpilogue(const ConvParams& p, float* sEpi, int m0, int tid) {
    if (tid < BM) {
        const int co = min(m0 + tid, p.Cout - 1);
        sEpi[tid] = p.bias ? p.bias[co] : 0.f;
        if (p.gamma) {
            sEpi[BM + tid] = p.mean[co];
            sEpi[2 * BM + tid] = 1.0f / sqrtf(p.var[co] + p.eps);
            sEpi[3 * BM + tid] = p.gamma[co];
            sEpi[4 * BM + tid] = p.beta[co];
        }
    }
}

template <class Cfg, bool VA, int MODE>
__global__ __launch_bounds__(Cfg::NT) void conv_igemm_kernel(ConvParams p) {
    extern __shared__ float smem[];
    using SA = LdsShape<true, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<true, Cfg::BN, Cfg::BK>;
    constexpr int STAGE = SA::SIZE + SB::SIZE;
    float* sEpi = smem + 2 * STAGE;   // [5][BM]: bias, mean, invStd, gamma, beta
    int* sFlag = reinterpret_cast<int*>(sEpi + 5 * Cfg::BM);   // last-arrival flag of a split tile

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N;
    const int wn = wave % Cfg::WAVES_N;

    // Block -> (tile, k range). Split-K: blockIdx.y is the split. Otherwise the
    // first fullTiles blocks take whole tiles and the rest take K pieces of the
    // remaining tiles, which evens out the work per CU when the tile count is
    // not a multiple of the CU count.
    const int tiles = p.tilesM * p.tilesN;
    const int split = blockIdx.y;
    int tm, tn, kBeg, kEnd;
    int piece = -1, rtile = 0;
    if (p.splits > 1) {
        tile_coords(blockIdx.x, tiles, p.tilesM, p.tilesN, 4, tm, tn);
        kBeg = split * p.kChunk;
        kEnd = min(p.K, kBeg + p.kChunk);
    } else if ((int)blockIdx.x < p.fullTiles) {
        tile_coords(blockIdx.x, p.fullTiles, p.tilesM, p.tilesN, 4, tm, tn);
        kBeg = 0;
        kEnd = p.K;
    } else {
        const int b = blockIdx.x - p.fullTiles;
        rtile = b / p.remPieces;
        piece = b - rtile * p.remPieces;
        grouped_tile(p.fullTiles + rtile, p.tilesM, p.tilesN, 4, tm, tn);
        kBeg = piece * p.remChunk;
        kEnd = min(p.K, kBeg + p.remChunk);
    }
    const int m0 = tm * Cfg::BM;
    const int n0 = tn * Cfg::BN;

    WeightLoader<Cfg::BM, Cfg::BK, Cfg::NT, VA> la;
    la.init(p, m0, tid);
    GatherLoader<Cfg::BN, Cfg::BK, Cfg::NT, MODE> lb;
    lb.init(p, n0 + tid % Cfg::BN, tid);

    const bool direct = p.splits == 1 && piece < 0;
    stageEpilogue<Cfg::BM>(p, sEpi, m0, tid);   // the last part of a split tile applies the epilogue too

    f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = (kEnd - kBeg + Cfg::BK - 1) / Cfg::BK;
    lb.load(kBeg, tid);
    la.load(kBeg, kEnd, tid);
    la.store(smem, tid);
    lb.store(smem + SA::SIZE, tid);
    const int nFull = (kEnd - kBeg) / Cfg::BK;
    int t = 0;
    // Two slices in flight: while slice t is multiplied from LDS, slice t+1 (loaded
    // one slice earlier) is stored to the other stage and slice t+2 is loaded into a
    // second register set (la2 / lb2), so a load has two slices of MFMAs to land
    // instead of one. Measured on the ResNet-18 b32 convs: each layer alone takes the
    // same time, the 20 layers back to back 1.109-1.113 -> 1.089-1.090 ms. The
    // kernel's register peak is its epilogue, so the second set costs no occupancy.
    // Slice t is in stage t & 1; on entry to a trip la / lb hold slice t+1. The
    // unchecked loop runs while both slices it fetches (t+2, t+3) lie wholly inside
    // the K range; the schedule barriers keep each half in the order global loads,
    // MFMAs, LDS stores (left alone, the scheduler hoists the stores and the block
    // barrier above most MFMAs and then waits on the loads it has just issued).
    WeightLoader<Cfg::BM, Cfg::BK, Cfg::NT, VA> la2;
    la2.init(p, m0, tid);
    GatherLoader<Cfg::BN, Cfg::BK, Cfg::NT, MODE> lb2;
    lb2.init(p, n0 + tid % Cfg::BN, tid);
    if (nk > 1) {
        lb.load(kBeg + Cfg::BK, tid);
        la.load(kBeg + Cfg::BK, kEnd, tid);
    }
    __syncthreads();
    for (; t + 3 < nFull; t += 2) {
        lb2.template load<true>(kBeg + (t + 2) * Cfg::BK, tid);
        la2.template load<true>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
        __builtin_amdgcn_sched_barrier(0);
        mma_slice<Cfg, true, true>(smem, smem + SA::SIZE, acc, wm, wn, lane);
        __builtin_amdgcn_sched_barrier(0);
        la.store(smem + STAGE, tid);
        lb.store(smem + STAGE + SA::SIZE, tid);
        __syncthreads();
        lb.template load<true>(kBeg + (t + 3) * Cfg::BK, tid);
        la.template load<true>(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
        __builtin_amdgcn_sched_barrier(0);
        mma_slice<Cfg, true, true>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane);
        __builtin_amdgcn_sched_barrier(0);
        la2.store(smem, tid);
        lb2.store(smem + SA::SIZE, tid);
        __syncthreads();
    }
    for (; t < nk; t += 2) {
        if (t + 2 < nk) {
            lb2.load(kBeg + (t + 2) * Cfg::BK, tid);
            la2.load(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
        }
        mma_slice<Cfg, true, true>(smem, smem + SA::SIZE, acc, wm, wn, lane);
        if (t + 1 < nk) {
            la.store(smem + STAGE, tid);
            lb.store(smem + STAGE + SA::SIZE, tid);
        }
        __syncthreads();
        if (t + 1 < nk) {
            if (t + 3 < nk) {
                lb.load(kBeg + (t + 3) * Cfg::BK, tid);
                la.load(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
            }
            mma_slice<Cfg, true, true>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane);
            if (t + 2 < nk) {
                la2.store(smem, tid);
                lb2.store(smem + SA::SIZE, tid);
            }
            __syncthreads();
        }
    }

    finishBlock<Cfg>(p, acc, sEpi, sFlag, m0, n0, wm, wn, lane, piece, rtile, split, direct,
                     piece >= 0 ? rtile : tm * p.tilesN + tn);
}

// ---- tile configuration -------------------------------------------------------
// 64 x 64 output tile, 4 waves of 32 x 32, 16-deep K slices. Measured on MI355X
// across the ResNet conv shapes this tile beats 64x128 ... 256x128 tiles on
// every layer: it keeps 7 blocks per CU resident (7 waves per SIMD, 68 VGPRs and
// ~22 KB of LDS each), which hides the gather latency, and (with the buffer-load
// loaders) costs about two VALU per MFMA.
#ifndef OMHIP_CONV_BK
#define OMHIP_CONV_BK 16
#endif
#ifndef OMHIP_CONV_TILE
#define OMHIP_CONV_TILE 64, 64, 32, 32   // BM, BN, WM, WN
#endif
constexpr int kConvBK = OMHIP_CONV_BK;
template <int BM, int BN, int WM, int WN>
using ConvCfgT = TileCfg<BM, BN, kConvBK, WM, WN>;
using ConvCfg = ConvCfgT<OMHIP_CONV_TILE>;

template <class Cfg>
static size_t convLds() {
    // two A+B stages and the epilogue vectors
    return (2 * (LdsShape<true, Cfg::BM, Cfg::BK>::SIZE + LdsShape<true, Cfg::BN, Cfg::BK>::SIZE) + 5 * Cfg::BM + 4) *
           sizeof(float);
}

template <class Cfg, bool VA, int MODE>
static int launchConvT(ConvParams& p, int gridX) {
    auto kern = conv_igemm_kernel<Cfg, VA, MODE>;
    const size_t lds = convLds<Cfg>();
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    hipLaunchKernelGGL(kern, dim3(gridX, p.splits), dim3(Cfg::NT), lds, stream(), p);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

struct ConvPlan {
    int splits;      // uniform split-K factor
    int fullTiles;   // splits == 1: tiles run whole (the rest run as remPieces K pieces)
    int remPieces;
};

// Work split, from a model of per-CU time: all blocks of these launches are
// resident at once, so a layer takes as long as its busiest CU.
//  * Fewer than 2 tiles per CU (late ResNet stages: few pixels, many
//    channels): split K uniformly by the s in [1, 16] (>= 128 taps per split)
//    that minimises ceil(tiles*s/CUs)/s tile-times per CU plus s extra fp32
//    writes and reads of the output (e.g. 512x1568x4608: 5 splits).
//  * Otherwise, when the tile count is not a multiple of the CU count and the
//    CUs hold few tiles each: the tiles beyond the last whole round run as K
//    pieces (one per idle CU, at most 16 per tile), summed by each tile's last
//    piece to finish, e.g. 1568 tiles on 256 CUs: 1536 whole + 32 x 8 pieces,
//    6.125 tile-times per CU instead of 7 (K >= 256 only: shorter tiles do not
//    pay for the partial traffic).
static ConvPlan planConv(const ConvParams& p, bool haveSplitWs) {
    using Cfg = ConvCfg;
    ConvPlan pl{1, p.tilesM * p.tilesN, 1};
    const long long U = cuCount();
    const long long T = (long long)p.tilesM * p.tilesN;
    const int nk = (p.K + Cfg::BK - 1) / Cfg::BK;
    if (T < 2 * U) {
        if (!haveSplitWs) return pl;
        // seconds: one tile on one CU at 65 % of its share of peak; one split's partial
        // write + read at an effective 6 TB/s (it partly overlaps the MFMA work)
        const double tileT = 2.0 * Cfg::BM * Cfg::BN * p.K / (0.65 * 157.3e12 / 256.0);
        const double partT = 8.0 * p.Cout * (double)p.Nq / 6.0e12;
        double best = (double)((T + U - 1) / U) * tileT;
        for (int s = 2; s <= 16 && p.K / s >= 128; ++s) {
            const double c = (double)((T * s + U - 1) / U) / s * tileT + s * partT;
            if (c < best) { best = c; pl.splits = s; }
        }
        return pl;
    }
    if (T >= 12 * U || nk < 16) return pl;   // many rounds, or tiles too short to pay a second launch
    const long long R = T % U;
    const int pieces = (int)std::min<long long>({16, R ? U / R : 0, (long long)nk});
    if (R == 0 || pieces < 2) return pl;
    pl.fullTiles = (int)(T - R);
    pl.remPieces = pieces;
    return pl;
}

static int launchConv(ConvParams& p, const ConvPlan& pl, float* wsBuf) {
    using Cfg = ConvCfg;
    const int tiles = p.tilesM * p.tilesN;
    int gridX = tiles;
    p.splits = 1;
    p.kChunk = p.K;
    p.fullTiles = tiles;
    p.remPieces = 1;
    p.remChunk = p.K;
    p.ws = nullptr;
    p.rws = nullptr;
    if (pl.splits > 1) {
        p.kChunk = (p.K + pl.splits - 1) / pl.splits;
        p.kChunk = (p.kChunk + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
        p.splits = (p.K + p.kChunk - 1) / p.kChunk;
        p.ws = wsBuf;
    } else if (pl.fullTiles < tiles) {
        p.remChunk = (p.K + pl.remPieces - 1) / pl.remPieces;
        p.remChunk = (p.remChunk + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
        p.remPieces = (p.K + p.remChunk - 1) / p.remChunk;
        p.fullTiles = pl.fullTiles;
        p.rws = wsBuf;
        gridX = p.fullTiles + (tiles - p.fullTiles) * p.remPieces;
    }
    const bool va = (p.K % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.w) & 15u) == 0);
    const int khw = p.KH * p.KW;
    // an unpadded 1x1 kernel whose grid stays inside the image never gathers a padding tap
    const bool inside = p.KH == 1 && p.KW == 1 && p.padH == 0 && p.padW == 0 &&
                        (long long)(p.Ho - 1) * p.stride < p.H && (long long)(p.Wo - 1) * p.stride < p.W;
    const int mode = inside ? 3 : gatherMode(khw);
    int rc;
    if (va)
        rc = mode == 3 ? launchConvT<Cfg, true, 3>(p, gridX)
           : mode == 0 ? launchConvT<Cfg, true, 0>(p, gridX)
                       : (mode == 1 ? launchConvT<Cfg, true, 1>(p, gridX) : launchConvT<Cfg, true, 2>(p, gridX));
    else
        rc = mode == 3 ? launchConvT<Cfg, false, 3>(p, gridX)
           : mode == 0 ? launchConvT<Cfg, false, 0>(p, gridX)
                       : (mode == 1 ? launchConvT<Cfg, false, 1>(p, gridX) : launchConvT<Cfg, false, 2>(p, gridX));
    return rc;
}

// Workspace of a plan's partial sums and the tiles' arrival counters. A plan
// whose buffers cannot be had runs whole tiles (out of memory), or fails while
// the stream records a graph (workspace() recorded why).
static int planBuffers(ConvParams& p, ConvPlan& pl, int tiles, int bm, int bn, float*& ws) {
    ws = nullptr;
    p.ctr = nullptr;
    size_t bytes = 0;
    if (pl.splits > 1)
        bytes = (size_t)pl.splits * p.Cout * p.Nq * sizeof(float);
    else if (pl.fullTiles < tiles)
        bytes = (size_t)(tiles - pl.fullTiles) * pl.remPieces * bm * bn * sizeof(float);
    else
        return 0;
    ws = static_cast<float*>(workspace(bytes));
    unsigned* ctr = ws ? static_cast<unsigned*>(workspace((size_t)tiles * sizeof(unsigned), kWsCounters)) : nullptr;
    if (!ws || !ctr) {
        if (capturing(stream())) return -1;
        clearError();   // the whole-tile plan below succeeds: drop workspace()'s out-of-memory note
        pl.splits = 1;
        pl.fullTiles = tiles;
        ws = nullptr;
        return 0;
    }
    p.ctr = ctr;
    return 0;
}

// ---- tap tables, cached per (Cin, H, W, KH, KW) -------------------------------
static std::mutex g_tabMutex;
static std::map<std::tuple<int, int, int, int, int>, uint2*> g_tabs;

static void dropTapTables() {
    std::lock_guard<std::mutex> lock(g_tabMutex);
    g_tabs.clear();   // the pool that owned them is being cleared
}

static const uint2* tapTable(int Cin, int H, int W, int KH, int KW) {
    std::lock_guard<std::mutex> lock(g_tabMutex);
    static bool s_hooked = false;
    if (!s_hooked) {
        onCleanup(dropTapTables);
        s_hooked = true;
    }
    const auto key = std::make_tuple(Cin, H, W, KH, KW);
    auto it = g_tabs.find(key);
    if (it != g_tabs.end()) return it->second;
    const int K = Cin * KH * KW;
    const int Kpad = (K + 63) / 64 * 64 + 64;   // room for any slice that starts before K
    void* mem = nullptr;
    if (omHipMalloc(&mem, (size_t)Kpad * sizeof(uint2)) != 0) return nullptr;
    uint2* tab = static_cast<uint2*>(mem);
    if (capturing(stream())) {
        (void)omHipFree(mem);
        (void)publish(stream(), "conv tap table");
        return nullptr;
    }
    hipLaunchKernelGGL(build_tap_table, dim3((Kpad + 255) / 256), dim3(256), 0, stream(), tab, K, Kpad, KH, KW, H, W,
                       gatherMode(KH * KW));
    // complete before any stream reads it
    if (hipGetLastError() != hipSuccess || publish(stream(), "conv tap table")) {
        (void)omHipFree(mem);
        return nullptr;
    }
    g_tabs.emplace(key, tab);
    return tab;
}

// Buffer-view limits shared by every conv launch: one image with its border
// margin, one image's output and the weights fit a view (the batch is split
// into chunks that do), pixel indices stay below 2^30, and KH, KW < 2^16 and
// H + pad, W + pad < 65535 for the tap codes.
static int checkConvLimits(const char* name, int Cin, int H, int W, int Cout, int KH, int KW, int padH, int padW,
                           long long outPerImage) {
    const long long K = (long long)Cin * KH * KW;
    const long long margin = (long long)std::max(padH, 0) * W + std::max(padW, 0);
    const long long imgBytes = (long long)Cin * H * W * 4 + 8LL * (margin + W + 1);
    if (K > (1LL << 26) || imgBytes > (long long)kMaxBufferBytes / 2 || (long long)Cout * K * 4 > kMaxBufferBytes ||
        outPerImage > (long long)kMaxBufferBytes / 4 || H + std::abs(padH) >= 65535 || W + std::abs(padW) >= 65535 || KH >= 65536 ||
        KW >= 65536)
        return fail("%s: tensor exceeds the 2^30-byte buffer range of this kernel", name);
    return 0;
}

static int validateConv(const char* name, const float* x, const float* w, float* out, int N, int Cin, int H, int W,
                        int Cout, int KH, int KW, int stride, int pad, int& Ho, int& Wo) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0)
        return fail("%s: invalid geometry", name);
    if (!x || !w || !out) return fail("%s: null pointer", name);
    Ho = (H + 2 * pad - KH) / stride + 1;
    Wo = (W + 2 * pad - KW) / stride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("%s: kernel larger than the padded input", name);
    return checkConvLimits(name, Cin, H, W, Cout, KH, KW, pad, pad, (long long)Cout * Ho * Wo);
}

static int convChunk(ConvParams p, int n0, int nb) {
    // one batch chunk: x, out and the pixel axis restricted to images [n0, n0+nb)
    p.x = p.x + (long long)n0 * p.Cin * p.H * p.W;
    p.out = p.out + (long long)n0 * p.Cout * p.oH * p.oW;
    if (p.res) p.res = p.res + (long long)n0 * p.Cout * p.oH * p.oW;
    p.N = nb;
    if (p.oStride == 1 && p.oOffH == 0 && p.oOffW == 0 && p.oH == p.Ho && p.oW == p.Wo &&
        stemGeometry(p.Cin, p.W, p.KH, p.KW, p.stride, p.padH, p.padW))
        return convStem(p.x, p.w, p.bias, p.gamma, p.beta, p.mean, p.var, p.eps, p.res, p.act, p.out, nb, p.H, p.W,
                        p.Cout, p.Ho, p.Wo);
    p.Nq = nb * p.Ho * p.Wo;
    p.padOff = std::max(p.padH, 0) * p.W + std::max(p.padW, 0);
    p.xBytes = (uint32_t)(((long long)nb * p.Cin * p.H * p.W + p.padOff) * 4);
    p.tilesM = (p.Cout + ConvCfg::BM - 1) / ConvCfg::BM;
    p.tilesN = (p.Nq + ConvCfg::BN - 1) / ConvCfg::BN;
    // Split-K workspace only for outputs up to 64 MiB (late layers, where splitting pays).
    const bool wsOk = (size_t)p.Cout * p.Nq * sizeof(float) <= ((size_t)64 << 20);
    ConvPlan pl = planConv(p, wsOk);
    float* ws = nullptr;
    if (planBuffers(p, pl, p.tilesM * p.tilesN, ConvCfg::BM, ConvCfg::BN, ws)) return -1;
    return launchConv(p, pl, ws);
}

// Walks the batch in chunks whose x view stays below 2^29 bytes, whose pixel
// indices stay below 2^30 and whose output (and residual) view is at most 2^30
// bytes.
static int runConv(const char* name, ConvParams& p) {
    p.K = p.Cin * p.KH * p.KW;
    p.dHoWo = FastDiv::make((uint32_t)(p.Ho * p.Wo));
    p.dWo = FastDiv::make((uint32_t)p.Wo);
    p.rowRep = 0;
    if (p.KH * p.KW <= 63)
        for (int rr = 0; rr < p.KH; ++rr) p.rowRep |= 1ull << (rr * p.KW);
    p.tab = tapTable(p.Cin, p.H, p.W, p.KH, p.KW);
    if (!p.tab) {
        if (capturing(stream())) return -1;   // tapTable recorded why
        return fail("%s: could not build the tap table", name);
    }
    const long long perImg = (long long)p.Cin * p.H * p.W * 4;
    long long chunk = std::max<long long>(1, ((long long)kMaxBufferBytes / 2) / perImg);
    chunk = std::min<long long>(chunk, std::max<long long>(1, (1LL << 30) / ((long long)p.Cout * p.Ho * p.Wo)));
    chunk = std::min<long long>(chunk,
                              std::max<long long>(1, ((long long)kMaxBufferBytes / 4) / ((long long)p.Cout * p.oH * p.oW)));
    for (int n0 = 0; n0 < p.N; n0 += (int)chunk) {
        const int nb = (int)std::min<long long>(chunk, p.N - n0);
        if (convChunk(p, n0, nb)) return -1;
    }
    return 0;
}

int conv2dFused(const char* name, const float* x, const float* w, const float* bias, const float* gamma,
                const float* beta, const float* mean, const float* var, float eps, const float* res, int act,
                float* out, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    clearError();
    int Ho, Wo;
    if (validateConv(name, x, w, out, N, Cin, H, W, Cout, KH, KW, stride, pad, Ho, Wo)) return -1;
    const bool anyBn = gamma || beta || mean || var;
    if (anyBn && !(gamma && beta && mean && var)) return fail("%s: BN needs gamma, beta, mean and var", name);
    if (act != 0 && act != 1) return fail("%s: unknown activation %d", name, act);
    ConvParams p{};
    p.x = x; p.w = w; p.bias = bias;
    p.gamma = anyBn ? gamma : nullptr; p.beta = beta; p.mean = mean; p.var = var;
    p.eps = eps; p.act = act; p.res = res; p.out = out;
    p.N = N; p.Cin = Cin; p.H = H; p.W = W; p.Cout = Cout; p.KH = KH; p.KW = KW;
    p.stride = stride; p.padH = pad; p.padW = pad; p.Ho = Ho; p.Wo = Wo;
    p.oH = Ho; p.oW = Wo; p.oStride = 1; p.oOffH = 0; p.oOffW = 0;
    return runConv(name, p);
}

int conv2dToGrid(const char* name, const float* x, const float* w, float* out, int N, int Cin, int H, int W, int Cout,
                 int KH, int KW, int padH, int padW, int Ho, int Wo, int oH, int oW, int oStride, int oOffH,
                 int oOffW) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || Ho <= 0 || Wo <= 0 ||
        oStride <= 0 || oOffH < 0 || oOffW < 0 || (Ho - 1) * oStride + oOffH >= oH ||
        (Wo - 1) * oStride + oOffW >= oW)
        return fail("%s: invalid grid geometry", name);
    if (!x || !w || !out) return fail("%s: null pointer", name);
    if (checkConvLimits(name, Cin, H, W, Cout, KH, KW, padH, padW, (long long)Cout * oH * oW)) return -1;
    ConvParams p{};
    p.x = x; p.w = w; p.out = out;
    p.N = N; p.Cin = Cin; p.H = H; p.W = W; p.Cout = Cout; p.KH = KH; p.KW = KW;
    p.stride = 1; p.padH = padH; p.padW = padW; p.Ho = Ho; p.Wo = Wo;
    p.oH = oH; p.oW = oW; p.oStride = oStride; p.oOffH = oOffH; p.oOffW = oOffW;
    return runConv(name, p);
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipConv2d(const float* pInput, const float* pWeight, const float* pBias, float* pOutput, int nBatch, int nCin,
                int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    return conv2dFused("omHipConv2d", pInput, pWeight, pBias, nullptr, nullptr, nullptr, nullptr, 0.f, nullptr, 0,
                       pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad);
}

int omHipConv2dBiasBnAct(const float* pInput, const float* pWeight, const float* pBias, const float* pGamma,
                         const float* pBeta, const float* pMean, const float* pVar, float fEps, int nAct,
                         float* pOutput, int nBatch, int nCin, int nH, int nW, int nCout, int nKH, int nKW,
                         int nStride, int nPad) {
    return conv2dFused("omHipConv2dBiasBnAct", pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps, nullptr,
                       nAct, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad);
}

int omHipConv2dBiasBnAddAct(const float* pInput, const float* pWeight, const float* pBias, const float* pGamma,
                            const float* pBeta, const float* pMean, const float* pVar, float fEps,
                            const float* pResidual, int nAct, float* pOutput, int nBatch, int nCin, int nH, int nW,
                            int nCout, int nKH, int nKW, int nStride, int nPad) {
    if (!pResidual) {
        clearError();
        return fail("omHipConv2dBiasBnAddAct: null residual");
    }
    if (pResidual == pOutput) {
        clearError();
        return fail("omHipConv2dBiasBnAddAct: the residual must not alias the output");
    }
    return conv2dFused("omHipConv2dBiasBnAddAct", pInput, pWeight, pBias, pGamma, pBeta, pMean, pVar, fEps,
                       pResidual, nAct, pOutput, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad);
}

// Explicit lowering: im2col of every image into one buffer, then a batched
// GEMM with the weight shared across the batch (A stride 0), then bias.
int omHipConv2dIm2col(const float* pInput, const float* pWeight, const float* pBias, float* pOutput, int nBatch,
                      int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    clearError();
    if (nBatch <= 0 || nCin <= 0 || nH <= 0 || nW <= 0 || nCout <= 0 || nKH <= 0 || nKW <= 0 || nStride <= 0 ||
        nPad < 0)
        return fail("omHipConv2dIm2col: invalid geometry");
    if (!pInput || !pWeight || !pOutput) return fail("omHipConv2dIm2col: null pointer");
    const int Ho = (nH + 2 * nPad - nKH) / nStride + 1;
    const int Wo = (nW + 2 * nPad - nKW) / nStride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("omHipConv2dIm2col: kernel larger than the padded input");
    const long long K = (long long)nCin * nKH * nKW;
    const long long HWo = (long long)Ho * Wo;
    if (K > (1LL << 30) || HWo > (1LL << 30)) return fail("omHipConv2dIm2col: tensor too large");
    void* col = workspace((size_t)nBatch * K * HWo * sizeof(float), kWsOperand);
    if (!col) return -1;   // workspace() recorded the cause
    int rc = im2colBatched(pInput, static_cast<float*>(col), nBatch, nCin, nH, nW, nKH, nKW, nPad, nStride, Ho, Wo);
    if (!rc)
        rc = gemmF32(false, false, nBatch, nCout, (int)HWo, (int)K, pWeight, K, 0, static_cast<const float*>(col), HWo,
                     K * HWo, pOutput, HWo, (long long)nCout * HWo);
    if (!rc && pBias) rc = omHipAddBias(pOutput, pBias, pOutput, nBatch, nCout, (int)HWo);
    return rc;
}

}  // extern "C"
