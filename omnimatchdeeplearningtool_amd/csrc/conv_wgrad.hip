// conv_wgrad.hip — conv2d weight gradient as an implicit GEMM on fp32 MFMA.
//
//   gW[co][kk] = sum_q gO^[co][q] * X^[kk][q]
//   kk = (ci*KH + kh)*KW + kw          (the reference im2col row order, cpu_backend.ixx:554-557)
//   q  = n*Ho*Wo + oh*Wo + ow          (every output pixel of every image: the reduction axis)
//   gO^[co][q] = gradOutput[n][co][oh][ow]
//   X^[kk][q]  = x[n][ci][oh*s-p+kh][ow*s-p+kw], zero outside the image
//
// The reference runs im2col per image and accumulates gradOutput[n] x col^T
// into the weight gradient (cpu_backend.ixx:714-772). Here the column matrix
// is never written: both operands are read from the tensors themselves.
//
//   gO slice (A, [BM co][BK q] in LDS): each thread owns fixed (co, q-offset)
//   positions, so consecutive lanes read consecutive pixels. The image index
//   of pixel q is q / (Ho*Wo), computed with a multiply-shift.
//
//   x slice (B, [BN kk][BK q] in LDS): each lane owns one column kk (its tap's
//   byte offset is fixed for the whole walk) and the rows of a wave are
//   uniform, so the per-pixel data — the byte offset of the pixel's window in
//   x and its "tap outside the image" mask — is one scalar load per row from a
//   pixel table. A padding tap costs the lane a bit extract and a shift-or that
//   pushes its offset past the buffer end, where the hardware range check
//   returns 0.
//
// The reduction axis is long (N*Ho*Wo) and the output small (Cout x Kc), so
// the pixel axis is split; each split writes a partial tile
// and a second kernel adds the partials in a fixed order (deterministic).
#include "omhip_internal.hpp"
#include "mfma_f32_tile.hpp"
#include "buffer_io.hpp"
#include "conv.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace omhip {

struct WgradParams {
    const float* x;       // [N][Cin][H][W] (this batch chunk)
    const float* gO;      // [N][Cout][Ho][Wo]
    float* dst;           // splits == 1: gW [Cout][Kc]; else partials [splits][Cout][Kc]
    const uint4* ptab;    // per pixel q: (x byte offset, mask lo / iw0, mask hi / ih0, 0); null for plane x
    int Cin, H, W, Cout, KH, KW;
    int Kc;               // Cin*KH*KW
    int Nq;               // pixels of this chunk
    int HWo;
    int tilesM, tilesN;
    int splits;
    int qChunk;           // pixels per split (multiple of BK)
    int accumulate;       // splits == 1 only: dst += instead of dst =
    int padOff;           // the x view starts pad*W + pad floats before x
    uint32_t xBytes;      // range of the x view
    uint32_t gBytes;      // range of gO
    uint32_t divMul, divShift;   // q / HWo == (q * divMul) >> divShift for q < 2^31
};

// Pixel table. Entry q < Nq: .x = 4*(n*Cin*H*W + ih0*W + iw0 + padOff) with
// ih0 = oh*s - pad, iw0 = ow*s - pad (never negative thanks to padOff); for the
// mask modes .y/.z = bits of the taps t = kh*KW + kw that fall outside the
// image, for the compare mode .y = iw0, .z = ih0. Entries past Nq (slices that
// run past the last pixel) mark every tap outside: .x = 0, masks all ones, or
// ih0 = iw0 = -2^29.
__global__ void build_pixel_table(uint4* tab, int Nq, int Nqpad, int Cin, int H, int W, int KH, int KW, int stride,
                                  int pad, int Ho, int Wo, int mode) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Nqpad) return;
    uint4 e;
    e.w = 0;
    if (q < Nq) {
        const int HWo = Ho * Wo;
        const int n = q / HWo;
        const int pix = q - n * HWo;
        const int oh = pix / Wo;
        const int ow = pix - oh * Wo;
        const int ih0 = oh * stride - pad, iw0 = ow * stride - pad;
        e.x = (uint32_t)((long long)n * Cin * H * W + (long long)ih0 * W + iw0 + (long long)pad * W + pad) * 4u;
        if (mode == 2) {
            e.y = (uint32_t)iw0;
            e.z = (uint32_t)ih0;
        } else {
            uint64_t colBits = 0, inside = 0;
            for (int c = 0; c < KW; ++c)
                if ((unsigned)(iw0 + c) < (unsigned)W) colBits |= 1ull << c;
            for (int r = 0; r < KH; ++r)
                if ((unsigned)(ih0 + r) < (unsigned)H) inside |= colBits << (r * KW);
            e.y = ~(uint32_t)inside;
            e.z = ~(uint32_t)(inside >> 32);
        }
    } else {
        e.x = 0;
        e.y = e.z = mode == 2 ? (uint32_t)(-(1 << 29)) : 0xffffffffu;
    }
    tab[q] = e;
}

// Plane loader -> LDS [R][BK+4] (q contiguous) for a tensor laid out
// [image][row][Ho*Wo]: gO (rows = Cout) and, for 1x1 stride-1 unpadded convs,
// x itself (rows = Cin). Each thread owns fixed (row, q-offset) positions, so
// consecutive lanes read consecutive pixels. VEC: 4 consecutive pixels per
// load; the host enables it when Ho*Wo % 4 == 0 and the tensor is 16-byte
// aligned, so a group of 4 never straddles two images. Rows past the tensor
// and pixels past the chunk land past the buffer end (zero).
template <int R, int BK, int NT, bool VEC>
struct PlaneLoader {
    static constexpr int PER_T = VEC ? R * BK / 4 / NT : R * BK / NT;
    static_assert(R * BK % (NT * (VEC ? 4 : 1)) == 0, "slice must split evenly");
    using Shape = LdsShape<true, R, BK>;
    __amdgpu_buffer_rsrc_t r;
    uint32_t rowOff[PER_T];
    uint32_t mul, shift, step;
    f32x4 v4[VEC ? PER_T : 1];
    float v1[VEC ? 1 : PER_T];

    static __device__ __forceinline__ void coords(int e, int& row, int& k) {
        if constexpr (VEC) { row = e / (BK / 4); k = (e % (BK / 4)) * 4; }
        else { row = e / BK; k = e % BK; }
    }

    // rows: valid rows of the tensor; r0: first row of the tile.
    __device__ void init(const WgradParams& p, const float* base, uint32_t bytes, int rows, int r0, int tid) {
        r = bufferRsrc(base, bytes);
        mul = p.divMul; shift = p.divShift;
        step = (uint32_t)((rows - 1) * p.HWo) * 4u;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int row, k;
            coords(tid + i * NT, row, k);
            rowOff[i] = (r0 + row < rows) ? (uint32_t)((r0 + row) * p.HWo) * 4u : kOOB;
        }
    }

    __device__ void load(int q0, int tid) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int row, k;
            coords(tid + i * NT, row, k);
            const uint32_t q = (uint32_t)(q0 + k);
            const uint32_t n = (uint32_t)(((uint64_t)q * mul) >> shift);
            const uint32_t off = rowOff[i] + 4u * q + n * step;
            if constexpr (VEC) v4[i] = bufLoad4(r, off, 0);
            else v1[i] = bufLoad1(r, off, 0);
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

// x as a plane operand (1x1 kernel, stride 1, no padding: X^[ci][q] = x[n][ci][pix]).
template <int BN, int BK, int NT, bool VEC>
struct DenseXLoader : PlaneLoader<BN, BK, NT, VEC> {
    __device__ void init(const WgradParams& p, int n0, int tid) {
        PlaneLoader<BN, BK, NT, VEC>::init(p, p.x, p.xBytes, p.Cin, n0, tid);
    }
};

// x tap loader -> LDS [BN][BK+4] (q contiguous). Thread t owns column
// c = t % BN and rows g*RPT .. g*RPT+RPT-1 of each slice (g = t / BN, uniform
// across a wave since BN >= 64); its RPT values are contiguous in the LDS row.
// MODE = gatherMode(KH*KW).
template <int BN, int BK, int NT, int MODE>
struct TapLoader {
    static constexpr int TPC = NT / BN;
    static constexpr int RPT = BK / TPC;
    static_assert(NT % BN == 0 && BK % TPC == 0 && BN >= 64 && RPT % 4 == 0, "tap loader mapping");
    using Shape = LdsShape<true, BN, BK>;
    __amdgpu_buffer_rsrc_t r;
    uint32_t tapOff;
    uint32_t tap;      // mask modes: kh*KW + kw
    int kh, kw, H, W;  // compare mode
    const uint4* tab;
    float v[RPT];

    __device__ void init(const WgradParams& p, int n0, int tid) {
        const int kk = n0 + tid % BN;
        r = bufferRsrc(p.x - p.padOff, p.xBytes);
        tab = p.ptab;
        H = p.H; W = p.W;
        const int khw = p.KH * p.KW;
        const bool valid = kk < p.Kc;
        const int kc = valid ? kk : 0;
        const int ci = kc / khw;
        const int t = kc - ci * khw;
        kh = t / p.KW;
        kw = t - kh * p.KW;
        tap = (uint32_t)t;
        tapOff = valid ? (uint32_t)(ci * p.H * p.W + kh * p.W + kw) * 4u : kOOB;
    }

    __device__ void load(int q0, int tid) {
        const int base = __builtin_amdgcn_readfirstlane(q0 + (tid / BN) * RPT);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const uint4 e = tab[base + j];
            uint32_t inv;
            if constexpr (MODE == 0) {
                inv = __builtin_amdgcn_ubfe(e.y, tap, 1);
            } else if constexpr (MODE == 1) {
                inv = (uint32_t)((((uint64_t)e.z << 32) | e.y) >> tap) & 1u;
            } else {
                inv = ((unsigned)((int)e.z + kh) >= (unsigned)H) | ((unsigned)((int)e.y + kw) >= (unsigned)W);
            }
            v[j] = bufLoad1(r, (inv << 30) | tapOff, e.x);
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

// x pixel loader -> LDS [BN][BK+4] for kernels of at most 31 taps: lanes run
// along the pixel axis (thread t owns q-offset k = t % BK and the columns
// c = t / BK + j * NT/BK), so a wave reads 16 consecutive pixels of 4 tap rows
// instead of 64 tap rows of one pixel. Each lane reads its pixel's table entry
// itself, one slice ahead of use, so the table latency hides behind a slice of
// MFMAs. Pays for 1x1 kernels, whose 64 tap rows are 64 channel planes.
template <int BN, int BK, int NT>
struct PixelLoader {
    static constexpr int CPT = BN * BK / NT;   // columns per thread
    static constexpr int CSTEP = NT / BK;
    static_assert(NT % BK == 0 && BN % CSTEP == 0, "pixel loader mapping");
    using Shape = LdsShape<true, BN, BK>;
    __amdgpu_buffer_rsrc_t r;
    uint32_t tapOff[CPT];
    uint32_t tap[CPT];
    const uint4* tab;
    uint4 next;        // table entry of the pixel this thread loads next
    float v[CPT];

    __device__ void init(const WgradParams& p, int n0, int tid) {
        r = bufferRsrc(p.x - p.padOff, p.xBytes);
        tab = p.ptab;
        const int khw = p.KH * p.KW;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int kk = n0 + tid / BK + j * CSTEP;
            const bool valid = kk < p.Kc;
            const int kc = valid ? kk : 0;
            const int ci = kc / khw;
            const int t = kc - ci * khw;
            const int kh = t / p.KW;
            const int kw = t - kh * p.KW;
            tap[j] = (uint32_t)t;
            tapOff[j] = valid ? (uint32_t)(ci * p.H * p.W + kh * p.W + kw) * 4u : kOOB;
        }
    }

    // The first slice's entry; later ones are fetched by load().
    __device__ void start(int q0, int tid) { next = tab[q0 + tid % BK]; }

    __device__ void load(int q0, int tid) {
        const uint4 e = next;
        next = tab[q0 + BK + tid % BK];   // at most 2*BK entries past the split: inside the padded table
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint32_t inv = __builtin_amdgcn_ubfe(e.y, tap[j], 1);
            v[j] = bufLoad1(r, (inv << 30) | (e.x + tapOff[j]), 0);
        }
    }

    __device__ void store(float* s, int tid) const {
        const int k = tid % BK, c0 = tid / BK;
#pragma unroll
        for (int j = 0; j < CPT; ++j) s[(c0 + j * CSTEP) * Shape::LD + k] = v[j];
    }
};

// Loader choice for the x operand.
enum WgradXKind { kXTaps0 = 0, kXTaps1 = 1, kXTaps2 = 2, kXPixels = 3, kXDense = 4, kXDenseVec = 5 };

template <class Cfg, int XK>
struct XLoaderFor;
template <class Cfg> struct XLoaderFor<Cfg, kXTaps0> { using T = TapLoader<Cfg::BN, Cfg::BK, Cfg::NT, 0>; };
template <class Cfg> struct XLoaderFor<Cfg, kXTaps1> { using T = TapLoader<Cfg::BN, Cfg::BK, Cfg::NT, 1>; };
template <class Cfg> struct XLoaderFor<Cfg, kXTaps2> { using T = TapLoader<Cfg::BN, Cfg::BK, Cfg::NT, 2>; };
template <class Cfg> struct XLoaderFor<Cfg, kXPixels> { using T = PixelLoader<Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg> struct XLoaderFor<Cfg, kXDense> { using T = DenseXLoader<Cfg::BN, Cfg::BK, Cfg::NT, false>; };
template <class Cfg> struct XLoaderFor<Cfg, kXDenseVec> { using T = DenseXLoader<Cfg::BN, Cfg::BK, Cfg::NT, true>; };

template <class L>
__device__ __forceinline__ void startLoader(L& l, int q0, int tid) {
    if constexpr (requires { l.start(q0, tid); }) l.start(q0, tid);
}

template <class Cfg, bool VA, int XK>
__global__ __launch_bounds__(Cfg::NT) void conv_wgrad_kernel(WgradParams p) {
    using SA = LdsShape<true, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<true, Cfg::BN, Cfg::BK>;
    constexpr int STAGE = SA::SIZE + SB::SIZE;
    __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N;
    const int wn = wave % Cfg::WAVES_N;

    // One linear grid over (split, tile) with the split outermost, remapped so
    // each XCD runs whole splits: the tiles of a split read the same pixel range
    // of x and gO, and then read it through one L2.
    const int tiles = p.tilesM * p.tilesN;
    const int lin = xcd_remap(blockIdx.x, tiles * p.splits);
    const int split = lin / tiles;
    const int t = lin - split * tiles;
    const int m0 = (t % p.tilesM) * Cfg::BM;
    const int n0 = (t / p.tilesM) * Cfg::BN;
    const int qBeg = split * p.qChunk;
    const int qEnd = min(p.Nq, qBeg + p.qChunk);

    PlaneLoader<Cfg::BM, Cfg::BK, Cfg::NT, VA> la;
    la.init(p, p.gO, p.gBytes, p.Cout, m0, tid);
    typename XLoaderFor<Cfg, XK>::T lb;
    lb.init(p, n0, tid);

    f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // qChunk is a multiple of BK, so only the chunk's last slice can run past
    // Nq; the pixel table and the gO range check zero those pixels.
    const int nk = (qEnd - qBeg + Cfg::BK - 1) / Cfg::BK;
    startLoader(lb, qBeg, tid);
    lb.load(qBeg, tid);
    la.load(qBeg, tid);
    la.store(smem, tid);
    lb.store(smem + SA::SIZE, tid);
    __syncthreads();
    // Two slices per trip so both LDS stage addresses are compile-time offsets.
    for (int t = 0; t < nk; t += 2) {
        {
            const bool more = (t + 1) < nk;
            if (more) {
                lb.load(qBeg + (t + 1) * Cfg::BK, tid);
                la.load(qBeg + (t + 1) * Cfg::BK, tid);
            }
            mma_slice<Cfg, true, true>(smem, smem + SA::SIZE, acc, wm, wn, lane);
            if (more) {
                la.store(smem + STAGE, tid);
                lb.store(smem + STAGE + SA::SIZE, tid);
            }
            __syncthreads();
        }
        if (t + 1 < nk) {
            const bool more = (t + 2) < nk;
            if (more) {
                lb.load(qBeg + (t + 2) * Cfg::BK, tid);
                la.load(qBeg + (t + 2) * Cfg::BK, tid);
            }
            mma_slice<Cfg, true, true>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane);
            if (more) {
                la.store(smem, tid);
                lb.store(smem + SA::SIZE, tid);
            }
            __syncthreads();
        }
    }

    const int li = lane & 31, h = lane >> 5;
    float* dst = p.dst + (long long)split * p.Cout * p.Kc;
#pragma unroll
    for (int fn = 0; fn < Cfg::FN; ++fn) {
        const int kk = n0 + wn * Cfg::WN + fn * 32 + li;
        if (kk >= p.Kc) continue;
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (co >= p.Cout) continue;
                float* o = dst + (long long)co * p.Kc + kk;
                *o = p.accumulate ? *o + acc[fm][fn][r] : acc[fm][fn][r];
            }
    }
}

// out[i] (+)= sum over s of part[s][i]. Each element is summed by G threads
// (thread g takes splits g, g+G, ...; its loads are issued 4 at a time) and
// the G results are added in g order: a fixed order, so the result does not
// depend on timing. Many splits over few elements (small weight tensors) take
// G = 16 so enough loads are in flight. VEC (total % 4 == 0, 16-byte aligned
// buffers): a thread takes four consecutive elements with one 16-byte load
// per split; each element's sum is formed in the same order as without VEC.
template <int G, bool VEC>
__global__ __launch_bounds__(256) void splits_sum_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                         long long total, int splits, int accumulate) {
    constexpr int E = 256 / G;
    constexpr int W = VEC ? 4 : 1;   // elements per thread
    __shared__ f32x4 red[G][E];
    const int e = threadIdx.x % E, g = threadIdx.x / E;
    for (long long base = blockIdx.x * (long long)(E * W); base < total; base += (long long)gridDim.x * E * W) {
        const long long i = base + (long long)e * W;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (i < total) {
            auto ld = [&](int s) -> f32x4 {
                if constexpr (VEC) return *reinterpret_cast<const f32x4*>(part + (long long)s * total + i);
                else return f32x4{part[(long long)s * total + i], 0.f, 0.f, 0.f};
            };
            int s = g;
            for (; s + 3 * G < splits; s += 4 * G) {
                const f32x4 a = ld(s), b = ld(s + G), c = ld(s + 2 * G), d = ld(s + 3 * G);
                v += a; v += b; v += c; v += d;
            }
            for (; s < splits; s += G) v += ld(s);
        }
        red[g][e] = v;
        __syncthreads();
        if (g == 0 && i < total) {
            f32x4 r = red[0][e];
#pragma unroll
            for (int k = 1; k < G; ++k) r += red[k][e];
#pragma unroll
            for (int w = 0; w < W; ++w) out[i + w] = accumulate ? out[i + w] + r[w] : r[w];
        }
        __syncthreads();
    }
}

template <int G>
static int launchSplitsSum(const float* part, float* out, long long total, int splits, bool accumulate) {
    constexpr int E = 256 / G;
    const bool vec = total % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    const int w = vec ? 4 : 1;
    const long long blocks = std::min<long long>((total + E * w - 1) / (E * w), (long long)cuCount() * 16);
    if (vec)
        hipLaunchKernelGGL((splits_sum_kernel<G, true>), dim3((unsigned)blocks), dim3(256), 0, stream(), part, out,
                           total, splits, accumulate ? 1 : 0);
    else
        hipLaunchKernelGGL((splits_sum_kernel<G, false>), dim3((unsigned)blocks), dim3(256), 0, stream(), part, out,
                           total, splits, accumulate ? 1 : 0);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// ---- tile configuration -------------------------------------------------------
#ifndef OMHIP_WGRAD_TILE
#define OMHIP_WGRAD_TILE 64, 64, 32, 32   // BM, BN, WM, WN
#endif
#ifndef OMHIP_WGRAD_BK
#define OMHIP_WGRAD_BK 16
#endif
template <int BM, int BN, int WM, int WN>
using WgradCfgT = TileCfg<BM, BN, OMHIP_WGRAD_BK, WM, WN>;
using WgradCfg = WgradCfgT<OMHIP_WGRAD_TILE>;

template <class Cfg, bool VA, int XK>
static int launchWgradT(const WgradParams& p, int splits) {
    hipLaunchKernelGGL((conv_wgrad_kernel<Cfg, VA, XK>), dim3(p.tilesM * p.tilesN * splits), dim3(Cfg::NT), 0,
                       stream(), p);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <bool VA>
static int launchWgrad(const WgradParams& p, int splits, int xk) {
    using Cfg = WgradCfg;
    switch (xk) {
    case kXTaps0: return launchWgradT<Cfg, VA, kXTaps0>(p, splits);
    case kXTaps1: return launchWgradT<Cfg, VA, kXTaps1>(p, splits);
    case kXTaps2: return launchWgradT<Cfg, VA, kXTaps2>(p, splits);
    case kXPixels: return launchWgradT<Cfg, VA, kXPixels>(p, splits);
    case kXDense: return launchWgradT<Cfg, VA, kXDense>(p, splits);
    default: return launchWgradT<Cfg, VA, kXDenseVec>(p, splits);
    }
}

// x loader: 1x1 stride-1 unpadded kernels read x as a plane (4-pixel vectors
// when Ho*Wo % 4 == 0 and x is 16-byte aligned); other 1x1 kernels read along
// pixels; larger kernels read along taps with the gather mode of their size.
static int xLoaderKind(int KH, int KW, int stride, int pad, long long HWo, const float* x) {
    if (KH == 1 && KW == 1 && stride == 1 && pad == 0)
        return (HWo % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0) ? kXDenseVec : kXDense;
    if (KH * KW == 1) return kXPixels;
    return gatherMode(KH * KW);
}

// q / d == (q * mul) >> shift for 0 <= q < 2^31 with l = ceil(log2 d),
// mul = floor(2^(31+l) / d) + 1 < 2^32 (Granlund & Montgomery 1994, Thm 4.2:
// 2^(31+l) < mul*d <= 2^(31+l) + 2^l).
static void magicDivisor(uint32_t d, uint32_t& mul, uint32_t& shift) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    mul = (uint32_t)((1ull << (31 + l)) / d + 1);
    shift = 31 + l;
}

// Pixel-axis splits: about 8 (tile, split) blocks per CU for kernels with
// several taps, 4 for 1x1 kernels (a tap-free split has fewer MFMAs per
// partial-sum byte), at least 4 slices per split and at most 256 MiB of
// partials. Measured on MI355X over the ResNet-18/50 weight gradients at batch
// 32 (e.g. 64x576x100352: 228 splits, 128x256x100352 1x1: 128 splits).
static int planWgradSplits(long long tiles, long long Nq, long long Cout, long long Kc, int taps) {
    const long long cus = cuCount();
    const long long target = (taps > 1 ? 8 : 4) * cus;
    long long s = (target + tiles - 1) / tiles;
    s = std::min(s, std::max(1LL, Nq / (4LL * WgradCfg::BK)));
    s = std::min(s, (long long)(((size_t)256 << 20) / ((size_t)Cout * Kc * sizeof(float))));
    return (int)std::max(1LL, s);
}

// ---- pixel tables, cached per (images, Cin, H, W, KH, KW, stride, pad) ----------
static std::mutex g_ptabMutex;
static std::map<std::tuple<int, int, int, int, int, int, int, int>, uint4*> g_ptabs;

static void dropPixelTables() {
    std::lock_guard<std::mutex> lock(g_ptabMutex);
    g_ptabs.clear();   // the pool that owned them is being cleared
}

static const uint4* pixelTable(int nb, int Cin, int H, int W, int KH, int KW, int stride, int pad, int Ho, int Wo) {
    std::lock_guard<std::mutex> lock(g_ptabMutex);
    static bool s_hooked = false;
    if (!s_hooked) {
        onCleanup(dropPixelTables);
        s_hooked = true;
    }
    const auto key = std::make_tuple(nb, Cin, H, W, KH, KW, stride, pad);
    auto it = g_ptabs.find(key);
    if (it != g_ptabs.end()) return it->second;
    const int Nq = nb * Ho * Wo;
    const int Nqpad = Nq + 64;   // room for the last slice of any split
    void* mem = nullptr;
    if (omHipMalloc(&mem, (size_t)Nqpad * sizeof(uint4)) != 0) return nullptr;
    uint4* tab = static_cast<uint4*>(mem);
    if (capturing(stream())) {
        (void)omHipFree(mem);
        (void)publish(stream(), "weight-gradient pixel table");
        return nullptr;
    }
    hipLaunchKernelGGL(build_pixel_table, dim3((Nqpad + 255) / 256), dim3(256), 0, stream(), tab, Nq, Nqpad, Cin, H,
                       W, KH, KW, stride, pad, Ho, Wo, gatherMode(KH * KW));
    // complete before any stream reads it
    if (hipGetLastError() != hipSuccess || publish(stream(), "weight-gradient pixel table")) {
        (void)omHipFree(mem);
        return nullptr;
    }
    g_ptabs.emplace(key, tab);
    return tab;
}

int conv2dWeightGrad(const char* name, const float* x, const float* gO, float* gW, int N, int Cin, int H, int W,
                     int Cout, int KH, int KW, int stride, int pad) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0)
        return fail("%s: invalid geometry", name);
    if (!x || !gO || !gW) return fail("%s: null pointer", name);
    const int Ho = (H + 2 * pad - KH) / stride + 1;
    const int Wo = (W + 2 * pad - KW) / stride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("%s: kernel larger than the padded input", name);
    const long long Kc = (long long)Cin * KH * KW;
    const long long HWo = (long long)Ho * Wo;
    // One image of x (with its border margin) and of gO must fit a buffer view;
    // the batch is walked in chunks that do.
    const long long padOff = (long long)pad * W + pad;
    const long long imgX = (long long)Cin * H * W * 4;
    const long long imgG = (long long)Cout * HWo * 4;
    if (Kc > (1LL << 26) || imgX + 4 * padOff > (1LL << 29) || imgG > (1LL << 28) || H + pad >= 65535 ||
        W + pad >= 65535)
        return fail("%s: tensor exceeds the 2^30-byte buffer range of this kernel", name);
    long long chunk = std::min<long long>({(long long)N, ((1LL << 29) - 4 * padOff) / imgX, (1LL << 28) / imgG,
                                           ((1LL << 30) - 64) / HWo});
    chunk = std::max(1LL, chunk);

    using Cfg = WgradCfg;
    WgradParams p{};
    p.Cin = Cin; p.H = H; p.W = W; p.Cout = Cout; p.KH = KH; p.KW = KW;
    p.Kc = (int)Kc;
    p.HWo = (int)HWo;
    p.padOff = (int)padOff;
    p.tilesM = (Cout + Cfg::BM - 1) / Cfg::BM;
    p.tilesN = (int)((Kc + Cfg::BN - 1) / Cfg::BN);
    magicDivisor((uint32_t)HWo, p.divMul, p.divShift);
    const int xk = xLoaderKind(KH, KW, stride, pad, HWo, x);
    const long long total = (long long)Cout * Kc;
    for (int n0 = 0; n0 < N; n0 += (int)chunk) {
        const int nb = (int)std::min<long long>(chunk, N - n0);
        p.x = x + (long long)n0 * Cin * H * W;
        p.gO = gO + (long long)n0 * Cout * HWo;
        p.Nq = (int)(nb * HWo);
        p.xBytes = (uint32_t)((long long)nb * imgX + 4 * padOff);
        p.gBytes = (uint32_t)((long long)nb * imgG);
        if (xk != kXDense && xk != kXDenseVec) {
            p.ptab = pixelTable(nb, Cin, H, W, KH, KW, stride, pad, Ho, Wo);
            if (!p.ptab) {
                if (capturing(stream())) return -1;   // pixelTable recorded why
                return fail("%s: could not build the pixel table", name);
            }
        }
        int splits = planWgradSplits((long long)p.tilesM * p.tilesN, p.Nq, Cout, Kc, KH * KW);
        float* ws = nullptr;
        if (splits > 1) {
            ws = static_cast<float*>(workspace((size_t)splits * total * sizeof(float)));
            if (!ws && capturing(stream())) return -1;
            if (!ws) splits = 1;   // out of memory: one pass without partials
        }
        p.qChunk = (p.Nq + splits - 1) / splits;
        p.qChunk = (p.qChunk + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
        splits = (p.Nq + p.qChunk - 1) / p.qChunk;
        p.splits = splits;
        p.dst = splits > 1 ? ws : gW;
        p.accumulate = (splits == 1 && n0 > 0) ? 1 : 0;
        const bool va = (HWo % 4 == 0) && ((reinterpret_cast<uintptr_t>(gO) & 15u) == 0);
        const int rc = va ? launchWgrad<true>(p, splits, xk) : launchWgrad<false>(p, splits, xk);
        if (rc) return rc;
        if (splits > 1) {
            const bool acc = n0 > 0;
            const int r = splits >= 64 ? launchSplitsSum<16>(ws, gW, total, splits, acc)
                                       : (splits >= 8 ? launchSplitsSum<4>(ws, gW, total, splits, acc)
                                                      : launchSplitsSum<1>(ws, gW, total, splits, acc));
            if (r) return r;
        }
    }
    return 0;
}

}  // namespace omhip
