// train.hip — the training half of the conv / BatchNorm path:
// conv2d input and weight gradients, BatchNorm2d training statistics and its
// backward pass.
//
// Reference: CPUBackend::conv2dBackwardInput / conv2dBackwardWeight
// (src/hal/om.hal.cpu_backend.ixx:666-772), batchNorm2d's training branch
// (:796-822) and batchNorm2dBackward (:847-890); C ABI counterparts
// omCudaConv2dBackwardInput / Weight and omCudaBatchNorm2dBackward
// (src/cuda/cuda_kernels.cuh:295-316).
//
// Input gradient. For stride 1 it is itself a stride-1 convolution of the
// output gradient with the weights swapped over (Cout, Cin) and flipped in
// (kh, kw), padded by K-1-pad: it runs on the forward implicit-GEMM kernel.
// A stride-s gradient splits into s*s output phases (ih mod s, iw mod s),
// each again a stride-1 convolution of the output gradient with a flipped
// sub-kernel, written straight to its pixels of the input gradient — no
// column buffer, no col2im, no work on taps that cannot reach a pixel.
//
// Weight gradient: an implicit GEMM over every output pixel of the batch
// (conv_wgrad.hip), no column matrix. Bias gradient and the BatchNorm
// reductions are per-channel reductions over N x H x W: each (channel, part)
// workgroup reduces a contiguous range of the channel's elements in a fixed
// order (the batch statistics as each part's mean and sum of squared
// deviations, read once), a second kernel combines the parts in order —
// deterministic.
#include "omhip_internal.hpp"
#include "buffer_io.hpp"
#include "conv.hpp"
#include "fastdiv.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

// ---- input gradient by output phase -------------------------------------------------
// For stride s, the input-gradient pixels with ih = a (mod s) receive only the
// taps kh = (a + p) (mod s): kh = r + s*j, oh = i + floor((a+p)/s) - j for
// ih = a + s*i. Over those pixels the gradient is a stride-1 correlation of
// gradOutput with the sub-kernel flipped in j (top pad KHa - 1 - floor((a+p)/s),
// possibly negative), and likewise in w. Stride 1 is the single phase (0, 0)
// with the whole flipped kernel and pad K - 1 - p.

// Taps k in [0, K) of phase a: k = (a + p) (mod s).
__host__ __device__ inline int phaseTaps(int K, int s, int p, int a) {
    const int r = (a + p) % s;
    return r < K ? (K - r + s - 1) / s : 0;
}
__host__ __device__ inline int phaseTapsBefore(int K, int s, int p, int a) {
    int n = 0;
    for (int b = 0; b < a; ++b) n += phaseTaps(K, s, p, b);
    return n;
}
// Offset (floats) of phase (a, b)'s sub-kernel in the phase-major buffer.
__host__ __device__ inline long long phaseOffset(int Cout, int Cin, int KH, int KW, int s, int p, int a, int b) {
    return (long long)Cin * Cout *
           ((long long)phaseTapsBefore(KH, s, p, a) * KW + (long long)phaseTaps(KH, s, p, a) * phaseTapsBefore(KW, s, p, b));
}

// Phase (a, b) sub-kernel: wf[ci][co][jf][lf] = W[co][ci][ra + s*(KHa-1-jf)][rb + s*(KWb-1-lf)].
// Every tap belongs to exactly one phase, so the sub-kernels tile a buffer of W's size.
// Per tap (kh, kw) of W the host precomputes where it lands: wf index =
// base + (ci*Cout + co) * span + inner. One thread per weight (reads
// coalesced); the divisions by taps and Cin use launch-time magic numbers
// (Cout*Cin*KH*KW < 2^28 by the conv limits).
constexpr int kMaxFlipTaps = 256;   // the table travels in the kernel arguments (3 KB)
struct FlipTaps {
    int base[kMaxFlipTaps];    // offset of the tap's phase sub-kernel
    int span[kMaxFlipTaps];    // KHa * KWb of that phase
    int inner[kMaxFlipTaps];   // jf * KWb + lf
};
// Kernels with more taps than the table holds: the same map computed per weight.
__global__ void phase_flip_generic_kernel(const float* __restrict__ w, float* __restrict__ wf, int Cout, int Cin,
                                          int KH, int KW, int s, int p) {
    const int taps = KH * KW;
    const int total = Cout * Cin * taps;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int t = i / taps;
        const int tap = i - t * taps;
        const int kh = tap / KW, kw = tap - (tap / KW) * KW;
        const int co = t / Cin, ci = t - (t / Cin) * Cin;
        const int a = ((kh % s) - (p % s) + s) % s;
        const int b = ((kw % s) - (p % s) + s) % s;
        const int KHa = phaseTaps(KH, s, p, a), KWb = phaseTaps(KW, s, p, b);
        const int jf = KHa - 1 - kh / s, lf = KWb - 1 - kw / s;
        wf[phaseOffset(Cout, Cin, KH, KW, s, p, a, b) + ((ci * Cout + co) * KHa + jf) * KWb + lf] = w[i];
    }
}

__global__ void phase_flip_kernel(const float* __restrict__ w, float* __restrict__ wf, int Cout, int Cin, int taps,
                                  FastDiv dTaps, FastDiv dCin, FlipTaps ft) {
    const int total = Cout * Cin * taps;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int t = (int)dTaps.div((uint32_t)i);
        const int tap = i - t * taps;
        const int co = (int)dCin.div((uint32_t)t), ci = t - co * Cin;
        wf[ft.base[tap] + (ci * Cout + co) * ft.span[tap] + ft.inner[tap]] = w[i];
    }
}

__global__ void zero_fill_kernel(float* __restrict__ y, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        y[i] = 0.f;
}

static int gridFor(long long n) {
    return (int)std::max<long long>(1, std::min<long long>((n + 255) / 256, (long long)cuCount() * 16));
}

// ---- per-channel reductions ------------------------------------------------------
// Parts per channel: enough (channel, part) workgroups to fill the chip, from
// the shape alone so the summation order does not depend on the device.
static int channelParts(int N, int C) { return std::max(1, std::min(N, (2048 + C - 1) / C)); }

template <int NV>
__device__ __forceinline__ void blockSum(float (&v)[NV], float* red) {
    // fixed-order tree over the 256 threads of the workgroup
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NV; ++k) red[k * 256 + tid] = v[k];
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s)
#pragma unroll
            for (int k = 0; k < NV; ++k) red[k * 256 + tid] += red[k * 256 + tid + s];
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = red[k * 256];
}

// Sum over the P parts of channel c, in part order, of part[..][k] — the
// reference's sequential sum split into P ordered pieces (one thread).
__device__ __forceinline__ float partSumSerial(const float* __restrict__ part, int c, int P, int k) {
    float a = 0.f;
    for (int p = 0; p < P; ++p) a += part[((long long)c * P + p) * 2 + k];
    return a;
}

// The same sum for a channel that is uniform across the wave, every lane
// active: lane l of each wave loads part l (all loads in flight at once),
// then every lane adds the lanes' values in part order from registers — the
// same rounding as the sequential loop without its chain of dependent loads.
__device__ __forceinline__ float partSum(const float* __restrict__ part, int c, int P, int k) {
    const int lane = threadIdx.x & 63;
    float a = 0.f;
    for (int p0 = 0; p0 < P; p0 += 64) {
        const int p = p0 + lane;
        const float v = p < P ? part[((long long)c * P + p) * 2 + k] : 0.f;
        const int n = min(64, P - p0);
        for (int j = 0; j < n; ++j)
            a += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j));
    }
    return a;
}

// Per-channel sum of x (a bias gradient), part p of channel c:
// part[(c*P + p)*2] = sum, part[(c*P + p)*2 + 1] = 0.
//
// The part's images n0..n1-1 are one sequence of (image, element) pairs —
// elements in groups of V (V = 4: 16-byte loads, when HW % 4 == 0 and the
// buffer is 16-byte aligned) — walked 256 groups per trip, so small planes
// keep every lane busy. U trips are loaded before any is added, so U loads of
// each lane are in flight at once; a lane adds its elements in sequence order
// (a fixed order: the result does not depend on timing).
template <int V>
__global__ __launch_bounds__(256) void chan_sum_kernel(const float* __restrict__ x, float* __restrict__ part, int N,
                                                       int C, int HW, int P) {
    typedef float fv __attribute__((ext_vector_type(V)));
    constexpr int U = 4;
    __shared__ float red[2 * 256];
    const int c = blockIdx.x, p = blockIdx.y;
    const int n0 = (int)((long long)p * N / P), n1 = (int)((long long)(p + 1) * N / P);
    const int HWV = HW / V;   // groups per plane
    float v[2] = {0.f, 0.f};
    const int dn = 256 / HWV, ds = 256 % HWV;
    int n = n0 + (int)threadIdx.x / HWV, sg = (int)threadIdx.x % HWV;
    auto advance = [&](int& nn, int& ss) {
        nn += dn;
        ss += ds;
        if (ss >= HWV) {
            ss -= HWV;
            ++nn;
        }
    };
    while (n < n1) {
        fv xv[U];
        bool ok[U];
        {
            int nn = n, ss = sg;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                ok[u] = nn < n1;
                if (ok[u]) xv[u] = *reinterpret_cast<const fv*>(x + ((long long)nn * C + c) * HW + (long long)ss * V);
                advance(nn, ss);
            }
            n = nn;
            sg = ss;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
#pragma unroll
            for (int k = 0; k < V; ++k) v[0] += V == 1 ? xv[u][0] : xv[u][k];
        }
    }
    blockSum<2>(v, red);
    if (threadIdx.x == 0) {
        part[((long long)c * P + p) * 2] = v[0];
        part[((long long)c * P + p) * 2 + 1] = v[1];
    }
}

// Sums the P parts of each channel in order; out0[c] = sum / divisor (and out1).
// The division is the reference's `sum /= count` (a true division; 1 leaves
// the sum unchanged).
__global__ void chan_finish_kernel(const float* __restrict__ part, float* out0, float* out1, int C, int P,
                                   float divisor, int accumulate) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const float a = partSumSerial(part, c, P, 0), b = partSumSerial(part, c, P, 1);
    if (out0) out0[c] = accumulate ? out0[c] + a / divisor : a / divisor;
    if (out1) out1[c] = accumulate ? out1[c] + b / divisor : b / divisor;
}

// ---- BatchNorm statistics in one pass ------------------------------------------------
// A channel's N*HW elements, taken as one sequence (image by image), split into
// parts of kStatPart elements (the last may be shorter); a part is one
// workgroup of 256 threads, each holding kStatElems of its elements in
// registers, so every load is issued before any arithmetic and the part is read
// from memory once. The part's mean and its sum of squared deviations from that
// mean (an exact two-pass over the registers, fixed-order tree sums) are
// combined across parts in part order by the pairwise update of Chan, Golub and
// LeVeque (1979): n = na + nb, d = mb - ma, mean = ma + d nb / n,
// M2 = M2a + M2b + d^2 na nb / n. The parts depend on the shape only, so the
// result is deterministic.
constexpr int kStatElems = 32;
constexpr int kStatPart = 256 * kStatElems;

static int statParts(long long L) { return (int)((L + kStatPart - 1) / kStatPart); }

// part[(c*P + p)*2] = (mean, M2) of part p of channel c.
template <int V>
__global__ __launch_bounds__(256) void bn_stats_part_kernel(const float* __restrict__ x, float* __restrict__ part, int C,
                                                            int HW, FastDiv dHW, long long L, int P) {
    typedef float fv __attribute__((ext_vector_type(V)));
    constexpr int G = kStatElems / V;   // loads per thread
    __shared__ float red[256];
    const int c = blockIdx.x, p = blockIdx.y;
    const long long beg = (long long)p * kStatPart;
    const int cntP = (int)min((long long)kStatPart, L - beg);
    fv xv[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int i = (int)threadIdx.x * V + j * 256 * V;   // element of the part
        if (i < cntP) {
            const uint32_t gi = (uint32_t)(beg + i);
            const uint32_t n = dHW.div(gi);
            xv[j] = *reinterpret_cast<const fv*>(x + ((long long)n * C + c) * HW + (gi - n * (uint32_t)HW));
        } else {
#pragma unroll
            for (int k = 0; k < V; ++k) xv[j][k] = 0.f;   // adds nothing; excluded from M2 below
        }
    }
    float v[1] = {0.f};
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int k = 0; k < V; ++k) v[0] += xv[j][k];
    blockSum<1>(v, red);
    const float mean = v[0] / (float)cntP;
    __syncthreads();   // red is reused
    float m2[1] = {0.f};
#pragma unroll
    for (int j = 0; j < G; ++j) {
        if ((int)threadIdx.x * V + j * 256 * V < cntP) {
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float d = xv[j][k] - mean;
                m2[0] = __builtin_fmaf(d, d, m2[0]);
            }
        }
    }
    blockSum<1>(m2, red);
    if (threadIdx.x == 0) {
        part[((long long)c * P + p) * 2] = mean;
        part[((long long)c * P + p) * 2 + 1] = m2[0];
    }
}

// Channel c's statistics from its P parts, merged in part order by the
// pairwise update (the first part as is, then each next part into the running
// result), by the 64 lanes of one wave: lane l loads part l (all loads in
// flight at once) and every lane folds the lanes' values in from registers —
// the rounding of a sequential loop, without its chain of dependent loads.
// The update's two weights, nb / (n + nb) and n nb / (n + nb) (in double,
// rounded to float), depend only on the part's index: every part before the
// last is full, so n = p * kStatPart exactly (a multiple of 2^13 below 2^32, a
// float that holds it exactly). Lane l computes part l's weights, so the
// serial fold has no division in it (each step of it had two in double).
// Returns mean and the biased variance M2 / L.
__device__ __forceinline__ void mergeStats(const float* __restrict__ part, int c, int P, long long L, float& mean,
                                           float& var) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    float mu = 0.f, m2 = 0.f;
    for (int p0 = 0; p0 < P; p0 += 64) {
        const int pl = p0 + lane;
        const bool have = pl < P;
        const float mv = have ? part[((long long)c * P + pl) * 2] : 0.f;
        const float m2v = have ? part[((long long)c * P + pl) * 2 + 1] : 0.f;
        const long long before = (long long)pl * kStatPart;
        const double na = (double)before;
        const double nb = have ? (double)min((long long)kStatPart, L - before) : 1.0;
        const double nn = na + nb;
        const float wMean = (float)(nb / nn);
        const float wM2 = (float)(na * nb / nn);
        const int cnt = min(64, P - p0);
        for (int j = 0; j < cnt; ++j) {
            const float mb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mv), j));
            const float m2b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m2v), j));
            if (p0 + j == 0) {
                mu = mb;
                m2 = m2b;
            } else {
                const float wa = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wMean), j));
                const float wb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wM2), j));
                const float d = mb - mu;
                mu = mu + d * wa;
                m2 = m2 + m2b + d * d * wb;
            }
        }
    }
    mean = mu;
    var = m2 / (float)L;
}

// BatchNorm backward sums of one part (the parts of bn_stats_part_kernel, 16
// elements per thread: dy, x and the mask are all in flight at once):
// part[(c*P + p)*2] = (sum dy*xhat, sum dy), xhat = (x - mean) * invStd, dy
// gated by mask > 0 when a mask is given (the reference's reluBackward folded
// in). Summed in a fixed order (per thread, then a fixed tree).
constexpr int kBwdElems = 16;
constexpr int kBwdPart = 256 * kBwdElems;

template <int V>
__global__ __launch_bounds__(256) void bn_bwd_part_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                          const float* __restrict__ mask,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ invStd, float* __restrict__ part,
                                                          int C, int HW, FastDiv dHW, long long L, int P) {
    typedef float fv __attribute__((ext_vector_type(V)));
    constexpr int G = kBwdElems / V;
    __shared__ float red[2 * 256];
    const int c = blockIdx.x, p = blockIdx.y;
    const long long beg = (long long)p * kBwdPart;
    const int cntP = (int)min((long long)kBwdPart, L - beg);
    const float m = mean[c], is = invStd[c];
    fv xv[G], gv[G], mv[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int i = (int)threadIdx.x * V + j * 256 * V;
#pragma unroll
        for (int k = 0; k < V; ++k) { xv[j][k] = 0.f; gv[j][k] = 0.f; mv[j][k] = 1.f; }
        if (i < cntP) {
            const uint32_t gi = (uint32_t)(beg + i);
            const uint32_t n = dHW.div(gi);
            const long long e = ((long long)n * C + c) * HW + (gi - n * (uint32_t)HW);
            xv[j] = *reinterpret_cast<const fv*>(x + e);
            gv[j] = *reinterpret_cast<const fv*>(dy + e);
            if (mask) mv[j] = *reinterpret_cast<const fv*>(mask + e);
        }
    }
    float v[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const float g = mv[j][k] > 0.f ? gv[j][k] : 0.f;
            const float xh = (xv[j][k] - m) * is;
            v[0] = __builtin_fmaf(g, xh, v[0]);
            v[1] += g;
        }
    blockSum<2>(v, red);
    if (threadIdx.x == 0) {
        part[((long long)c * P + p) * 2] = v[0];
        part[((long long)c * P + p) * 2 + 1] = v[1];
    }
}

// Element-wise BatchNorm passes, one workgroup per (channel, chunk of
// kApplyChunk<V> of the channel's N*HW elements): element i of channel c is
// x[(i / HW) * C + c][i % HW] (groups of V = 4 never straddle two planes:
// HW % 4 == 0). Wave 0 first forms the channel's statistics from the parts
// (the merge of the statistics kernel's parts), while every thread's loads
// are already in flight; workgroup (c, 0) also writes the channel's saved /
// running statistics or parameter gradients. Each thread takes U groups of V.
template <int V>
constexpr int kApplyChunk = 256 * V * 4;

struct BnChan {
    int C, HW, Q;   // Q: workgroups per channel
    long long L;    // elements per channel
    FastDiv dHW;
    __device__ __forceinline__ long long offset(int c, long long i) const {
        const uint32_t n = dHW.div((uint32_t)i);
        return ((long long)n * C + c) * HW + (long long)((uint32_t)i - n * (uint32_t)HW);
    }
};

// y = act(gamma*((x-mean)*invStd) + beta [+ res]) (the reference's
// batchNorm2d, add and relu, each rounded as there), with the batch
// statistics merged from the parts: mean, var = M2 / L, invStd =
// 1/sqrt(var + eps); saved statistics and running averages fma(1-m, run,
// m*batch) written once per channel.
template <int V>
__global__ __launch_bounds__(256) void bn_train_apply_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ part, int P, float eps,
                                                             float momentum, float* savedMean, float* savedInvStd,
                                                             float* runMean, float* runVar,
                                                             const float* __restrict__ res, int act, BnChan f) {
#pragma clang fp contract(off)
    typedef float fv __attribute__((ext_vector_type(V)));
    constexpr int U = 4;
    __shared__ float st[2];
    const int c = blockIdx.x / f.Q, q = blockIdx.x - c * f.Q;
    const long long i0 = (long long)q * kApplyChunk<V> + (long long)threadIdx.x * V;
    fv xv[U], rv[U];
    long long off[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = i0 + (long long)u * 256 * V;
        off[u] = i < f.L ? f.offset(c, i) : -1;
        if (off[u] >= 0) {
            xv[u] = *reinterpret_cast<const fv*>(x + off[u]);
            if (res) rv[u] = *reinterpret_cast<const fv*>(res + off[u]);
        }
    }
    if (threadIdx.x < 64) {
        float mu, var;
        mergeStats(part, c, P, f.L, mu, var);
        const float inv = 1.0f / sqrtf(var + eps);
        if (threadIdx.x == 0) {
            st[0] = mu;
            st[1] = inv;
            if (q == 0) {
                if (savedMean) savedMean[c] = mu;
                if (savedInvStd) savedInvStd[c] = inv;
                runMean[c] = __builtin_fmaf(1.0f - momentum, runMean[c], momentum * mu);
                runVar[c] = __builtin_fmaf(1.0f - momentum, runVar[c], momentum * var);
            }
        }
    }
    __syncthreads();
    const float mu = st[0], inv = st[1], g = gamma[c], b = beta[c];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (off[u] < 0) break;
        fv out;
#pragma unroll
        for (int k = 0; k < V; ++k) {
            float v = __builtin_fmaf(g, (xv[u][k] - mu) * inv, b);
            if (res) v = v + rv[u][k];
            if (act == 1) v = v > 0.f ? v : 0.f;
            out[k] = v;
        }
        *reinterpret_cast<fv*>(y + off[u]) = out;
    }
}

// dx = gamma*invStd*(1/cnt) * (cnt*dy - sum(dy) - xhat*sum(dy*xhat)) (cpu_backend.ixx:883-886),
// with the multiply-adds fused as the reference compiled by clang fuses them;
// dy gated by mask > 0 when mask is given. sum(dy*xhat) and sum(dy) are the
// parts summed in part order (also gradGamma and gradBeta, written once per
// channel).
template <int V>
__global__ __launch_bounds__(256) void bn_backward_apply_kernel(const float* __restrict__ dy,
                                                                const float* __restrict__ mask,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ mean,
                                                                const float* __restrict__ invStd,
                                                                const float* __restrict__ gamma,
                                                                const float* __restrict__ part, int P,
                                                                float* gradGamma, float* gradBeta,
                                                                float* __restrict__ dx, float cnt, float invCnt,
                                                                BnChan f) {
    typedef float fv __attribute__((ext_vector_type(V)));
    constexpr int U = 4;
    __shared__ float st[2];
    const int c = blockIdx.x / f.Q, q = blockIdx.x - c * f.Q;
    const long long i0 = (long long)q * kApplyChunk<V> + (long long)threadIdx.x * V;
    fv dv[U], xv[U], mv[U];
    long long off[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = i0 + (long long)u * 256 * V;
        off[u] = i < f.L ? f.offset(c, i) : -1;
        if (off[u] >= 0) {
            dv[u] = *reinterpret_cast<const fv*>(dy + off[u]);
            xv[u] = *reinterpret_cast<const fv*>(x + off[u]);
            if (mask) mv[u] = *reinterpret_cast<const fv*>(mask + off[u]);
        }
    }
    if (threadIdx.x < 64) {
        const float sg = partSum(part, c, P, 0), sb = partSum(part, c, P, 1);
        if (threadIdx.x == 0) {
            st[0] = sg;
            st[1] = sb;
            if (q == 0) {
                if (gradGamma) gradGamma[c] = sg;
                if (gradBeta) gradBeta[c] = sb;
            }
        }
    }
    __syncthreads();
    const float m = mean[c], is = invStd[c], sg = st[0], sb = st[1];
    const float k = gamma[c] * is * invCnt;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (off[u] < 0) break;
        fv out;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const float d = (mask && !(mv[u][j] > 0.f)) ? 0.f : dv[u][j];
            const float xh = (xv[u][j] - m) * is;
            out[j] = k * __builtin_fmaf(-xh, sg, __builtin_fmaf(cnt, d, -sb));
        }
        *reinterpret_cast<fv*>(dx + off[u]) = out;
    }
}

static BnChan bnChan(int N, int C, int HW, int V) {
    BnChan f{};
    f.C = C;
    f.HW = HW;
    f.L = (long long)N * HW;
    f.Q = (int)((f.L + (256LL * V * 4) - 1) / (256LL * V * 4));
    f.dHW = FastDiv::make((uint32_t)HW);
    return f;
}

static bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Per-channel sums of x over N x HW into out0 (divided by divisor, or added
// to it when accumulating): parts in a fixed order, then the parts in order.
static int channelSums(const float* x, float* out0, int N, int C, int HW, float divisor, bool accumulate) {
    const int P = channelParts(N, C);
    float* part = static_cast<float*>(workspace((size_t)C * P * 2 * sizeof(float)));
    if (!part) return -1;   // workspace() recorded the cause
    if (HW % 4 == 0 && aligned16(x))
        hipLaunchKernelGGL(chan_sum_kernel<4>, dim3(C, P), dim3(256), 0, stream(), x, part, N, C, HW, P);
    else
        hipLaunchKernelGGL(chan_sum_kernel<1>, dim3(C, P), dim3(256), 0, stream(), x, part, N, C, HW, P);
    OMHIP_CHECK_LAUNCH();
    hipLaunchKernelGGL(chan_finish_kernel, dim3((C + 255) / 256), dim3(256), 0, stream(), part, out0, nullptr, C, P,
                       divisor, accumulate ? 1 : 0);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int batchNorm2dTrainAct(const float* x, float* y, const float* gamma, const float* beta, float* runMean,
                        float* runVar, float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps,
                        float momentum, const float* res, int act) {
    const int HW = H * W;
    const long long L = (long long)N * HW;   // elements per channel
    if (L >= (1LL << 32)) return fail("batchNorm2d: %lld elements per channel exceed 2^32", L);
    const int P = statParts(L);
    float* part = static_cast<float*>(workspace((size_t)C * P * 2 * sizeof(float)));
    if (!part) return -1;
    // one read of x: each part's mean and M2 (two passes over registers), merged in part order
    const bool vx = HW % 4 == 0 && aligned16(x);
    const FastDiv dHW = FastDiv::make((uint32_t)HW);
    if (vx)
        hipLaunchKernelGGL(bn_stats_part_kernel<4>, dim3(C, P), dim3(256), 0, stream(), x, part, C, HW, dHW, L, P);
    else
        hipLaunchKernelGGL(bn_stats_part_kernel<1>, dim3(C, P), dim3(256), 0, stream(), x, part, C, HW, dHW, L, P);
    OMHIP_CHECK_LAUNCH();
    const bool vec = HW % 4 == 0 && aligned16(x) && aligned16(y) && (!res || aligned16(res));
    const BnChan f = bnChan(N, C, HW, vec ? 4 : 1);
    if ((long long)C * f.Q >= (1LL << 31)) return fail("batchNorm2d: tensor too large");
    if (vec)
        hipLaunchKernelGGL(bn_train_apply_kernel<4>, dim3(C * f.Q), dim3(256), 0, stream(), x, y, gamma, beta, part, P,
                           eps, momentum, savedMean, savedInvStd, runMean, runVar, res, act, f);
    else
        hipLaunchKernelGGL(bn_train_apply_kernel<1>, dim3(C * f.Q), dim3(256), 0, stream(), x, y, gamma, beta, part, P,
                           eps, momentum, savedMean, savedInvStd, runMean, runVar, res, act, f);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int batchNorm2dTrain(const float* x, float* y, const float* gamma, const float* beta, float* runMean, float* runVar,
                     float* savedMean, float* savedInvStd, int N, int C, int H, int W, float eps, float momentum) {
    return batchNorm2dTrainAct(x, y, gamma, beta, runMean, runVar, savedMean, savedInvStd, N, C, H, W, eps, momentum,
                               nullptr, 0);
}

// BatchNorm2d backward with an optional ReLU mask on the incoming gradient.
static int batchNorm2dBackwardMasked(const char* name, const float* gO, const float* mask, const float* x,
                                     const float* mean, const float* invStd, const float* gamma, float* gI,
                                     float* gGamma, float* gBeta, int N, int C, int H, int W) {
    if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return 0;
    if (!gO || !x || !mean || !invStd || !gamma || !gI) return fail("%s: null pointer", name);
    const int HW = H * W;
    const long long L = (long long)N * HW;
    if (L >= (1LL << 32)) return fail("%s: %lld elements per channel exceed 2^32", name, L);
    const int P = (int)((L + kBwdPart - 1) / kBwdPart);
    float* part = static_cast<float*>(workspace((size_t)C * P * 2 * sizeof(float)));
    if (!part) return -1;
    const bool vp = HW % 4 == 0 && aligned16(x) && aligned16(gO) && (!mask || aligned16(mask));
    const FastDiv dHW = FastDiv::make((uint32_t)HW);
    if (vp)
        hipLaunchKernelGGL(bn_bwd_part_kernel<4>, dim3(C, P), dim3(256), 0, stream(), x, gO, mask, mean, invStd, part,
                           C, HW, dHW, L, P);
    else
        hipLaunchKernelGGL(bn_bwd_part_kernel<1>, dim3(C, P), dim3(256), 0, stream(), x, gO, mask, mean, invStd, part,
                           C, HW, dHW, L, P);
    OMHIP_CHECK_LAUNCH();
    const long long cntL = (long long)N * HW;
    const float fcnt = (float)cntL;
    const float invCnt = 1.0f / fcnt;
    const bool vec = HW % 4 == 0 && aligned16(gO) && aligned16(x) && aligned16(gI) && (!mask || aligned16(mask));
    const BnChan f = bnChan(N, C, HW, vec ? 4 : 1);
    if ((long long)C * f.Q >= (1LL << 31)) return fail("%s: tensor too large", name);
    if (vec)
        hipLaunchKernelGGL(bn_backward_apply_kernel<4>, dim3(C * f.Q), dim3(256), 0, stream(), gO, mask, x, mean,
                           invStd, gamma, part, P, gGamma, gBeta, gI, fcnt, invCnt, f);
    else
        hipLaunchKernelGGL(bn_backward_apply_kernel<1>, dim3(C * f.Q), dim3(256), 0, stream(), gO, mask, x, mean,
                           invStd, gamma, part, P, gGamma, gBeta, gI, fcnt, invCnt, f);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

static int validateConvGrad(const char* name, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride,
                            int pad, int& Ho, int& Wo) {
    if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0)
        return fail("%s: invalid geometry", name);
    Ho = (H + 2 * pad - KH) / stride + 1;
    Wo = (W + 2 * pad - KW) / stride + 1;
    if (Ho <= 0 || Wo <= 0) return fail("%s: kernel larger than the padded input", name);
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipConv2dBackwardInput(const float* pGradOutput, const float* pWeight, float* pGradInput, int nBatch,
                             int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride, int nPad) {
    clearError();
    const char* name = "omHipConv2dBackwardInput";
    int Ho, Wo;
    if (validateConvGrad(name, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad, Ho, Wo)) return -1;
    if (!pGradOutput || !pWeight || !pGradInput) return fail("%s: null pointer", name);
    const int s = nStride, p = nPad;
    const long long wsz = (long long)nCout * nCin * nKH * nKW;
    if (wsz * 4 > (long long)kMaxBufferBytes)
        return fail("%s: weights exceed the 2^30-byte buffer range of this kernel", name);
    // Pixels of a phase without taps (stride > kernel) get no contribution.
    bool emptyPhase = false;
    for (int a = 0; a < std::min(s, nH); ++a)
        for (int b = 0; b < std::min(s, nW); ++b)
            if (phaseTaps(nKH, s, p, a) == 0 || phaseTaps(nKW, s, p, b) == 0) emptyPhase = true;
    if (emptyPhase) {
        const long long n = (long long)nBatch * nCin * nH * nW;
        hipLaunchKernelGGL(zero_fill_kernel, dim3(gridFor(n)), dim3(256), 0, stream(), pGradInput, n);
        OMHIP_CHECK_LAUNCH();
    }
    float* wf = static_cast<float*>(workspace((size_t)wsz * sizeof(float), kWsOperand));
    if (!wf) return -1;   // workspace() recorded the cause
    if (nKH * nKW > kMaxFlipTaps) {
        hipLaunchKernelGGL(phase_flip_generic_kernel, dim3(gridFor(wsz)), dim3(256), 0, stream(), pWeight, wf, nCout,
                           nCin, nKH, nKW, s, p);
    } else {
        FlipTaps ft{};
        for (int kh = 0; kh < nKH; ++kh)
            for (int kw = 0; kw < nKW; ++kw) {
                const int a = ((kh % s) - (p % s) + s) % s;
                const int b = ((kw % s) - (p % s) + s) % s;
                const int KHa = phaseTaps(nKH, s, p, a), KWb = phaseTaps(nKW, s, p, b);
                const int jf = KHa - 1 - kh / s, lf = KWb - 1 - kw / s;
                const int tap = kh * nKW + kw;
                ft.base[tap] = (int)phaseOffset(nCout, nCin, nKH, nKW, s, p, a, b);
                ft.span[tap] = KHa * KWb;
                ft.inner[tap] = jf * KWb + lf;
            }
        hipLaunchKernelGGL(phase_flip_kernel, dim3(gridFor(wsz)), dim3(256), 0, stream(), pWeight, wf, nCout, nCin,
                           nKH * nKW, FastDiv::make((uint32_t)(nKH * nKW)), FastDiv::make((uint32_t)nCin), ft);
    }
    int rc = hipGetLastError() == hipSuccess ? 0 : fail("%s: flip launch failed", name);
    for (int a = 0; a < std::min(s, nH) && !rc; ++a) {
        const int KHa = phaseTaps(nKH, s, p, a);
        if (KHa == 0) continue;
        const int Hp = (nH - a + s - 1) / s;
        for (int b = 0; b < std::min(s, nW) && !rc; ++b) {
            const int KWb = phaseTaps(nKW, s, p, b);
            if (KWb == 0) continue;
            const int Wp = (nW - b + s - 1) / s;
            rc = conv2dToGrid(name, pGradOutput, wf + phaseOffset(nCout, nCin, nKH, nKW, s, p, a, b), pGradInput,
                              nBatch, nCout, Ho, Wo, nCin, KHa, KWb, KHa - 1 - (a + p) / s, KWb - 1 - (b + p) / s, Hp,
                              Wp, nH, nW, s, a, b);
        }
    }
    return rc;
}

int omHipConv2dBackwardWeight(const float* pInput, const float* pGradOutput, float* pGradWeight, float* pGradBias,
                              int nBatch, int nCin, int nH, int nW, int nCout, int nKH, int nKW, int nStride,
                              int nPad) {
    clearError();
    const char* name = "omHipConv2dBackwardWeight";
    int Ho, Wo;
    if (validateConvGrad(name, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride, nPad, Ho, Wo)) return -1;
    if (!pInput || !pGradOutput || !pGradWeight) return fail("%s: null pointer", name);
    if (conv2dWeightGrad(name, pInput, pGradOutput, pGradWeight, nBatch, nCin, nH, nW, nCout, nKH, nKW, nStride,
                         nPad))
        return -1;
    const long long HWo = (long long)Ho * Wo;
    if (pGradBias) return channelSums(pGradOutput, pGradBias, nBatch, nCout, (int)HWo, 1.0f, false);
    return 0;
}

int omHipBatchNorm2dBackward(const float* pGradOutput, const float* pInput, const float* pMean, const float* pInvStd,
                             const float* pGamma, float* pGradInput, float* pGradGamma, float* pGradBeta, int nBatch,
                             int nChannels, int nH, int nW, float fEps) {
    clearError();
    (void)fEps;   // the saved inverse standard deviation already carries eps
    return batchNorm2dBackwardMasked("omHipBatchNorm2dBackward", pGradOutput, nullptr, pInput, pMean, pInvStd, pGamma,
                                     pGradInput, pGradGamma, pGradBeta, nBatch, nChannels, nH, nW);
}

int omHipBatchNorm2dBackwardRelu(const float* pGradOutput, const float* pReluInput, const float* pInput,
                                 const float* pMean, const float* pInvStd, const float* pGamma, float* pGradInput,
                                 float* pGradGamma, float* pGradBeta, int nBatch, int nChannels, int nH, int nW,
                                 float fEps) {
    clearError();
    (void)fEps;
    if (!pReluInput) return fail("omHipBatchNorm2dBackwardRelu: null ReLU input");
    return batchNorm2dBackwardMasked("omHipBatchNorm2dBackwardRelu", pGradOutput, pReluInput, pInput, pMean, pInvStd,
                                     pGamma, pGradInput, pGradGamma, pGradBeta, nBatch, nChannels, nH, nW);
}

int omHipBatchNorm2dTrainAct(const float* pInput, float* pOutput, const float* pGamma, const float* pBeta,
                             float* pRunningMean, float* pRunningVar, float* pSavedMean, float* pSavedInvStd,
                             int nBatch, int nChannels, int nH, int nW, float fEps, float fMomentum,
                             const float* pResidual, int nAct) {
    clearError();
    if (nBatch <= 0 || nChannels <= 0 || nH <= 0 || nW <= 0) return 0;
    if (!pInput || !pOutput || !pGamma || !pBeta || !pRunningMean || !pRunningVar)
        return fail("omHipBatchNorm2dTrainAct: null pointer");
    if (nAct != 0 && nAct != 1) return fail("omHipBatchNorm2dTrainAct: unknown activation %d", nAct);
    return batchNorm2dTrainAct(pInput, pOutput, pGamma, pBeta, pRunningMean, pRunningVar, pSavedMean, pSavedInvStd,
                               nBatch, nChannels, nH, nW, fEps, fMomentum, pResidual, nAct);
}

}  // extern "C"
