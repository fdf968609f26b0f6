// loss.hip — the loss end of a Linear network's training step and the Linear
// bias gradient: softmax over the last axis, the cross-entropy of softmax
// outputs against one-hot targets, their joint gradient, and the bias
// gradient (sum of the output gradient over every axis but the channel).
//
// Reference (CPUBackend, the parity target): softmax cpu_backend.ixx:352-370,
// crossEntropy :375-388, crossEntropySoftmaxBackward :393-410; the bias
// gradient of AddBiasBackward autograd.ixx:428-433. The GPU path the
// reference calls: omCudaSoftmax / omCudaCrossEntropy /
// omCudaSoftmaxCrossEntropyBackward / omCudaAddBiasBackward
// (cuda_kernels.cuh:122, :399, :288, :348).
//
// Rows are small (a batch of class scores), so every kernel is latency- and
// launch-bound, not HBM-bound: a wave owns a row, lanes stride its classes,
// and every reduction has a fixed order (butterfly within a wave, waves and
// row contributions added in index order), so results do not depend on the
// device or the launch.
#include "omhip_internal.hpp"
#include "fastdiv.hpp"
#include "buffer_io.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

namespace {

typedef float f32x4l __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float waveSum(float v) {
    // fixed butterfly: every lane ends with the same sum in the same order
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// max with the reference's semantics: the scan keeps a candidate unless an
// element is strictly greater, so NaN elements are skipped (and a NaN first
// element is kept, handled by the caller).
__device__ __forceinline__ float gtMax(float m, float v) { return v > m ? v : m; }

__device__ __forceinline__ float waveMax(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = gtMax(v, __shfl_xor(v, off, 64));
    return v;
}

// Row maximum as the reference's scan computes it (cpu_backend.ixx:356-358):
// the first element when it is NaN, else the largest non-NaN element.
__device__ __forceinline__ float rowMax(const float* r, int cols, int lane) {
    float m = -INFINITY;
    for (int j = lane; j < cols; j += 64) m = gtMax(m, r[j]);
    m = waveMax(m);
    const float r0 = r[0];
    return r0 != r0 ? r0 : gtMax(r0, m);
}

// Softmax of one row by one wave: exp(x - max) stored to o, wave sum, then
// o /= sum (each lane rereads only what it wrote).
__device__ __forceinline__ void softmaxRow(const float* r, float* o, int cols, int lane) {
    const float m = rowMax(r, cols, lane);
    float s = 0.f;
    for (int j = lane; j < cols; j += 64) {
        const float e = expf(r[j] - m);
        o[j] = e;
        s += e;
    }
    s = waveSum(s);
    for (int j = lane; j < cols; j += 64) o[j] = o[j] / s;
}

// One row's cross-entropy terms (cpu_backend.ixx:378-384): -log(max(p, 1e-7))
// where the target exceeds 0.5, summed over the row by the wave.
__device__ __forceinline__ float rowLoss(const float* p, const float* t, int cols, int lane) {
    float acc = 0.f;
    for (int j = lane; j < cols; j += 64) {
        if (t[j] > 0.5f) {
            float q = p[j];
            if (q < 1e-7f) q = 1e-7f;
            acc -= logf(q);
        }
    }
    return waveSum(acc);
}

constexpr int kLossWaves = 16;   // the loss kernels run as one workgroup of 16 waves

// Adds the 16 waves' loss partials in wave order and writes sum / batch.
__device__ __forceinline__ void finishLoss(float waveAcc, float* result, int rows, float* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = waveAcc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float tot = 0.f;
        for (int w = 0; w < kLossWaves; ++w) tot += lds[w];
        result[0] = tot / (float)rows;
    }
}

}  // namespace

__global__ void __launch_bounds__(256) softmax_rows_kernel(const float* in, float* out, int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    softmaxRow(in + row * cols, out + row * cols, cols, lane);
}

// Wave w takes rows w, w+16, ...; its partial adds the row sums in row order.
__global__ void __launch_bounds__(1024) cross_entropy_kernel(const float* pred, const float* tgt, float* result,
                                                             int rows, int cols) {
    __shared__ float lds[kLossWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r = wave; r < rows; r += kLossWaves) acc += rowLoss(pred + r * cols, tgt + r * cols, cols, lane);
    finishLoss(acc, result, rows, lds);
}

__global__ void softmax_ce_backward_kernel(const float* s, const float* t, float* g, long long n, float scale) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += stride)
        g[i] = (s[i] - t[i]) * scale;
}

// softmax -> crossEntropy -> crossEntropySoftmaxBackward in one workgroup, with
// the same per-row code and loss order as the three kernels above (so each
// output is bit-identical to theirs). Any output pointer may be null; the
// softmax row is written to `prob` when given, else to `grad` (and then
// overwritten by the gradient), else kept in the scratch row `rowBuf`.
__global__ void __launch_bounds__(1024) softmax_ce_fused_kernel(const float* logits, const float* tgt, float* prob,
                                                                float* loss, float* grad, float* rowBuf, int rows,
                                                                int cols, float scale) {
    __shared__ float lds[kLossWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r = wave; r < rows; r += kLossWaves) {
        float* p = prob ? prob + r * cols : (grad ? grad + r * cols : rowBuf + (long long)wave * cols);
        const float* t = tgt + r * cols;
        softmaxRow(logits + r * cols, p, cols, lane);
        if (loss) acc += rowLoss(p, t, cols, lane);
        if (grad)
            for (int j = lane; j < cols; j += 64) grad[r * cols + j] = (p[j] - t[j]) * scale;
    }
    if (loss) finishLoss(acc, loss, rows, lds);
}

// The same fused pass for rows of at most 64 * CPL classes with the row in
// registers: a wave loads RB rows at once (logits and targets, lane l holding
// classes l, l+64, ...), then each row runs the same operations in the same
// order as softmaxRow / rowLoss / the gradient above — only the values stay in
// registers instead of being written and read back — so every output is
// bit-identical to the three kernels'.
template <int CPL>
__global__ void __launch_bounds__(1024) softmax_ce_fused_reg_kernel(const float* logits, const float* tgt, float* prob,
                                                                    float* loss, float* grad, int rows, int cols,
                                                                    float scale) {
    __shared__ float lds[kLossWaves];
    constexpr int RB = 8;   // rows of a wave whose loads are in flight together
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.f;
    for (long long r0 = wave; r0 < rows; r0 += (long long)kLossWaves * RB) {
        float x[RB][CPL], t[RB][CPL];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const long long r = r0 + (long long)i * kLossWaves;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int j = lane + 64 * c;
                const bool ok = r < rows && j < cols;
                x[i][c] = ok ? logits[r * cols + j] : 0.f;
                t[i][c] = ok ? tgt[r * cols + j] : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const long long r = r0 + (long long)i * kLossWaves;
            if (r >= rows) break;   // wave-uniform
            // rowMax: the first element when it is NaN, else the largest non-NaN element
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (lane + 64 * c < cols) m = gtMax(m, x[i][c]);
            m = waveMax(m);
            const float e0 = __shfl(x[i][0], 0, 64);
            m = e0 != e0 ? e0 : gtMax(e0, m);
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (lane + 64 * c < cols) {
                    const float e = expf(x[i][c] - m);
                    x[i][c] = e;
                    sum += e;
                }
            sum = waveSum(sum);
            float la = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int j = lane + 64 * c;
                if (j >= cols) continue;
                const float pv = x[i][c] / sum;
                if (prob) prob[r * cols + j] = pv;
                if (loss && t[i][c] > 0.5f) {
                    float q = pv;
                    if (q < 1e-7f) q = 1e-7f;
                    la -= logf(q);
                }
                if (grad) grad[r * cols + j] = (pv - t[i][c]) * scale;
            }
            if (loss) acc += waveSum(la);
        }
    }
    if (loss) finishLoss(acc, loss, rows, lds);
}

// Bias gradient, nHW == 1 (a Linear layer's [rows, cols] gradient): a thread per
// column adds the rows in order, starting from 0 — the reference's loop order
// (autograd.ixx:428-433), so the result is bit-identical to it.
__global__ void bias_grad_cols_kernel(const float* g, float* gb, int rows, int cols) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    const float* p = g + c;
    float acc = 0.f;
    int r = 0;
    for (; r + 64 <= rows; r += 64) {   // 64 loads in flight, then the adds in row order
        float a[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) a[i] = p[(long long)(r + i) * cols];
#pragma unroll
        for (int i = 0; i < 64; ++i) acc += a[i];
    }
    for (; r < rows; ++r) acc += p[(long long)r * cols];
    gb[c] = acc;
}

// Bias gradient for many rows: block = 64 columns x 16 row parts; each part adds
// its contiguous rows in order, then the parts are added in order.
__global__ void __launch_bounds__(1024) bias_grad_cols_parts_kernel(const float* g, float* gb, int rows, int cols) {
    __shared__ float part[16][65];
    const int cl = threadIdx.x & 63, pi = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    const int len = (rows + 15) / 16;
    const int r0 = pi * len, r1 = min(rows, r0 + len);
    float acc = 0.f;
    if (c < cols)
        for (int r = r0; r < r1; ++r) acc += g[(long long)r * cols + c];
    part[pi][cl] = acc;
    __syncthreads();
    if (pi == 0 && c < cols) {
        float tot = 0.f;
        for (int q = 0; q < 16; ++q) tot += part[q][cl];
        gb[c] = tot;
    }
}

// Bias gradient of an [N, C, HW] gradient (conv layout): a workgroup per channel,
// thread t adds elements hw = t, t+256, ... of every image in (image, hw) order,
// then a fixed tree over the 256 partials.
__global__ void __launch_bounds__(256) bias_grad_planes_kernel(const float* g, float* gb, int N, int C, int HW) {
    __shared__ float red[256];
    const int c = blockIdx.x;
    float acc = 0.f;
    for (int n = 0; n < N; ++n) {
        const float* p = g + ((long long)n * C + c) * HW;
        for (int i = threadIdx.x; i < HW; i += 256) acc += p[i];
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s >= 1; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) gb[c] = red[0];
}

// ---- the classifier head of a training step, a workgroup per block of rows ----------
// From A [M][K] (the last hidden layer's output), W [K][N], b [N] and targets
// T [M][N], N <= 64:
//   z = A W + b; p = softmax(z) per row; loss = mean over rows of the terms
//   -log(max(p_j, 1e-7)) of the classes whose target exceeds 0.5;
//   g = (p - T) / M; gW = A^T g; gb = column sums of g; gA = g W^T (kept where gate > 0).
// Workgroup b takes rows [bR, bR + R): its rows of A, all of W and its targets go to
// LDS, zero-padded to whole 16 x 16 tiles, and its three products run on
// v_mfma_f32_16x16x4_f32 (a 16 x 16 tile of D = X Y takes lane l's X[i = l%16][k = l/16]
// and Y[k = l/16][j = l%16] and leaves D[4(l/16) + r][l%16] in register r): z and gA for
// its rows, and its part of gW (the sum over its rows). The softmax runs a lane per
// (row, class): each lane scans its row's maximum and adds its row's exponentials in
// class order, as the reference's loops (cpu_backend.ixx:352-370), then forms its own
// p = e / sum, g = (p - t) / M and loss term (cpu_backend.ixx:375-410); the row's terms
// are subtracted in class order by the row's first lane.
// The workgroups hand their gW parts, g and the rows' terms to the one that arrives
// last through workspace (device-coherent stores and loads, an arrival counter, as the
// split-K GEMM's pieces), and that one writes gW = 0 + part 0 + part 1 + ..., the bias
// gradient as the rows of g added in order from 0 and the loss as the rows' terms added
// in row order, divided by M (the reference's orders), then returns the counter to zero.
constexpr int kHeadMaxThreads = 1024;   // one workgroup for the whole batch
constexpr int kHeadRowThreads = 256;    // a workgroup per block of rows
constexpr int kHeadMaxRows = 256;       // batches (padded to 16) that run in one workgroup
constexpr int kHeadLdsBytes = 128 * 1024;

struct HeadDims {
    int M, K, N;      // logical
    int R, Kp, Np;    // rows per workgroup (a multiple of 16); K and N padded to 16
    int KA, NS;       // LDS row strides of A and of W / z / g: 17 mod 64, so the MFMA
                      // operand reads (16 lanes along one index, 4 along the other) hit
                      // at most two lanes per bank
    int G;            // softmax lanes per row: 16, 32 or 64 (>= N)
    int parts;        // workgroups
    FastDiv dKA;      // division by K / 4 (vector copy of A) or by K
    FastDiv dN;       // division by N
    uint32_t partBytes, gOff, termOff, wsBytes;   // workspace: parts of gW, then g, then terms
};

static int stride17(int v) { return v + ((17 - v % 64) + 64) % 64; }

__device__ __forceinline__ f32x4l mfma16f(float a, float b, const f32x4l& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One 16 x 16 output tile, D = sum over kk of X[i][kk] Y[kk][j], X element (i, kk) at
// px[i * xi + kk * xk] and Y element (kk, j) at py[kk * yk + j * yj] (LDS), kk < kLen
// (a multiple of 16). Two register sets alternate: the next sixteen steps' operands are
// read into one while the MFMAs consume the other (the read past the end repeats the
// last chunk). Even and odd steps accumulate apart and are added at the end (a fixed
// order).
__device__ __forceinline__ void readChunk(float (&x)[4], float (&y)[4], const float* px, int xk, const float* py,
                                          int yk, int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        x[u] = px[(k0 + 4 * u) * xk];
        y[u] = py[(k0 + 4 * u) * yk];
    }
}
__device__ __forceinline__ void mfmaChunk(f32x4l& a0, f32x4l& a1, const float (&x)[4], const float (&y)[4]) {
    a0 = mfma16f(x[0], y[0], a0);
    a1 = mfma16f(x[1], y[1], a1);
    a0 = mfma16f(x[2], y[2], a0);
    a1 = mfma16f(x[3], y[3], a1);
}
__device__ __forceinline__ f32x4l tileProduct(const float* px, int xi, int xk, const float* py, int yk, int yj,
                                              int kLen, int li, int lg) {
    f32x4l a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
    px += li * xi + lg * xk;
    py += lg * yk + li * yj;
    float xa[4], ya[4], xb[4], yb[4];
    readChunk(xa, ya, px, xk, py, yk, 0);
    if (kLen == 16) {   // one chunk
        mfmaChunk(a0, a1, xa, ya);
        return a0 + a1;
    }
    const int lastK = kLen - 16;
    for (int k0 = 0;; k0 += 32) {
        readChunk(xb, yb, px, xk, py, yk, min(k0 + 16, lastK));
        mfmaChunk(a0, a1, xa, ya);
        if (k0 + 16 >= kLen) break;
        readChunk(xa, ya, px, xk, py, yk, min(k0 + 32, lastK));
        mfmaChunk(a0, a1, xb, yb);
        if (k0 + 32 >= kLen) break;
    }
    return a0 + a1;
}

// VEC: A's rows are copied as 16-byte words (K % 4 == 0, A 16-byte aligned).
template <bool VEC>
__global__ void __launch_bounds__(kHeadMaxThreads) linear_ce_rows_kernel(
    const float* __restrict__ A, const float* __restrict__ W, const float* __restrict__ bias,
    const float* __restrict__ T, float* logits, float* loss, float* grad, float* gW, float* gb, float* gA,
    const float* __restrict__ gate, float* ws, unsigned* ctr, HeadDims d, float scale) {
#pragma clang fp contract(off)
    extern __shared__ float hsm[];
    __shared__ int lastFlag;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nT = blockDim.x, nW = nT >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const bool single = d.parts == 1;      // one workgroup: no hand-over
    const int r0 = blockIdx.x * d.R;
    const int rows = min(d.R, d.M - r0);   // real rows of this workgroup
    float* sA = hsm;                       // [R][KA]
    float* sW = sA + d.R * d.KA;           // [Kp][NS]
    float* sG = sW + d.Kp * d.NS;          // [R][NS]: z, then exp(z - max), then g
    float* sT = sG + d.R * d.NS;           // [rows][N]: targets, then loss terms
    float* sL = sT + d.R * d.N;            // [R]: the rows' terms (one workgroup)
    const auto rws = bufferRsrc(ws, d.wsBytes);
    // operands into LDS: each pass issues a thread's global loads (up to 8 units of A,
    // 8 of W and 4 of T) before its LDS stores
    {
        const int KU = VEC ? d.K / 4 : d.K;
        const int cA = rows * KU, cW = d.K * d.N, cT = rows * d.N;   // units to copy
        const float* Ab = A + (long long)r0 * d.K;
        const float* Tb = T + (long long)r0 * d.N;
        for (int it = 0; it * 8 * nT < cA || it * 8 * nT < cW || it * 4 * nT < cT;
             ++it) {
            f32x4 va[8];
            float vw[8], vt[4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int e = (it * 8 + j) * nT + tid;
                if (e < cA) {
                    if constexpr (VEC) va[j] = *reinterpret_cast<const f32x4*>(Ab + 4 * (long long)e);
                    else va[j][0] = Ab[e];
                }
                if (e < cW) vw[j] = W[e];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = (it * 4 + j) * nT + tid;
                if (e < cT) vt[j] = Tb[e];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int e = (it * 8 + j) * nT + tid;
                if (e < cA) {
                    const int m = (int)d.dKA.div((uint32_t)e), u = e - m * KU;
                    if constexpr (VEC) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) sA[m * d.KA + 4 * u + q] = va[j][q];
                    } else {
                        sA[m * d.KA + u] = va[j][0];
                    }
                }
                if (e < cW) {
                    const int k = (int)d.dN.div((uint32_t)e), n = e - k * d.N;
                    sW[k * d.NS + n] = vw[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = (it * 4 + j) * nT + tid;
                if (e < cT) sT[e] = vt[j];
            }
        }
        // zero padding: A's columns past K and rows past the real ones, W's past K and N
        const int padK = d.Kp - d.K, padN = d.Np - d.N;
        if (padK)
            for (int e = tid; e < rows * padK; e += nT) sA[(e / padK) * d.KA + d.K + e % padK] = 0.f;
        for (int e = tid; e < (d.R - rows) * d.Kp; e += nT)
            sA[(rows + e / d.Kp) * d.KA + e % d.Kp] = 0.f;
        if (padN)
            for (int e = tid; e < d.K * padN; e += nT) sW[(e / padN) * d.NS + d.N + e % padN] = 0.f;
        for (int e = tid; e < padK * d.Np; e += nT) sW[(d.K + e / d.Np) * d.NS + e % d.Np] = 0.f;
    }
    __syncthreads();
    // z = A W + b for the workgroup's rows
    {
        const int tn = d.Np / 16, tiles = (d.R / 16) * tn;
        for (int t = wave; t < tiles; t += nW) {
            const int m0 = (t / tn) * 16, n0 = (t % tn) * 16;
            const int n = n0 + li;
            const float bn = (bias && n < d.N) ? bias[n] : 0.f;
            const f32x4l acc = tileProduct(sA + m0 * d.KA, d.KA, 1, sW + n0, d.NS, 1, d.Kp, li, lg);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 4 * lg + r;
                const float z = acc[r] + bn;
                sG[m * d.NS + n] = z;
                if (logits && m < rows && n < d.N) logits[(long long)(r0 + m) * d.N + n] = z;
            }
        }
    }
    __syncthreads();
    // softmax, g and the loss terms. Up to 16 classes: a thread per row with the row in
    // registers (the scans are sequential either way; one thread per row issues each
    // exponential, divide and logarithm once).
    if (d.Np == 16) {
        for (int r = tid; r < d.R; r += nT) {
            float* zr = sG + r * d.NS;
            if (r >= rows) {   // padded rows: g = 0
#pragma unroll
                for (int i = 0; i < 16; ++i) zr[i] = 0.f;
                continue;
            }
            // whole rows of 16 are read: a row of z has 17 slots, the targets' rows are
            // followed by more LDS; the values past N are not used
            float v[16], t[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = zr[i];
#pragma unroll
            for (int i = 0; i < 16; ++i) t[i] = sT[r * d.N + i];
            float mx = v[0];   // the reference's scan: a NaN first element stays
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = (i < d.N && v[i] > mx) ? v[i] : mx;
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i < d.N) {
                    v[i] = expf(v[i] - mx);
                    sum += v[i];
                }
            float term = 0.f;
            const long long o = (long long)(r0 + r) * d.N;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float g = 0.f;
                if (i < d.N) {
                    const float p = v[i] / sum;
                    if (t[i] > 0.5f) term -= logf(p < 1e-7f ? 1e-7f : p);
                    g = (p - t[i]) * scale;
                    if (!single) bufStore1Agent(rws, d.gOff + (uint32_t)(o + i) * 4u, 0, g);
                    if (grad) grad[o + i] = g;
                }
                zr[i] = g;
            }
            if (single) sL[r] = term;
            else bufStore1Agent(rws, d.termOff + (uint32_t)(r0 + r) * 4u, 0, term);
        }
    } else {
        // 17 to 64 classes: a lane per (row, class), G lanes per row, a row's
        // lanes in one wave (padded rows and classes: g = 0)
        const int per = 64 / d.G;   // rows per wave and pass
        const int j = lane % d.G;
        for (int rb = wave * per; rb < d.R; rb += nW * per) {
            const int r = rb + lane / d.G;
            float* zr = sG + r * d.NS;
            const bool real = r < rows && j < d.N;
            float g = 0.f;
            if (r < rows) {
                // the row's maximum as the reference's scan: a NaN first element stays
                // (whole chunks of 16 are read: a row of z has Np + 1 >= 16 slots, the targets'
                // rows are followed by more LDS; the values past N are not used)
                float mx = zr[0];
                for (int c0 = 0; c0 < d.N; c0 += 16) {
                    float v[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) v[i] = zr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i) mx = (c0 + i < d.N && v[i] > mx) ? v[i] : mx;
                }
                const float e = real ? expf(zr[j] - mx) : 0.f;
                __builtin_amdgcn_wave_barrier();
                if (real) zr[j] = e;
                __builtin_amdgcn_wave_barrier();
                float sum = 0.f;   // + 0 for the classes past N: exact
                for (int c0 = 0; c0 < d.N; c0 += 16) {
                    float v[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) v[i] = zr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i) sum += c0 + i < d.N ? v[i] : 0.f;
                }
                float lt = 0.f;   // subtracted from the row's term: exact for the classes that add none
                if (real) {
                    const float p = e / sum;
                    const float t = sT[r * d.N + j];
                    if (t > 0.5f) lt = logf(p < 1e-7f ? 1e-7f : p);
                    g = (p - t) * scale;
                }
                __builtin_amdgcn_wave_barrier();
                if (real) sT[r * d.N + j] = lt;
                __builtin_amdgcn_wave_barrier();
                if (j == 0) {
                    float term = 0.f;
                    for (int c0 = 0; c0 < d.N; c0 += 16) {
                        float v[16];
#pragma unroll
                        for (int i = 0; i < 16; ++i) v[i] = sT[r * d.N + c0 + i];
#pragma unroll
                        for (int i = 0; i < 16; ++i) term -= c0 + i < d.N ? v[i] : 0.f;
                    }
                    if (single) sL[r] = term;
                    else bufStore1Agent(rws, d.termOff + (uint32_t)(r0 + r) * 4u, 0, term);
                }
                if (real) {
                    const long long o = (long long)(r0 + r) * d.N + j;
                    if (!single) bufStore1Agent(rws, d.gOff + (uint32_t)o * 4u, 0, g);
                    if (grad) grad[o] = g;
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (j < d.Np) zr[j] = g;
        }
    }
    __syncthreads();
    if (single) {
        // the loss (thread 0) and the bias gradient (a thread per class of the second
        // wave) from LDS, while the other waves start on the products
        if (loss && tid == 0) {
            float tot = 0.f;
            int r = 0;
            for (; r + 16 <= d.M; r += 16) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = sL[r + i];
#pragma unroll
                for (int i = 0; i < 16; ++i) tot += v[i];
            }
            for (; r < d.M; ++r) tot += sL[r];
            loss[0] = tot / (float)d.M;
        }
        const int n = tid - 64;
        if (gb && n >= 0 && n < d.N) {
            float acc = 0.f;
            int m = 0;
            for (; m + 16 <= d.M; m += 16) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = sG[(m + i) * d.NS + n];
#pragma unroll
                for (int i = 0; i < 16; ++i) acc += v[i];
            }
            for (; m < d.M; ++m) acc += sG[m * d.NS + n];
            gb[n] = acc;
        }
    }
    // gA = g W^T for the workgroup's rows ([R][Kp], reduction over Np), kept where the
    // gate is positive. Each tile is computed transposed (W g^T), so that a lane holds
    // four consecutive columns of one row: with K % 4 == 0 and 16-byte aligned rows, the
    // gate is one 16-byte load and the output one 16-byte store.
    if (gA) {
        const int tk = d.Kp / 16, tiles = (d.R / 16) * tk;
        const bool vec4 = d.K % 4 == 0 && (reinterpret_cast<uintptr_t>(gA) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(gate) & 15) == 0;
        const auto gateAt = [&](int t) {   // the lane's four gate values of tile t (1 where none)
            f32x4 v = {1.f, 1.f, 1.f, 1.f};
            const int m = (t / tk) * 16 + li, kq = (t % tk) * 16 + 4 * lg;
            if (gate && vec4 && t < tiles && m < rows && kq < d.K)
                v = *reinterpret_cast<const f32x4*>(gate + (long long)(r0 + m) * d.K + kq);
            return v;
        };
        // a wave's tiles four at a time: the four gates are loaded before the first product
        for (int t0 = wave; t0 < tiles; t0 += 4 * nW) {
            f32x4 gq[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) gq[q] = gateAt(t0 + q * nW);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = t0 + q * nW;
                if (t >= tiles) break;
                const int m0 = (t / tk) * 16, k0 = (t % tk) * 16;
                const int m = m0 + li, kq = k0 + 4 * lg;
                const f32x4l acc = tileProduct(sW + k0 * d.NS, d.NS, 1, sG + m0 * d.NS, 1, d.NS, d.Np, li, lg);
                if (m >= rows) continue;
                float* out = gA + (long long)(r0 + m) * d.K + kq;
                if (vec4) {
                    if (kq < d.K) {
                        f32x4 o;
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = (gate && !(gq[q][r] > 0.f)) ? 0.f : acc[r];
                        *reinterpret_cast<f32x4*>(out) = o;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kq + r < d.K) {
                            const bool keep = !gate || gate[(long long)(r0 + m) * d.K + kq + r] > 0.f;
                            out[r] = keep ? acc[r] : 0.f;
                        }
                }
            }
        }
    }
    // this workgroup's part of gW = A^T g ([Kp][Np], reduction over its R rows)
    {
        const int tn = d.Np / 16, tiles = (d.Kp / 16) * tn;
        const uint32_t own = (uint32_t)blockIdx.x * d.partBytes;
        for (int t = wave; t < tiles; t += nW) {
            const int k0 = (t / tn) * 16, n0 = (t % tn) * 16;
            const f32x4l acc = tileProduct(sA + k0, 1, d.KA, sG + n0, d.NS, 1, d.R, li, lg);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int k = k0 + 4 * lg + r, n = n0 + li;
                if (!single) bufStore1Agent(rws, (uint32_t)(k * d.Np + n) * 4u, own, acc[r]);
                else if (k < d.K && n < d.N) gW[(long long)k * d.N + n] = acc[r];
            }
        }
    }
    if (single) return;
    // arrival: every wave's stores have completed before thread 0 adds to the counter
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        lastFlag = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (unsigned)(d.parts - 1);
    __syncthreads();
    if (!lastFlag) return;
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // gW = 0 + part 0 + part 1 + ..., four elements and eight parts in flight a thread
    {
        const int cW = d.K * d.N;
        for (int e0 = tid; e0 < cW; e0 += 4 * nT) {
            uint32_t off[4];
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = e0 + i * nT;
                const int k = (int)d.dN.div((uint32_t)e), n = e - k * d.N;
                off[i] = e < cW ? (uint32_t)(k * d.Np + n) * 4u : kOOB;
            }
            for (int b0 = 0; b0 < d.parts; b0 += 8) {
                float v[4][8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t pb = (uint32_t)min(b0 + q, d.parts - 1) * d.partBytes;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i][q] = bufLoad1Agent(rws, off[i], pb);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (b0 + q < d.parts)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i] += v[i][q];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (e0 + i * nT < cW) gW[e0 + i * nT] = acc[i];
        }
    }
    // g and the rows' terms into LDS, then the bias gradient (a thread per class) and
    // the loss (one thread of the second wave)
    if (gb || loss) {
        float* sAll = hsm;   // [M][N] g, then [M] terms
        const int nAll = d.M * d.N + d.M;
        for (int e0 = tid; e0 < nAll; e0 += 16 * nT) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int e = e0 + i * nT;
                v[i] = bufLoad1Agent(rws, e < nAll ? (uint32_t)e * 4u : kOOB, d.gOff);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (e0 + i * nT < nAll) sAll[e0 + i * nT] = v[i];
        }
        __syncthreads();
        if (gb && tid < d.N) {
            float acc = 0.f;
            int m = 0;
            for (; m + 16 <= d.M; m += 16) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = sAll[(m + i) * d.N + tid];
#pragma unroll
                for (int i = 0; i < 16; ++i) acc += v[i];
            }
            for (; m < d.M; ++m) acc += sAll[m * d.N + tid];
            gb[tid] = acc;
        }
        if (loss && tid == 64) {
            const float* terms = sAll + d.M * d.N;
            float tot = 0.f;
            int r = 0;
            for (; r + 16 <= d.M; r += 16) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = terms[r + i];
#pragma unroll
                for (int i = 0; i < 16; ++i) tot += v[i];
            }
            for (; r < d.M; ++r) tot += terms[r];
            loss[0] = tot / (float)d.M;
        }
    }
}

static int checkRows(const char* name, const void* a, const void* b, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return fail("%s: rows and classes must be positive (%d, %d)", name, rows, cols);
    if (!a || !b) return fail("%s: null pointer", name);
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipSoftmax(const float* pIn, float* pOut, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipSoftmax", pIn, pOut, nBatch, nClasses)) return -1;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((nBatch + 3) / 4), dim3(256), 0, stream(), pIn, pOut, nBatch,
                       nClasses);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipCrossEntropy(const float* pSoftmax, const float* pTarget, float* pResult, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipCrossEntropy", pSoftmax, pTarget, nBatch, nClasses)) return -1;
    if (!pResult) return fail("omHipCrossEntropy: null result");
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(1), dim3(64 * kLossWaves), 0, stream(), pSoftmax, pTarget, pResult,
                       nBatch, nClasses);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipSoftmaxCrossEntropyBackward(const float* pSoftmax, const float* pTarget, float* pGradLogits, int nBatch,
                                     int nClasses) {
    clearError();
    if (checkRows("omHipSoftmaxCrossEntropyBackward", pSoftmax, pTarget, nBatch, nClasses)) return -1;
    if (!pGradLogits) return fail("omHipSoftmaxCrossEntropyBackward: null output");
    const float scale = 1.0f / static_cast<float>(nBatch);   // as cpu_backend.ixx:395
    const long long n = (long long)nBatch * nClasses;
    const int blocks = (int)std::min<long long>((n + 255) / 256, (long long)cuCount() * 16);
    hipLaunchKernelGGL(softmax_ce_backward_kernel, dim3(blocks), dim3(256), 0, stream(), pSoftmax, pTarget,
                       pGradLogits, n, scale);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipSoftmaxCrossEntropy(const float* pLogits, const float* pTarget, float* pSoftmax, float* pLoss,
                             float* pGradLogits, int nBatch, int nClasses) {
    clearError();
    if (checkRows("omHipSoftmaxCrossEntropy", pLogits, pTarget, nBatch, nClasses)) return -1;
    if (!pSoftmax && !pGradLogits && (long long)kLossWaves * nClasses > (1LL << 20))
        return fail("omHipSoftmaxCrossEntropy: %d classes need the softmax or gradient output", nClasses);
    float* rowBuf = nullptr;
    if (!pSoftmax && !pGradLogits && nClasses > 256) {
        rowBuf = static_cast<float*>(workspace((size_t)kLossWaves * nClasses * sizeof(float)));
        if (!rowBuf) return -1;
    }
    const float scale = 1.0f / static_cast<float>(nBatch);
    if (nClasses <= 64)
        hipLaunchKernelGGL(softmax_ce_fused_reg_kernel<1>, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits,
                           pTarget, pSoftmax, pLoss, pGradLogits, nBatch, nClasses, scale);
    else if (nClasses <= 256)
        hipLaunchKernelGGL(softmax_ce_fused_reg_kernel<4>, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits,
                           pTarget, pSoftmax, pLoss, pGradLogits, nBatch, nClasses, scale);
    else
        hipLaunchKernelGGL(softmax_ce_fused_kernel, dim3(1), dim3(64 * kLossWaves), 0, stream(), pLogits, pTarget,
                           pSoftmax, pLoss, pGradLogits, rowBuf, nBatch, nClasses, scale);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipLinearSoftmaxCrossEntropyStep(const float* pInput, const float* pWeight, const float* pBias,
                                       const float* pTarget, const float* pGate, float* pLogits, float* pLoss,
                                       float* pGradLogits, float* pGradWeight, float* pGradBias, float* pGradInput,
                                       int nBatch, int nIn, int nClasses) {
    clearError();
    const char* name = "omHipLinearSoftmaxCrossEntropyStep";
    if (nBatch <= 0 || nIn <= 0 || nClasses <= 0) return fail("%s: sizes must be positive", name);
    if (!pInput || !pWeight || !pTarget || !pGradWeight) return fail("%s: null pointer", name);
    if (nClasses <= 64) {
        HeadDims d{};
        d.M = nBatch; d.K = nIn; d.N = nClasses;
        d.Kp = (nIn + 15) / 16 * 16; d.Np = (nClasses + 15) / 16 * 16;
        d.KA = stride17(d.Kp); d.NS = stride17(d.Np);
        d.G = d.Np <= 16 ? 16 : d.Np <= 32 ? 32 : 64;
        // LDS of a workgroup of R rows: A, W, z / g, the targets and the rows' terms
        const auto blockFloats = [&](int R) {
            return (long long)R * d.KA + (long long)d.Kp * d.NS + (long long)R * d.NS + (long long)R * d.N + R;
        };
        const int Mp = (nBatch + 15) / 16 * 16;
        const long long last = (long long)nBatch * nClasses + nBatch;   // the last workgroup's g and terms
        long long floats = 0, wsBytes = 0;
        int threads = 0;
        if (Mp <= kHeadMaxRows && blockFloats(Mp) * 4 <= kHeadLdsBytes) {   // the whole batch in one workgroup
            d.R = Mp;
            d.parts = 1;
            floats = blockFloats(Mp);
            threads = kHeadMaxThreads;
        } else if (last * 4 <= kHeadLdsBytes) {
            for (int R = 64; R >= 16 && !threads; R /= 2)
                if (blockFloats(R) * 4 <= kHeadLdsBytes) {
                    d.R = R;
                    d.parts = (nBatch + R - 1) / R;
                    floats = std::max(blockFloats(R), last);
                    threads = kHeadRowThreads;
                }
            const long long part = (long long)d.Kp * d.Np * 4;
            wsBytes = part * d.parts + last * 4;
            d.partBytes = (uint32_t)part;
            d.gOff = (uint32_t)(part * d.parts);
            d.termOff = d.gOff + (uint32_t)nBatch * nClasses * 4u;
            if (wsBytes >= (1LL << 30)) threads = 0;
            d.wsBytes = (uint32_t)wsBytes;
        }
        if (threads) {
            const bool vec = nIn % 4 == 0 && (reinterpret_cast<uintptr_t>(pInput) & 15) == 0;
            d.dKA = FastDiv::make((uint32_t)(vec ? nIn / 4 : nIn));
            d.dN = FastDiv::make((uint32_t)nClasses);
            float* ws = nullptr;
            unsigned* ctr = nullptr;
            if (d.parts > 1) {
                ws = static_cast<float*>(workspace((size_t)wsBytes, kWsPartials));
                if (!ws) return -1;
                ctr = static_cast<unsigned*>(workspace(sizeof(unsigned), kWsCounters));
                if (!ctr) return -1;
            }
            const size_t lds = (size_t)floats * sizeof(float);
            const float scale = 1.0f / static_cast<float>(nBatch);
            if (vec) {
                OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(linear_ce_rows_kernel<true>, kHeadLdsBytes));
                hipLaunchKernelGGL(linear_ce_rows_kernel<true>, dim3(d.parts), dim3(threads), lds, stream(), pInput,
                                   pWeight, pBias, pTarget, pLogits, pLoss, pGradLogits, pGradWeight, pGradBias,
                                   pGradInput, pGate, ws, ctr, d, scale);
            } else {
                OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(linear_ce_rows_kernel<false>, kHeadLdsBytes));
                hipLaunchKernelGGL(linear_ce_rows_kernel<false>, dim3(d.parts), dim3(threads), lds, stream(), pInput,
                                   pWeight, pBias, pTarget, pLogits, pLoss, pGradLogits, pGradWeight, pGradBias,
                                   pGradInput, pGate, ws, ctr, d, scale);
            }
            OMHIP_CHECK_LAUNCH();
            return 0;
        }
    }
    // larger heads: the same step from the separate entries (logits and the
    // gradient of the logits go through workspace when not requested)
    float* z = pLogits;
    float* g = pGradLogits;
    if (!z || !g) {
        float* ws = static_cast<float*>(workspace((size_t)2 * nBatch * nClasses * sizeof(float), kWsStaging));
        if (!ws) return -1;
        if (!z) z = ws;
        if (!g) g = ws + (size_t)nBatch * nClasses;
    }
    if (omHipLinearBiasAct(pInput, pWeight, pBias, z, nBatch, nIn, nClasses, 0)) return -1;
    if (omHipSoftmaxCrossEntropy(z, pTarget, nullptr, pLoss, g, nBatch, nClasses)) return -1;
    return omHipLinearBackward(pInput, g, pWeight, pGate, pGradWeight, pGradBias, pGradInput, nBatch, nIn,
                               nClasses);
}

int omHipAddBiasBackward(const float* pGradOut, float* pGradBias, int nN, int nC, int nHW) {
    clearError();
    if (nC <= 0) return 0;
    if (!pGradBias) return fail("omHipAddBiasBackward: null output");
    if (nN < 0 || nHW < 0) return fail("omHipAddBiasBackward: negative size");
    if (nN == 0 || nHW == 0) return omHipFillZeros(pGradBias, nC);
    if (!pGradOut) return fail("omHipAddBiasBackward: null gradient");
    if (nHW == 1 && nN <= 4096)
        hipLaunchKernelGGL(bias_grad_cols_kernel, dim3((nC + 255) / 256), dim3(256), 0, stream(), pGradOut, pGradBias,
                           nN, nC);
    else if (nHW == 1)
        hipLaunchKernelGGL(bias_grad_cols_parts_kernel, dim3((nC + 63) / 64), dim3(1024), 0, stream(), pGradOut,
                           pGradBias, nN, nC);
    else
        hipLaunchKernelGGL(bias_grad_planes_kernel, dim3(nC), dim3(256), 0, stream(), pGradOut, pGradBias, nN, nC,
                           nHW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // extern "C"
