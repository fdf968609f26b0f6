// pool.hip — pooling and the elementwise add that join the conv layers of a
// ResNet: max / average / adaptive-average pooling (forward and backward) and
// a + b (the residual sum).
//
// Reference: CPUBackend::maxPool2d / maxPool2dBackward / avgPool2d /
// avgPool2dBackward / adaptiveAvgPool2d / adaptiveAvgPool2dBackward / add
// (src/hal/om.hal.cpu_backend.ixx:897-1023, :1467-1510, :147-160); C ABI
// counterparts omCudaMaxPool2d ... omCudaAdaptiveAvgPool2d and omCudaAdd
// (src/cuda/cuda_kernels.cuh:218-245, :74).
//
// All are HBM-bound. Forward kernels run one thread per output. The backward
// kernels are gathers, one thread per input element: it visits the output
// windows covering it in ascending (oh, ow) order and adds their
// contributions in that order — the order in which the reference's scatter
// loop (outputs ascending) adds into that element, so the results are
// bit-identical and no atomics are involved.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>

namespace omhip {

static int gridFor(long long n) {
    return (int)std::max<long long>(1, std::min<long long>((n + 255) / 256, (long long)cuCount() * 16));
}

// Grid over (64-column, 4-row) blocks of a plane and the planes: about 16 k
// workgroups (64 per CU), blockIdx.z walking the further planes. One element
// per thread over every plane at once left the launch bound by workgroup
// dispatch (ResNet stem max-pool backward: 83 us with 115 k workgroups, 59 us
// with 16 k).
static dim3 planeGrid(long long planes, int rows, int cols) {
    const long long bx = (cols + 63) / 64, by = (rows + 3) / 4;
    long long zmax = std::max<long long>(1, 16384 / (bx * by));
    return dim3((unsigned)bx, (unsigned)by,
                (unsigned)std::max<long long>(1, std::min<long long>({planes, zmax, 65535LL})));
}

struct PoolGeom {
    int N, C, H, W, KH, KW, SH, SW, PH, PW, Ho, Wo;
    uint32_t mulH, shH, mulW, shW;   // x / SH == (x * mulH) >> shH for 0 <= x < 2^31 (likewise W)
};

// x / d == (x * mul) >> shift for 0 <= x < 2^31: l = ceil(log2 d), mul =
// floor(2^(31+l) / d) + 1 < 2^32 (Granlund & Montgomery 1994, Thm 4.2).
static void magicDivisor(uint32_t d, uint32_t& mul, uint32_t& shift) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    mul = (uint32_t)((1ull << (31 + l)) / d + 1);
    shift = 31 + l;
}

__device__ __forceinline__ int divMagic(int x, uint32_t mul, uint32_t shift) {
    return (int)(((uint64_t)(uint32_t)x * mul) >> shift);
}

// Window range of outputs covering input coordinate i along one axis:
// o*s - p <= i <= o*s - p + K - 1  ->  o in [ceil((i+p-K+1)/s), floor((i+p)/s)] within [0, O).
__device__ __forceinline__ void coverRange(int i, int K, int s, int p, int O, uint32_t mul, uint32_t shift, int& o0,
                                           int& o1) {
    const int hi = i + p;   // >= 0
    const int lo = hi - K + 1;
    o0 = lo <= 0 ? 0 : divMagic(lo + s - 1, mul, shift);
    o1 = min(divMagic(hi, mul, shift), O - 1);
}

// Kernels run over (column, row, plane): blocks of 64 columns x 4 rows,
// blockIdx.z walking the N*C planes. In-plane indices are 32-bit, the plane
// base 64-bit; no division is needed to locate a pixel.
#define OMHIP_FOR_PLANE_PIXELS(P, ROWS, COLS, r, c)                                          \
    const int c = blockIdx.x * 64 + (int)threadIdx.x;                                        \
    const int r = blockIdx.y * 4 + (int)threadIdx.y;                                         \
    if (c < (COLS) && r < (ROWS))                                                            \
        for (long long pl = blockIdx.z; pl < (P); pl += gridDim.z)

// cpu_backend.ixx:897-934: strict '>' keeps the first maximum in (kh, kw) order;
// index = flat input index, -1 (value -1e30) for a window wholly in the padding.
__global__ void maxpool_kernel(const float* __restrict__ x, float* __restrict__ y, int* __restrict__ idx, PoolGeom g) {
    const long long planes = (long long)g.N * g.C;
    const int S = g.Ho * g.Wo;
    OMHIP_FOR_PLANE_PIXELS(planes, g.Ho, g.Wo, oh, ow) {
        const int px = oh * g.Wo + ow;
        const long long ib = pl * g.H * g.W;
        float best = -1e30f;
        int bi = -1;
        for (int kh = 0; kh < g.KH; ++kh) {
            const int ih = oh * g.SH - g.PH + kh;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                const int iw = ow * g.SW - g.PW + kw;
                if (iw < 0 || iw >= g.W) continue;
                const float v = x[ib + ih * g.W + iw];
                if (v > best) {
                    best = v;
                    bi = (int)(ib + ih * g.W + iw);
                }
            }
        }
        const long long o = pl * S + px;
        y[o] = best;
        if (idx) idx[o] = bi;
    }
}

// The ResNet stem pooling (3x3, stride 2, pad 1; W a multiple of 4, H even):
// one thread per pair of outputs (oh, 2j), (oh, 2j+1), whose windows cover
// input columns 4j-1 .. 4j+3. Each window row is one 16-byte load of columns
// 4j .. 4j+3 plus column 4j-1 from the neighbouring lane (a load of its own
// for lane 0). The candidates are scanned in the same (kh, kw) order with the
// same strict '>' as maxpool_kernel, so values and indices are identical.
__global__ void maxpool_3s2_kernel(const float* __restrict__ x, float* __restrict__ y, int* __restrict__ idx,
                                   long long planes, int H, int W) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int Ho = H / 2, Wo = W / 2, J = W / 4;
    const long long total = planes * Ho * J;
    const int lane = threadIdx.x & 63;
    // every lane of a wave runs the same trip count (the shuffle needs the whole wave)
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long t0 = blockIdx.x * (long long)blockDim.x + (threadIdx.x & ~63); t0 < total; t0 += stride) {
        const long long t = t0 + lane;
        const bool active = t < total;
        const long long tt = active ? t : total - 1;
        const int j = (int)(tt % J);
        const long long r = tt / J;
        const int oh = (int)(r % Ho);
        const long long pl = r / Ho;
        const long long ib = pl * H * W;
        float best0 = -1e30f, best1 = -1e30f;
        int bi0 = -1, bi1 = -1;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
            const int ih = 2 * oh - 1 + kh;
            const bool rowOk = ih >= 0;   // ih <= H-1 always
            const long long rb = ib + (long long)(rowOk ? ih : 0) * W;
            const f4 q = rowOk ? *reinterpret_cast<const f4*>(x + rb + 4 * j) : f4{0.f, 0.f, 0.f, 0.f};
            float left = __shfl_up(q[3], 1, 64);
            if (lane == 0 && j > 0 && rowOk) left = x[rb + 4 * j - 1];
            if (rowOk) {
                const int c0 = (int)(rb - ib) + 4 * j;   // in-plane index of column 4j
                // output 2j: columns 4j-1, 4j, 4j+1
                if (j > 0 && left > best0) { best0 = left; bi0 = (int)(ib + c0 - 1); }
                if (q[0] > best0) { best0 = q[0]; bi0 = (int)(ib + c0); }
                if (q[1] > best0) { best0 = q[1]; bi0 = (int)(ib + c0 + 1); }
                // output 2j+1: columns 4j+1, 4j+2, 4j+3
                if (q[1] > best1) { best1 = q[1]; bi1 = (int)(ib + c0 + 1); }
                if (q[2] > best1) { best1 = q[2]; bi1 = (int)(ib + c0 + 2); }
                if (q[3] > best1) { best1 = q[3]; bi1 = (int)(ib + c0 + 3); }
            }
        }
        if (active) {
            const long long o = (pl * Ho + oh) * Wo + 2 * j;
            typedef float f2 __attribute__((ext_vector_type(2)));
            typedef int i2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<f2*>(y + o) = f2{best0, best1};
            if (idx) *reinterpret_cast<i2*>(idx + o) = i2{bi0, bi1};
        }
    }
}

// Backward of the stem pooling as a gather over 2x2 input blocks: input rows
// 2a, 2a+1 and columns 2i, 2i+1 are covered only by outputs (a or a, a+1) x
// (i or i, i+1), so a thread reads those four outputs once and adds, for each
// of its four inputs, the gradients of the covering outputs whose saved index
// is that input, in ascending (oh, ow) order as maxpool_backward_kernel does.
__global__ void maxpool_3s2_backward_kernel(const float* __restrict__ gO, const int* __restrict__ idx,
                                            float* __restrict__ gI, long long planes, int H, int W) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int Ho = H / 2, Wo = W / 2;
    const long long total = planes * Ho * Wo;   // one thread per 2x2 input block
    for (long long t = blockIdx.x * (long long)blockDim.x + threadIdx.x; t < total;
         t += (long long)gridDim.x * blockDim.x) {
        const int i = (int)(t % Wo);
        const long long r = t / Wo;
        const int a = (int)(r % Ho);
        const long long pl = r / Ho;
        const long long ob = pl * Ho * Wo;
        const bool a1 = a + 1 < Ho, i1 = i + 1 < Wo;
        const long long o00 = ob + (long long)a * Wo + i;
        const int x00 = idx[o00];
        const int x01 = i1 ? idx[o00 + 1] : -1;
        const int x10 = a1 ? idx[o00 + Wo] : -1;
        const int x11 = (a1 && i1) ? idx[o00 + Wo + 1] : -1;
        const float g00 = gO[o00];
        const float g01 = i1 ? gO[o00 + 1] : 0.f;
        const float g10 = a1 ? gO[o00 + Wo] : 0.f;
        const float g11 = (a1 && i1) ? gO[o00 + Wo + 1] : 0.f;
        const long long ib = pl * H * W;
        const int f = (int)(ib + (long long)(2 * a) * W + 2 * i);   // flat index of input (2a, 2i)
        // (2a, 2i): output (a, i) only
        const float v00 = x00 == f ? 0.f + g00 : 0.f;   // 0 + g as the running sum would give (-0 -> +0)
        // (2a, 2i+1): outputs (a, i), (a, i+1)
        float v01 = 0.f;
        if (x00 == f + 1) v01 += g00;
        if (x01 == f + 1) v01 += g01;
        // (2a+1, 2i): outputs (a, i), (a+1, i)
        float v10 = 0.f;
        if (x00 == f + W) v10 += g00;
        if (x10 == f + W) v10 += g10;
        // (2a+1, 2i+1): outputs (a, i), (a, i+1), (a+1, i), (a+1, i+1)
        float v11 = 0.f;
        if (x00 == f + W + 1) v11 += g00;
        if (x01 == f + W + 1) v11 += g01;
        if (x10 == f + W + 1) v11 += g10;
        if (x11 == f + W + 1) v11 += g11;
        *reinterpret_cast<f2*>(gI + f) = f2{v00, v01};
        *reinterpret_cast<f2*>(gI + f + W) = f2{v10, v11};
    }
}

// cpu_backend.ixx:937-955 as a gather: gI[i] = sum of gO[o] over the outputs o
// (ascending) whose saved index is i.
__global__ void maxpool_backward_kernel(const float* __restrict__ gO, const int* __restrict__ idx,
                                        float* __restrict__ gI, PoolGeom g) {
    const long long planes = (long long)g.N * g.C;
    const int S = g.H * g.W;
    OMHIP_FOR_PLANE_PIXELS(planes, g.H, g.W, ih, iw) {
        const int px = ih * g.W + iw;
        const long long i = pl * S + px;
        const long long ob = pl * g.Ho * g.Wo;
        int oh0, oh1, ow0, ow1;
        coverRange(ih, g.KH, g.SH, g.PH, g.Ho, g.mulH, g.shH, oh0, oh1);
        coverRange(iw, g.KW, g.SW, g.PW, g.Wo, g.mulW, g.shW, ow0, ow1);
        float v = 0.f;
        if (oh1 - oh0 <= 1 && ow1 - ow0 <= 1) {
            // at most 2 x 2 covering windows (K <= 2*stride): issue every load, then
            // add the matching ones in ascending (oh, ow) order
            const int oh1c = max(oh1, oh0), ow1c = max(ow1, ow0);
            const long long o00 = ob + oh0 * g.Wo + ow0, o01 = ob + oh0 * g.Wo + ow1c;
            const long long o10 = ob + oh1c * g.Wo + ow0, o11 = ob + oh1c * g.Wo + ow1c;
            const bool r0 = oh0 <= oh1, r1 = oh1 > oh0, c0 = ow0 <= ow1, c1 = ow1 > ow0;
            const int i00 = (r0 && c0) ? idx[o00] : -1, i01 = (r0 && c1) ? idx[o01] : -1;
            const int i10 = (r1 && c0) ? idx[o10] : -1, i11 = (r1 && c1) ? idx[o11] : -1;
            const float g00 = (r0 && c0) ? gO[o00] : 0.f, g01 = (r0 && c1) ? gO[o01] : 0.f;
            const float g10 = (r1 && c0) ? gO[o10] : 0.f, g11 = (r1 && c1) ? gO[o11] : 0.f;
            if (i00 == (int)i) v += g00;
            if (i01 == (int)i) v += g01;
            if (i10 == (int)i) v += g10;
            if (i11 == (int)i) v += g11;
        } else {
            for (int oh = oh0; oh <= oh1; ++oh)
                for (int ow = ow0; ow <= ow1; ++ow) {
                    const long long o = ob + oh * g.Wo + ow;
                    if (idx[o] == (int)i) v += gO[o];
                }
        }
        gI[i] = v;
    }
}

__global__ void zero_kernel(float* __restrict__ p, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        p[i] = 0.f;
}

// cpu_backend.ixx:937-955 with the reference's signature (no window geometry):
// scatter through the saved indices with atomic adds. An input that is the
// maximum of several windows receives their gradients in an unspecified order
// (at most ceil(K/s)^2 of them); omHipMaxPool2dBackwardEx is the ordered,
// bit-reproducible gather when the window geometry is known.
__global__ void maxpool_scatter_kernel(const float* __restrict__ gO, const int* __restrict__ idx, float* gI,
                                       long long nout, long long nin) {
    for (long long o = blockIdx.x * (long long)blockDim.x + threadIdx.x; o < nout;
         o += (long long)gridDim.x * blockDim.x) {
        const int t = idx[o];
        if (t >= 0 && t < nin) atomicAdd(gI + t, gO[o]);
    }
}

// cpu_backend.ixx:958-990: sum over the valid taps divided by KH*KW.
__global__ void avgpool_kernel(const float* __restrict__ x, float* __restrict__ y, PoolGeom g) {
    const long long planes = (long long)g.N * g.C;
    const int S = g.Ho * g.Wo;
    const float div = (float)(g.KH * g.KW);
    OMHIP_FOR_PLANE_PIXELS(planes, g.Ho, g.Wo, oh, ow) {
        const int px = oh * g.Wo + ow;
        const long long ib = pl * g.H * g.W;
        float sum = 0.f;
        for (int kh = 0; kh < g.KH; ++kh) {
            const int ih = oh * g.SH - g.PH + kh;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw) {
                const int iw = ow * g.SW - g.PW + kw;
                if (iw < 0 || iw >= g.W) continue;
                sum += x[ib + ih * g.W + iw];
            }
        }
        y[pl * S + px] = sum / div;
    }
}

// cpu_backend.ixx:994-1023 as a gather: each covering output adds gO * (1/(KH*KW)).
// The reference rounds the product before adding it (separate statements), so
// the multiply must not be fused into the add here.
__global__ void avgpool_backward_kernel(const float* __restrict__ gO, float* __restrict__ gI, PoolGeom g) {
#pragma clang fp contract(off)
    const long long planes = (long long)g.N * g.C;
    const int S = g.H * g.W;
    const float scale = 1.0f / (float)(g.KH * g.KW);
    OMHIP_FOR_PLANE_PIXELS(planes, g.H, g.W, ih, iw) {
        const int px = ih * g.W + iw;
        const long long ob = pl * g.Ho * g.Wo;
        int oh0, oh1, ow0, ow1;
        coverRange(ih, g.KH, g.SH, g.PH, g.Ho, g.mulH, g.shH, oh0, oh1);
        coverRange(iw, g.KW, g.SW, g.PW, g.Wo, g.mulW, g.shW, ow0, ow1);
        float v = 0.f;
        for (int oh = oh0; oh <= oh1; ++oh)
            for (int ow = ow0; ow <= ow1; ++ow) v += gO[ob + oh * g.Wo + ow] * scale;
        gI[pl * S + px] = v;
    }
}

// cpu_backend.ixx:1467-1488: region [floor(o*H/OH), floor((o+1)*H/OH)) per axis;
// an empty region divides 0 by 0, as the reference does.
__global__ void adaptive_avgpool_kernel(const float* __restrict__ x, float* __restrict__ y, int NC, int H, int W,
                                        int OH, int OW) {
    const long long total = (long long)NC * OH * OW;
    for (long long o = blockIdx.x * (long long)blockDim.x + threadIdx.x; o < total;
         o += (long long)gridDim.x * blockDim.x) {
        const int ow = (int)(o % OW);
        const int oh = (int)((o / OW) % OH);
        const long long nc = o / ((long long)OW * OH);
        const int h0 = (int)((long long)oh * H / OH), h1 = (int)((long long)(oh + 1) * H / OH);
        const int w0 = (int)((long long)ow * W / OW), w1 = (int)((long long)(ow + 1) * W / OW);
        float sum = 0.f;
        int cnt = 0;
        for (int ih = h0; ih < h1; ++ih)
            for (int iw = w0; iw < w1; ++iw) {
                sum += x[(nc * H + ih) * W + iw];
                ++cnt;
            }
        y[o] = sum / (float)cnt;
    }
}

// The global case (OH = OW = 1, a plane of at most kGlobalPoolMaxHW pixels: the
// network's final pooling): a workgroup copies 64 consecutive planes into LDS
// with coalesced loads, then each of 64 threads adds its plane in the order
// above (rows, then columns, from 0) and divides by the count: the same
// result, without a thread per plane striding over 64 planes per load.
constexpr int kGlobalPoolPlanes = 64, kGlobalPoolMaxHW = 256;
__global__ __launch_bounds__(256) void global_avgpool_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             int NC, int HW) {
    __shared__ float tile[kGlobalPoolPlanes * kGlobalPoolMaxHW];
    const long long nc0 = (long long)blockIdx.x * kGlobalPoolPlanes;
    const int planes = (int)min<long long>(kGlobalPoolPlanes, NC - nc0);
    const int n = planes * HW;
    const float* src = x + nc0 * HW;
    for (int i = threadIdx.x; i < n; i += blockDim.x) tile[i] = src[i];
    __syncthreads();
    if ((int)threadIdx.x < planes) {
        const float* t = tile + threadIdx.x * HW;
        float sum = 0.f;
        for (int i = 0; i < HW; ++i) sum += t[i];
        y[nc0 + threadIdx.x] = sum / (float)HW;
    }
}

// cpu_backend.ixx:1491-1510: the regions partition the input (each region's end
// is the next one's start), so every input element takes gO / count of its one region.
__global__ void adaptive_avgpool_backward_kernel(const float* __restrict__ gO, float* __restrict__ gI, int NC, int H,
                                                 int W, int OH, int OW) {
    const long long total = (long long)NC * H * W;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const int iw = (int)(i % W);
        const int ih = (int)((i / W) % H);
        const long long nc = i / ((long long)W * H);
        // the region o with floor(o*H/OH) <= ih < floor((o+1)*H/OH)
        int oh = (int)(((long long)ih * OH) / H);
        while (oh + 1 < OH && (long long)(oh + 1) * H / OH <= ih) ++oh;
        while (oh > 0 && (long long)oh * H / OH > ih) --oh;
        int ow = (int)(((long long)iw * OW) / W);
        while (ow + 1 < OW && (long long)(ow + 1) * W / OW <= iw) ++ow;
        while (ow > 0 && (long long)ow * W / OW > iw) --ow;
        const int h0 = (int)((long long)oh * H / OH), h1 = (int)((long long)(oh + 1) * H / OH);
        const int w0 = (int)((long long)ow * W / OW), w1 = (int)((long long)(ow + 1) * W / OW);
        const float g = gO[(nc * OH + oh) * OW + ow] / (float)((h1 - h0) * (w1 - w0));
        gI[i] = g;
    }
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
                           long long n) {
    const long long n4 = n / 4;
    const long long stride = (long long)gridDim.x * blockDim.x;
    const long long t = blockIdx.x * (long long)blockDim.x + threadIdx.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(c)) & 15u) == 0;
    if (vec) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        for (long long i = t; i < n4; i += stride) {
            const f4 u = reinterpret_cast<const f4*>(a)[i], v = reinterpret_cast<const f4*>(b)[i];
            reinterpret_cast<f4*>(c)[i] = u + v;
        }
        for (long long i = n4 * 4 + t; i < n; i += stride) c[i] = a[i] + b[i];
    } else {
        for (long long i = t; i < n; i += stride) c[i] = a[i] + b[i];
    }
}

// 3x3 window, stride 2, pad 1 over an even H and W (the ResNet stem pooling):
// Ho = H/2, Wo = W/2 and the outputs tile the input in 2x2 blocks.
static bool stemPool(const PoolGeom& g) {
    return g.KH == 3 && g.KW == 3 && g.SH == 2 && g.SW == 2 && g.PH == 1 && g.PW == 1 && g.H % 2 == 0 &&
           g.W % 2 == 0;
}
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
static bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }   // null passes

static int poolGeom(const char* name, int N, int C, int H, int W, int KH, int KW, int SH, int SW, int PH, int PW,
                    PoolGeom& g) {
    if (N <= 0 || C <= 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0 || PH < 0 || PW < 0)
        return fail("%s: invalid geometry", name);
    g = {N, C, H, W, KH, KW, SH, SW, PH, PW, (H + 2 * PH - KH) / SH + 1, (W + 2 * PW - KW) / SW + 1, 0, 0, 0, 0};
    magicDivisor((uint32_t)SH, g.mulH, g.shH);
    magicDivisor((uint32_t)SW, g.mulW, g.shW);
    if (g.Ho <= 0 || g.Wo <= 0) return fail("%s: window larger than the padded input", name);
    if ((long long)N * C * H * W >= (1LL << 31)) return fail("%s: input exceeds 2^31 elements (int indices)", name);
    if (H > 4 * 65535) return fail("%s: more than %d rows", name, 4 * 65535);
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipMaxPool2d(const float* pIn, float* pOut, int* pIndices, int nN, int nC, int nH, int nW, int nKH, int nKW,
                   int nSH, int nSW, int nPH, int nPW) {
    clearError();
    PoolGeom g;
    if (poolGeom("omHipMaxPool2d", nN, nC, nH, nW, nKH, nKW, nSH, nSW, nPH, nPW, g)) return -1;
    if (!pIn || !pOut) return fail("omHipMaxPool2d: null pointer");
    if (stemPool(g) && nW % 4 == 0 && aligned16(pIn) && aligned8(pOut) && aligned8(pIndices)) {
        const long long planes = (long long)nN * nC;
        hipLaunchKernelGGL(maxpool_3s2_kernel, dim3(gridFor(planes * g.Ho * (nW / 4))), dim3(256), 0, stream(), pIn,
                           pOut, pIndices, planes, nH, nW);
        OMHIP_CHECK_LAUNCH();
        return 0;
    }
    hipLaunchKernelGGL(maxpool_kernel, planeGrid((long long)nN * nC, g.Ho, g.Wo), dim3(64, 4), 0, stream(), pIn,
                       pOut, pIndices, g);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipMaxPool2dBackward(const float* pGradOut, const int* pIndices, float* pGradIn, int nN, int nC, int nH, int nW,
                           int nHout, int nWout) {
    clearError();
    if (nN <= 0 || nC <= 0 || nH <= 0 || nW <= 0 || nHout <= 0 || nWout <= 0)
        return fail("omHipMaxPool2dBackward: invalid geometry");
    if (!pGradOut || !pIndices || !pGradIn) return fail("omHipMaxPool2dBackward: null pointer");
    const long long nin = (long long)nN * nC * nH * nW, nout = (long long)nN * nC * nHout * nWout;
    if (nin >= (1LL << 31)) return fail("omHipMaxPool2dBackward: input exceeds 2^31 elements (int indices)");
    hipLaunchKernelGGL(zero_kernel, dim3(gridFor(nin)), dim3(256), 0, stream(), pGradIn, nin);
    OMHIP_CHECK_LAUNCH();
    hipLaunchKernelGGL(maxpool_scatter_kernel, dim3(gridFor(nout)), dim3(256), 0, stream(), pGradOut, pIndices,
                       pGradIn, nout, nin);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipMaxPool2dBackwardEx(const float* pGradOut, const int* pIndices, float* pGradIn, int nN, int nC, int nH,
                             int nW, int nKH, int nKW, int nSH, int nSW, int nPH, int nPW) {
    clearError();
    PoolGeom g;
    if (poolGeom("omHipMaxPool2dBackwardEx", nN, nC, nH, nW, nKH, nKW, nSH, nSW, nPH, nPW, g)) return -1;
    if (!pGradOut || !pIndices || !pGradIn) return fail("omHipMaxPool2dBackwardEx: null pointer");
    if (stemPool(g) && aligned8(pGradIn)) {
        const long long planes = (long long)nN * nC;
        hipLaunchKernelGGL(maxpool_3s2_backward_kernel, dim3(gridFor(planes * g.Ho * g.Wo)), dim3(256), 0, stream(),
                           pGradOut, pIndices, pGradIn, planes, nH, nW);
        OMHIP_CHECK_LAUNCH();
        return 0;
    }
    hipLaunchKernelGGL(maxpool_backward_kernel, planeGrid((long long)nN * nC, nH, nW), dim3(64, 4), 0, stream(),
                       pGradOut, pIndices, pGradIn, g);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAvgPool2d(const float* pIn, float* pOut, int nN, int nC, int nH, int nW, int nKH, int nKW, int nSH, int nSW,
                   int nPH, int nPW) {
    clearError();
    PoolGeom g;
    if (poolGeom("omHipAvgPool2d", nN, nC, nH, nW, nKH, nKW, nSH, nSW, nPH, nPW, g)) return -1;
    if (!pIn || !pOut) return fail("omHipAvgPool2d: null pointer");
    hipLaunchKernelGGL(avgpool_kernel, planeGrid((long long)nN * nC, g.Ho, g.Wo), dim3(64, 4), 0, stream(), pIn,
                       pOut, g);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAvgPool2dBackward(const float* pGradOut, float* pGradIn, int nN, int nC, int nH, int nW, int nKH, int nKW,
                           int nSH, int nSW, int nPH, int nPW) {
    clearError();
    PoolGeom g;
    if (poolGeom("omHipAvgPool2dBackward", nN, nC, nH, nW, nKH, nKW, nSH, nSW, nPH, nPW, g)) return -1;
    if (!pGradOut || !pGradIn) return fail("omHipAvgPool2dBackward: null pointer");
    hipLaunchKernelGGL(avgpool_backward_kernel, planeGrid((long long)nN * nC, nH, nW), dim3(64, 4), 0, stream(),
                       pGradOut, pGradIn, g);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAdaptiveAvgPool2d(const float* pIn, float* pOut, int nN, int nC, int nH, int nW, int nOutH, int nOutW) {
    clearError();
    if (nN <= 0 || nC <= 0 || nH <= 0 || nW <= 0 || nOutH <= 0 || nOutW <= 0)
        return fail("omHipAdaptiveAvgPool2d: invalid geometry");
    if (!pIn || !pOut) return fail("omHipAdaptiveAvgPool2d: null pointer");
    const long long nc = (long long)nN * nC, hw = (long long)nH * nW;
    if (nOutH == 1 && nOutW == 1 && hw <= kGlobalPoolMaxHW &&
        (nc + kGlobalPoolPlanes - 1) / kGlobalPoolPlanes <= 0x7fffffffLL) {
        hipLaunchKernelGGL(global_avgpool_kernel, dim3((unsigned)((nc + kGlobalPoolPlanes - 1) / kGlobalPoolPlanes)),
                           dim3(256), 0, stream(), pIn, pOut, (int)nc, (int)hw);
        OMHIP_CHECK_LAUNCH();
        return 0;
    }
    hipLaunchKernelGGL(adaptive_avgpool_kernel, dim3(gridFor((long long)nN * nC * nOutH * nOutW)), dim3(256), 0,
                       stream(), pIn, pOut, nN * nC, nH, nW, nOutH, nOutW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAdaptiveAvgPool2dBackward(const float* pGradOut, float* pGradIn, int nN, int nC, int nH, int nW, int nOutH,
                                   int nOutW) {
    clearError();
    if (nN <= 0 || nC <= 0 || nH <= 0 || nW <= 0 || nOutH <= 0 || nOutW <= 0)
        return fail("omHipAdaptiveAvgPool2dBackward: invalid geometry");
    if (!pGradOut || !pGradIn) return fail("omHipAdaptiveAvgPool2dBackward: null pointer");
    hipLaunchKernelGGL(adaptive_avgpool_backward_kernel, dim3(gridFor((long long)nN * nC * nH * nW)), dim3(256), 0,
                       stream(), pGradOut, pGradIn, nN * nC, nH, nW, nOutH, nOutW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int omHipAdd(const float* pA, const float* pB, float* pC, int nCount) {
    clearError();
    if (nCount <= 0) return 0;
    if (!pA || !pB || !pC) return fail("omHipAdd: null pointer");
    hipLaunchKernelGGL(add_kernel, dim3(gridFor((nCount + 3) / 4)), dim3(256), 0, stream(), pA, pB, pC,
                       (long long)nCount);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

}  // extern "C"
