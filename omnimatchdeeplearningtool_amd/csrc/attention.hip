// attention.hip — fused multi-head attention for fp16 / bf16 inputs:
// QKV split + scaled Q.K^T + row softmax + P.V + head merge in one kernel.
//
// Reference: MultiHeadAttention::forward (src/engine/om.engine.vit.ixx:150-239):
// split the QKV projection into heads with Q scaled (qkvSplitHeads), scores =
// Q x K^T (tensorTranspose2dBatched + tensorBatchedMatmul), softmax over the
// keys (CPUBackend::softmax cpu_backend.ixx:352-370: max, exp(x - max), sum,
// divide), context = P x V, merge heads — five passes that write the S x S
// score and probability matrices to memory. Here one workgroup owns one
// (image, head): K and V^T for all keys stay in LDS, and each wave takes 16
// queries at a time: it computes their score rows with v_mfma_f32_16x16x32,
// does the softmax on the full row in registers (the row fits, so no running
// rescale), rounds P to half precision in registers — already laid out as
// the A operand of P x V — and multiplies by V^T. Only the QKV rows are read
// and the context is written.
//
// Layouts: qkv [B*S, 3*H*D] half (row = token; Q | K | V, each head-major
// [H][D]); out [B*S, H*D] (merged heads), fp32 or the input's half type.
// D is 64 (ViT-B/16); S <= 384 (all keys in LDS).
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>

namespace omhip {

namespace {

typedef _Float16 f16x8a __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8a __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));
typedef float f32x4a __attribute__((ext_vector_type(4)));

constexpr int kD = 64;          // head dimension
constexpr int kLdK = kD + 8;    // halves per K row in LDS
constexpr int kMaxSeq = 384;

#ifndef OMHIP_ATTN_SPLIT
#define OMHIP_ATTN_SPLIT 0   // 1: one workgroup per (image, head, block of 128 queries); measured slower on ViT-B/16 (37 vs 34 us)
#endif

struct AttnParams {
    const uint16_t* qkv;
    void* out;
    int B, S, H, SP;    // SP: keys padded to a multiple of 32
    long long ldq;      // 3*H*D
    long long ldo;      // H*D
    float scale;
};

template <bool BF16>
__device__ __forceinline__ f32x4a mfma16(const u32x4a& a, const u32x4a& b, const f32x4a& c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8a, a), __builtin_bit_cast(bf16x8a, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8a, a), __builtin_bit_cast(f16x8a, b), c,
                                                      0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ uint16_t toHalf(float v) {   // round to nearest even
    if constexpr (BF16)
        return __builtin_bit_cast(uint16_t, (__bf16)v);
    else
        return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Two floats rounded to nearest even into the half type, low then high.
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16)
        return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
    else
        return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

__device__ __forceinline__ uint32_t pickHalves(uint32_t lo, uint32_t hi, bool upper) {
    // (lo.half[upper], hi.half[upper]) packed low-to-high
    return __builtin_amdgcn_perm(hi, lo, upper ? 0x07060302u : 0x05040100u);
}

// Reductions across the four 16-lane groups (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float maxAcross4(float v) {
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float sumAcross4(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// One workgroup of NW waves per (image, head); NT = SP/16 key tiles per score
// row. Every global load of the head (K, V, and the Q fragments of all query
// blocks) is issued before the first LDS store, so the workgroup waits for
// memory once. After K and V^T are in LDS the waves are independent: each
// owns 16 query rows per block of NW*16 queries and its own rows of P.
template <bool BF16, bool OUT_HALF, int NT, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void attention_kernel(AttnParams p) {
    extern __shared__ uint16_t sm[];
    constexpr int SP = NT * 16;
    constexpr int NTH = NW * 64;
    constexpr int ldv = SP + 8;                   // halves per V^T row
    constexpr int QB = NW * 16;                   // queries per block
    constexpr int NIT = (SP + QB - 1) / QB;       // query blocks (upper bound: S <= SP)
    constexpr int KPT = (SP * 8 + NTH - 1) / NTH; // 16-byte K chunks per thread
    constexpr int VPT = (SP + NTH - 1) / NTH;     // 8x8 V blocks per thread (SP/8 x 8 blocks)
    uint16_t* sK = sm;                            // [SP][kLdK]
    uint16_t* sVt = sK + SP * kLdK;               // [kD][ldv]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;    // MFMA lane group: k chunk 8*g4, output rows 4*g4..4*g4+3
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const uint16_t* rowQ = p.qkv + (long long)b * p.S * p.ldq + (long long)h * kD;
    const uint16_t* rowK = rowQ + (long long)p.H * kD;
    const uint16_t* rowV = rowQ + 2LL * p.H * kD;
    const u32x4a zero = {0u, 0u, 0u, 0u};

    // ---- all global loads of the head ----
    u32x4a kr[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int e = tid + i * NTH;
        const int j = e >> 3, c = (e & 7) * 8;
        kr[i] = (e < SP * 8 && j < p.S) ? *reinterpret_cast<const u32x4a*>(rowK + (long long)j * p.ldq + c) : zero;
    }
    u32x4a vr[VPT][8];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int blk = tid + i * NTH;
        const int jb = blk >> 3, db = (blk & 7) * 8;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int j = jb * 8 + t;
            vr[i][t] = (blk < SP && j < p.S) ? *reinterpret_cast<const u32x4a*>(rowV + (long long)j * p.ldq + db)
                                             : zero;
        }
    }
    // With SPLIT, workgroup y of the head takes query block y only.
    constexpr int NQ = SPLIT ? 1 : NIT;
    const int it0 = SPLIT ? (int)blockIdx.y : 0;
    u32x4a qr[NQ][2];
#pragma unroll
    for (int iq = 0; iq < NQ; ++iq) {
        const int it = it0 + iq;
        const int qa = it * QB + wave * 16 + l16;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            qr[iq][ks] = (qa < p.S) ? *reinterpret_cast<const u32x4a*>(rowQ + (long long)qa * p.ldq + ks * 32 + g4 * 8)
                                    : zero;
    }
    // ---- K rows and V^T (8x8 register transposes) into LDS ----
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int e = tid + i * NTH;
        if (e < SP * 8) *reinterpret_cast<u32x4a*>(sK + (e >> 3) * kLdK + (e & 7) * 8) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int blk = tid + i * NTH;
        if (blk >= SP) continue;
        const int jb = blk >> 3, db = (blk & 7) * 8;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int w = d >> 1;
            const bool up = (d & 1) != 0;
            const u32x4a col = {pickHalves(vr[i][0][w], vr[i][1][w], up), pickHalves(vr[i][2][w], vr[i][3][w], up),
                                pickHalves(vr[i][4][w], vr[i][5][w], up), pickHalves(vr[i][6][w], vr[i][7][w], up)};
            *reinterpret_cast<u32x4a*>(sVt + (db + d) * ldv + jb * 8) = col;
        }
    }
    __syncthreads();

    constexpr float kLog2e = 1.4426950408889634f;
    const float sl2 = p.scale * kLog2e;
#pragma unroll
    for (int iq = 0; iq < NQ; ++iq) {
        const int q0 = (it0 + iq) * QB + wave * 16;
        if (q0 >= p.S) break;   // wave-uniform; nothing below synchronises the workgroup
        // Transposed scores (K as the first operand): lane (l16, g4) holds
        // s[t][r] = S[query q0 + l16][key 16*t + 4*g4 + r], so each query's row sits
        // in the four 16-lane groups that share l16.
        f32x4a s[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f32x4a acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const u32x4a kf = *reinterpret_cast<const u32x4a*>(sK + (t * 16 + l16) * kLdK + ks * 32 + g4 * 8);
                acc = mfma16<BF16>(kf, qr[iq][ks], acc);
            }
            s[t] = acc;
        }
        // softmax of the row: max, exp(x - max), sum, normalise. exp is v_exp_f32 of
        // (x - max) * scale * log2(e) and the normalisation a reciprocal multiply,
        // both well inside the half-precision rounding P receives next.
        float m = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = (t * 16 + g4 * 4 + r < p.S) ? s[t][r] * sl2 : -INFINITY;
                s[t][r] = v;
                m = fmaxf(m, v);
            }
        m = maxAcross4(m);
        float sum = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(s[t][r] - m);   // exp2(-inf) = 0 for padded keys
                s[t][r] = e;
                sum += e;
            }
        const float inv = __builtin_amdgcn_rcpf(sumAcross4(sum));
        // P stays in registers as the A operand of P x V. In MFMA step ks the lane
        // group g4 supplies keys {32ks + 4g4 + r, 32ks + 16 + 4g4 + r} (r = 0..3),
        // the tiles t = 2ks and 2ks+1 it already holds; V^T is read in the same
        // key order, so the sum over keys is unchanged.
        u32x4a pf[NT / 2];
#pragma unroll
        for (int ks = 0; ks < NT / 2; ++ks) {
            const f32x4a& a0 = s[2 * ks];
            const f32x4a& a1 = s[2 * ks + 1];
            pf[ks] = u32x4a{pack2<BF16>(a0[0] * inv, a0[1] * inv), pack2<BF16>(a0[2] * inv, a0[3] * inv),
                            pack2<BF16>(a1[0] * inv, a1[1] * inv), pack2<BF16>(a1[2] * inv, a1[3] * inv)};
        }
        // context: O[query][d] = sum_key P[query][key] V^T[d][key]
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            f32x4a acc = {0.f, 0.f, 0.f, 0.f};
            const uint16_t* vrow = sVt + (dt * 16 + l16) * ldv + g4 * 4;
#pragma unroll
            for (int ks = 0; ks < NT / 2; ++ks) {
                typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
                const u32x2a lo = *reinterpret_cast<const u32x2a*>(vrow + ks * 32);
                const u32x2a hi = *reinterpret_cast<const u32x2a*>(vrow + ks * 32 + 16);
                const u32x4a vb = {lo[0], lo[1], hi[0], hi[1]};
                acc = mfma16<BF16>(pf[ks], vb, acc);
            }
            // output rows are queries q0 + 4*g4 + r, columns d = dt*16 + l16
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = q0 + g4 * 4 + r;
                if (qi >= p.S) continue;
                const long long o = ((long long)b * p.S + qi) * p.ldo + (long long)h * kD + dt * 16 + l16;
                if constexpr (OUT_HALF)
                    static_cast<uint16_t*>(p.out)[o] = toHalf<BF16>(acc[r]);
                else
                    static_cast<float*>(p.out)[o] = acc[r];
            }
        }
    }
}

template <bool BF16, bool OUT_HALF, int NT, int NW>
int launchAttnT(const AttnParams& prm) {
    constexpr int NIT = (NT * 16 + NW * 16 - 1) / (NW * 16);
    auto kern = attention_kernel<BF16, OUT_HALF, NT, NW, (OMHIP_ATTN_SPLIT != 0)>;
    constexpr int SP = NT * 16;
    constexpr size_t lds = (size_t)(SP * kLdK + kD * (SP + 8)) * sizeof(uint16_t);   // K, V^T
    static_assert(lds <= 160 * 1024, "attention tile exceeds LDS");
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    const int nq = OMHIP_ATTN_SPLIT ? std::min(NIT, (prm.S + NW * 16 - 1) / (NW * 16)) : 1;
    hipLaunchKernelGGL(kern, dim3(prm.B * prm.H, nq), dim3(NW * 64), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// Key tiles (16 keys each) are a compile-time count: SP = 32 * ceil(S / 32).
// Eight waves per workgroup; LDS holds K and V^T only (62 KB at 224 keys).
template <bool BF16, bool OUT_HALF>
int launchAttn(const AttnParams& prm) {
    switch (prm.SP / 16) {
#define OMHIP_ATTN_CASE(n, nw) \
    case n: return launchAttnT<BF16, OUT_HALF, n, nw>(prm);
        OMHIP_ATTN_CASE(2, 8) OMHIP_ATTN_CASE(4, 8) OMHIP_ATTN_CASE(6, 8) OMHIP_ATTN_CASE(8, 8) OMHIP_ATTN_CASE(10, 8)
        OMHIP_ATTN_CASE(12, 8) OMHIP_ATTN_CASE(14, 8) OMHIP_ATTN_CASE(16, 8) OMHIP_ATTN_CASE(18, 8)
        OMHIP_ATTN_CASE(20, 8) OMHIP_ATTN_CASE(22, 8) OMHIP_ATTN_CASE(24, 8)
#undef OMHIP_ATTN_CASE
        default: return fail("omHipAttentionHalf: unsupported padded sequence length %d", prm.SP);
    }
}

}  // namespace

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipAttentionHalf(int nDtype, const uint16_t* pQKV, void* pOut, int nOutHalf, int nBatch, int nSeq, int nHeads,
                       int nHeadDim, float fScale) {
    clearError();
    if (nBatch <= 0 || nSeq <= 0 || nHeads <= 0) return 0;
    if (!pQKV || !pOut) return fail("omHipAttentionHalf: null pointer");
    if (nDtype != 0 && nDtype != 1) return fail("omHipAttentionHalf: dtype must be 0 (fp16) or 1 (bf16)");
    if (nHeadDim != kD) return fail("omHipAttentionHalf: head dimension %d (this kernel: 64)", nHeadDim);
    if (nSeq > kMaxSeq) return fail("omHipAttentionHalf: sequence length %d exceeds %d", nSeq, kMaxSeq);
    if (((reinterpret_cast<uintptr_t>(pQKV)) & 15u) != 0) return fail("omHipAttentionHalf: qkv must be 16-byte aligned");
    if ((long long)nBatch * nHeads > 0x7fffffffLL) return fail("omHipAttentionHalf: too many (image, head) pairs");
    AttnParams prm{};
    prm.qkv = pQKV;
    prm.out = pOut;
    prm.B = nBatch;
    prm.S = nSeq;
    prm.H = nHeads;
    prm.SP = (nSeq + 31) / 32 * 32;
    prm.ldq = 3LL * nHeads * kD;
    prm.ldo = (long long)nHeads * kD;
    prm.scale = fScale;
    if (nDtype == 1) return nOutHalf ? launchAttn<true, true>(prm) : launchAttn<true, false>(prm);
    return nOutHalf ? launchAttn<false, true>(prm) : launchAttn<false, false>(prm);
}

}  // extern "C"
