// attention.hip — fused multi-head attention for fp16 / bf16 inputs:
// QKV split + scaled Q.K^T + row softmax + P.V + head merge in one kernel.
//
// Reference: MultiHeadAttention::forward (src/engine/om.engine.vit.ixx:150-239):
// split the QKV projection into heads with Q scaled (qkvSplitHeads), scores =
// Q x K^T (tensorTranspose2dBatched + tensorBatchedMatmul), softmax over the
// keys (CPUBackend::softmax cpu_backend.ixx:352-370: max, exp(x - max), sum,
// divide), context = P x V, merge heads — five passes that write the S x S
// score and probability matrices to memory. Here one kernel reads the QKV
// rows once and writes only the context.
//
// Layouts: qkv [B*S, 3*H*D] half (row = token; Q | K | V, each head-major
// [H][D]); out [B*S, H*D] (merged heads), fp32 or the input's half type.
// D is 64 (ViT-B/16); S <= 384 (all keys in LDS).
//
// One workgroup per (image, head). K and V rows of the head go straight from
// memory into LDS (buffer_load ... lds, 16 keys per tile, NT = ceil(S/16)
// tiles: 4 KB of LDS per tile, 52 KB at 197 tokens); rows past S read as
// zeros. Each wave takes blocks of 16 queries:
//  * scores S^T = K . Q^T with v_mfma_f32_16x16x32 (K from LDS as the first
//    operand, Q fragments straight from memory): lane (l16, g4) holds
//    S[query q0 + l16][key 16t + 4 g4 + r] for tile t, r = 0..3, so each
//    query's row lives in the four 16-lane groups that share l16;
//  * softmax on the full row in registers: m = max_j s_j, e_j = exp2(s_j c
//    - m c) with c = scale log2(e) (one fma and one v_exp_f32 per score);
//    e_j in [0, 1] is rounded to the half type as the second operand of P.V,
//    the row sum of the rounded e_j comes from one more MFMA per step (a d
//    tile of ones), and 1/sum is applied to the context at the end;
//  * context^T = V^T . P^T: V^T fragments come from V's natural [key][d] LDS
//    rows through ds_read_b64_tr_b16 (lane i of a 16-lane group receives
//    element E[4j + i/4][i%4] of what the group addressed), so lane (l16, g4)
//    ends up with 4 consecutive d of query q0 + l16 and stores them at once.
// The key order inside a P.V step (keys 32ks + 4g4 + r and 32ks + 16 + 4g4 +
// r) is the order of the score tiles the lane holds; the sum over keys is
// order-free, so only rounding order differs from the reference chain.
// Latency hiding inside a wave: the first block's Q fragments load under the
// K / V copy and each later block's during the previous block's math; the
// transposing V^T reads of P.V step ks + 1 are in flight during step ks's
// MFMAs.
#include "omhip_internal.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace omhip {

namespace {

typedef _Float16 f16x8a __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8a __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
typedef float f32x4a __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* LdsPtrA;

constexpr int kD = 64;          // head dimension
constexpr int kMaxSeq = 384;
constexpr uint32_t kOOBA = 0x40000000u;   // an offset past every view

struct AttnParams {
    const uint16_t* qkv;
    void* out;
    int B, S, H;
    long long ldq;      // 3*H*D
    long long ldo;      // H*D
    float scale;
    int outVec;         // the output allows 4-element stores (base and ldo aligned)
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

// Two floats rounded to nearest even into the half type, low then high (one
// v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32).
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef float f32x2c __attribute__((ext_vector_type(2)));
    if constexpr (BF16) {
        typedef __bf16 bf16x2c __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2c{a, b}, bf16x2c));
    } else {
        typedef _Float16 f16x2c __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2c{a, b}, f16x2c));
    }
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

__device__ __forceinline__ void dmaRow16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtrA)dst, 16, voff, 0, 0, 0);
}

// LDS rows are 64 halves (8 chunks of 16 bytes), unpadded. Chunk c of K row r
// sits in slot c ^ ((r >> 1) & 7): the 16 lanes of a quarter-wave read one
// chunk of 16 consecutive rows and hit 16 distinct 16-byte bank groups. Chunk
// c of V row r sits in slot c ^ (2 ((r >> 1) & 3)): a transposing read takes
// two chunks of 8 consecutive rows per 32 lanes, again 16 distinct groups.
__device__ __forceinline__ int kSlot(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int vSlot(int r, int c) { return c ^ (2 * ((r >> 1) & 3)); }

// Per-lane LDS offsets (halves): the K fragment of step ks at tile 0 (row
// l16, chunk 4ks + g4) and the V^T fragment of d tile dt at step 0 (row
// 4 g4 + l16/4, columns 16 dt + 4 (l16 % 4)); rows further on add whole
// 16-row tiles, which keep the slot swizzle.
struct AttnLane {
    uint32_t kOff[2], vOff[4];
    __device__ void init(int l16, int g4) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) kOff[ks] = (uint32_t)(l16 * kD + (kSlot(l16, 4 * ks + g4) << 3));
        const int vr = 4 * g4 + (l16 >> 2);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int c = 2 * dt + ((l16 & 3) >> 1);
            vOff[dt] = (uint32_t)(vr * kD + (vSlot(vr, c) << 3) + 4 * (l16 & 1));
        }
    }
};

// K and V rows of head (b, h) into sK / sV, 8 rows per instruction; rows >= S
// read as zeros. Instructions i = first, first + step, ... < SP / 8.
template <int SP>
__device__ __forceinline__ void dmaHead(const AttnParams& p, int b, int h, uint16_t* sK, uint16_t* sV, int first,
                                        int step, int lane) {
    const uint16_t* rowK = p.qkv + (long long)b * p.S * p.ldq + (long long)(p.H + h) * kD;
    const uint16_t* rowV = rowK + (long long)p.H * kD;
    const uint32_t ldq2 = (uint32_t)p.ldq * 2u;
    const uint32_t view = (uint32_t)(p.S - 1) * ldq2 + kD * 2u;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(rowK), 0, (int)view, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(rowV), 0, (int)view, 0x00020000);
    const int rsub = lane >> 3, slot = lane & 7;
    for (int i = first; i < SP / 8; i += step) {
        const int r = i * 8 + rsub;
        const uint32_t rb = r < p.S ? (uint32_t)r * ldq2 : kOOBA;
        dmaRow16(rk, sK + i * 512, rb + (uint32_t)kSlot(r, slot) * 16u);
        dmaRow16(rv, sV + i * 512, rb + (uint32_t)vSlot(r, slot) * 16u);
    }
}

// Q fragments of the 16 queries q0 .. q0+15 (lane: query q0 + l16, d 32ks + 8g4 ..).
__device__ __forceinline__ void loadQ(const AttnParams& p, int b, int h, int qa, int g4, u32x4a (&qf)[2]) {
    const u32x4a zero = {0u, 0u, 0u, 0u};
    const uint16_t* rowQ = p.qkv + (long long)b * p.S * p.ldq + (long long)h * kD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        qf[ks] = qa < p.S ? *reinterpret_cast<const u32x4a*>(rowQ + (long long)qa * p.ldq + ks * 32 + g4 * 8) : zero;
}

// One block of 16 queries against all keys of the head in sK / sV: scores,
// softmax (unnormalised weights; 1/sum of the rounded weights returned in
// inv) and the context,
// o[dt][r] = sum_key e * V[key][16 dt + 4 g4 + r] for query q0 + l16.
template <bool BF16, int NT>
__device__ __forceinline__ void attnBlock(const uint16_t* sK, uint32_t sVa, const AttnLane& L, const u32x4a (&qf)[2],
                                          int S, float c, int g4, f32x4a (&o)[4], float& inv) {
    constexpr int NKS = (NT + 1) / 2;   // P.V steps of 32 keys
    f32x4a s[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        f32x4a acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const u32x4a kf = *reinterpret_cast<const u32x4a*>(sK + L.kOff[ks] + t * 16 * kD);
            acc = mfma16<BF16>(kf, qf[ks], acc);
        }
        s[t] = acc;
    }
    // Keys past S exist only in the last tile: their scores are excluded from
    // the max and their weights set to 0. With c < 0 the order flips, so the
    // maximum of s*c is c times the minimum of s.
    const int lastValid = S - 16 * (NT - 1) - 4 * g4;   // valid r in the last tile: r < lastValid
    auto extreme = [&](auto negTag) {
        constexpr bool NEG = decltype(negTag)::value;
        float m = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = NEG ? -s[t][r] : s[t][r];
                if (t == NT - 1 && r >= lastValid) v = -INFINITY;
                m = fmaxf(m, v);
            }
        return maxAcross4(m);
    };
    const float mc = c < 0.f ? -extreme(std::true_type{}) * c : extreme(std::false_type{}) * c;   // max of s*c
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][r], c, -mc));
            if (t == NT - 1 && r >= lastValid) e = 0.f;
            s[t][r] = e;
        }
    // The row sum comes from the matrix cores: a fifth d tile of ones makes
    // rs[r] = sum_key e (the rounded weights, the same ones P.V uses).
    const uint32_t one2 = BF16 ? 0x3f803f80u : 0x3c003c00u;
    const u32x4a ones = {one2, one2, one2, one2};
    f32x4a rs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4a{0.f, 0.f, 0.f, 0.f};
    // V^T fragments of step ks: rows 32ks + 4g4 + j (first read) and + 16
    // (second read; a missing tile re-reads the first rows, whose weights are
    // zero), into buffer ks & 1. Step ks + 1's reads are issued before step
    // ks's MFMAs; LDS reads return in order, so "at most 8 outstanding" means
    // step ks's 8 have landed. The reads are inline assembly and waited for
    // here: through the builtin the compiler would also wait for any LDS DMA
    // in flight, i.e. for every global load still outstanding. The wait does
    // not depend on what else the compiler places around the reads: other LDS
    // operations complete in order with them and scalar loads only add to the
    // count, so "at most 8 outstanding" can only be reached once every
    // operation older than step ks + 1's 8 reads has completed (the 8 volatile
    // reads keep their order, and the waits' "memory" clobber keeps the
    // compiler's own LDS accesses on their side of the wait).
    u32x2a lo[2][4], up[2][4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        const uint32_t a = sVa + 2u * L.vOff[dt];
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo[0][dt]) : "v"(a), "i"(0));
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(up[0][dt]) : "v"(a), "i"(NT > 1 ? 16 * kD * 2 : 0));
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < NKS) {
            const bool hin = 2 * (ks + 1) + 1 < NT;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint32_t a = sVa + 2u * L.vOff[dt];
                asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                             : "=v"(lo[cur ^ 1][dt]) : "v"(a), "i"((ks + 1) * 32 * kD * 2));
                asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                             : "=v"(up[cur ^ 1][dt]) : "v"(a), "i"((ks + 1) * 32 * kD * 2 + (hin ? 16 * kD * 2 : 0)));
            }
            asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
        } else {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        const f32x4a& a0 = s[2 * ks];
        constexpr int dummy = 0;
        const bool hi = 2 * ks + 1 < NT;   // the second score tile of this step exists
        const f32x4a& a1 = s[hi ? 2 * ks + 1 : dummy];
        const u32x4a pf = {pack2<BF16>(a0[0], a0[1]), pack2<BF16>(a0[2], a0[3]), hi ? pack2<BF16>(a1[0], a1[1]) : 0u,
                           hi ? pack2<BF16>(a1[2], a1[3]) : 0u};
        rs = mfma16<BF16>(ones, pf, rs);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            asm volatile("" : "+v"(lo[cur][dt]), "+v"(up[cur][dt]));
            const u32x4a vf = {lo[cur][dt][0], lo[cur][dt][1], up[cur][dt][0], up[cur][dt][1]};
            o[dt] = mfma16<BF16>(vf, pf, o[dt]);
        }
    }
    inv = __builtin_amdgcn_rcpf(rs[0]);
}

// Context row segment of one lane: O[query][16 dt + 4 g4 + r] = o[dt][r] * inv
// at element offset ob (+ 16 dt).
template <bool BF16, bool OUT_HALF>
__device__ __forceinline__ void storeBlock(const AttnParams& p, long long ob, const f32x4a (&o)[4], float inv) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        const float v0 = o[dt][0] * inv, v1 = o[dt][1] * inv, v2 = o[dt][2] * inv, v3 = o[dt][3] * inv;
        if constexpr (OUT_HALF) {
            uint16_t* op = static_cast<uint16_t*>(p.out) + ob + 16 * dt;
            if (p.outVec) {
                *reinterpret_cast<u32x2a*>(op) = u32x2a{pack2<BF16>(v0, v1), pack2<BF16>(v2, v3)};
            } else {
                op[0] = toHalf<BF16>(v0); op[1] = toHalf<BF16>(v1); op[2] = toHalf<BF16>(v2); op[3] = toHalf<BF16>(v3);
            }
        } else {
            float* op = static_cast<float*>(p.out) + ob + 16 * dt;
            if (p.outVec) {
                // streaming store: 23.2 -> 22.0 us at ViT-B/16 b64 (for the
                // 8-byte half stores it was slower)
                __builtin_nontemporal_store(f32x4a{v0, v1, v2, v3}, reinterpret_cast<f32x4a*>(op));
            } else {
                op[0] = v0; op[1] = v1; op[2] = v2; op[3] = v3;
            }
        }
    }
}

__device__ __forceinline__ long long outOffset(const AttnParams& p, int b, int h, int qa, int g4) {
    return ((long long)b * p.S + qa) * p.ldo + (long long)h * kD + 4 * g4;
}

// One workgroup of NW waves per head (S up to 384); wave w takes query
// blocks w, w + NW, ...
template <bool BF16, bool OUT_HALF, int NT, int NW>
__global__ __launch_bounds__(NW * 64) void attention_kernel(AttnParams p) {
    extern __shared__ uint16_t sm[];
    constexpr int SP = NT * 16;
    uint16_t* sK = sm;
    uint16_t* sV = sm + SP * kD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g4 = lane >> 4;
    const int b = blockIdx.x / p.H, h = blockIdx.x % p.H;
    u32x4a qf[2];
    loadQ(p, b, h, wave * 16 + l16, g4, qf);   // the first block's queries load under the K / V copy
    dmaHead<SP>(p, b, h, sK, sV, wave, NW, lane);
    AttnLane L;
    L.init(l16, g4);
    const uint32_t sVa = (uint32_t)(uintptr_t)(LdsPtrA)sV;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's LDS DMA landed
    __syncthreads();
    constexpr float kLog2e = 1.4426950408889634f;
    const float c = p.scale * kLog2e;
    const int nb = (p.S + 15) >> 4;
    for (int jb = wave; jb < nb; jb += NW) {   // wave-uniform; nothing below synchronises the workgroup
        const int qa = jb * 16 + l16;
        u32x4a qn[2] = {qf[0], qf[1]};
        if (jb + NW < nb) loadQ(p, b, h, qa + NW * 16, g4, qn);   // the next block's queries
        f32x4a o[4];
        float inv;
        attnBlock<BF16, NT>(sK, sVa, L, qf, p.S, c, g4, o, inv);
        if (qa < p.S) storeBlock<BF16, OUT_HALF>(p, outOffset(p, b, h, qa, g4), o, inv);
        qf[0] = qn[0];
        qf[1] = qn[1];
    }
}

// Key tiles (16 keys each) are a compile-time count: NT = ceil(S / 16).
// Eight waves per head: at 197 tokens (122 VGPRs, 52 KB of LDS) two heads share
// a CU, and the 768 heads of ViT-B/16 at batch 64 run in 1.5 rounds, whose
// second half loads while the first computes; measured against 4 waves
// (three heads per CU, one round), two or three workgroups per head and a
// persistent two-stage kernel that copies the next head under this head's
// math, it was as fast or faster (22.3–23.5 against 23.1–25.3 µs).
template <bool BF16, bool OUT_HALF, int NT>
int launchAttnT(const AttnParams& prm) {
    constexpr int NW = 8;
    auto kern = attention_kernel<BF16, OUT_HALF, NT, NW>;
    constexpr size_t lds = (size_t)2 * NT * 16 * kD * sizeof(uint16_t);   // K and V rows
    static_assert(lds <= 160 * 1024, "attention tile exceeds LDS");
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    hipLaunchKernelGGL(kern, dim3(prm.B * prm.H), dim3(NW * 64), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

template <bool BF16, bool OUT_HALF>
int launchAttn(const AttnParams& prm) {
    switch ((prm.S + 15) / 16) {
#define OMHIP_ATTN_CASE(n) \
    case n: return launchAttnT<BF16, OUT_HALF, n>(prm);
        OMHIP_ATTN_CASE(1) OMHIP_ATTN_CASE(2) OMHIP_ATTN_CASE(3) OMHIP_ATTN_CASE(4) OMHIP_ATTN_CASE(5) OMHIP_ATTN_CASE(6)
        OMHIP_ATTN_CASE(7) OMHIP_ATTN_CASE(8) OMHIP_ATTN_CASE(9) OMHIP_ATTN_CASE(10) OMHIP_ATTN_CASE(11) OMHIP_ATTN_CASE(12)
        OMHIP_ATTN_CASE(13) OMHIP_ATTN_CASE(14) OMHIP_ATTN_CASE(15) OMHIP_ATTN_CASE(16) OMHIP_ATTN_CASE(17)
        OMHIP_ATTN_CASE(18) OMHIP_ATTN_CASE(19) OMHIP_ATTN_CASE(20) OMHIP_ATTN_CASE(21) OMHIP_ATTN_CASE(22)
        OMHIP_ATTN_CASE(23) OMHIP_ATTN_CASE(24)
#undef OMHIP_ATTN_CASE
        default: return fail("omHipAttentionHalf: unsupported sequence length %d", prm.S);
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
    prm.ldq = 3LL * nHeads * kD;
    prm.ldo = (long long)nHeads * kD;
    prm.scale = fScale;
    const uintptr_t oAlign = nOutHalf ? 7u : 15u;
    prm.outVec = ((reinterpret_cast<uintptr_t>(pOut) & oAlign) == 0 && (prm.ldo % 4) == 0) ? 1 : 0;
    if ((long long)(nSeq - 1) * prm.ldq * 2 + 2 * kD >= (1LL << 30))
        return fail("omHipAttentionHalf: a head's rows span more than 2^30 bytes");
    if (nDtype == 1) return nOutHalf ? launchAttn<true, true>(prm) : launchAttn<true, false>(prm);
    return nOutHalf ? launchAttn<false, true>(prm) : launchAttn<false, false>(prm);
}

}  // extern "C"
