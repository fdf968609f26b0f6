// gemm_f32.hip — fp32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Entry points: omHipMatmul / MatmulTransB / MatmulTransA / BatchedMatmul /
// BatchedMatmulTransB / GemmStridedBatched. They replace the reference's
// omCudaMatmul (src/cuda/cuda_kernels.cu:768-804) and omCudaBatchedMatmul
// (:843-878) and compute what CPUBackend::matmul / batchedMatmul compute
// (src/hal/om.hal.cpu_backend.ixx:239-286, :1520-1532); the transposed
// variants replace the reference's explicit transpose2d + matmul compositions
// (src/engine/om.engine.autograd.ixx:261-286).
#include "omhip_internal.hpp"
#include "mfma_f32_tile.hpp"
#include "buffer_io.hpp"
#include "gemm_f32.hpp"
#include "../../include/omhip.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace omhip {

// Dense operand loader through range-checked buffer loads, 16-byte vectors
// along the contiguous axis (element (r,k) at P[r*ld + k] when KMAJOR, at
// P[k*ld + r] otherwise). A thread's byte offsets inside the tile are fixed
// at init, rows past the matrix get kOOB (read as zeros), and each slice
// re-bases the buffer view at the slice's first element with scalar
// arithmetic: a whole slice is PER_T buffer loads and no vector ALU work.
// Only the last, partial slice of a K range tests k per vector.
// Host conditions (bufVecOk): the vector layout of DenseLoader (contiguous
// axis, ld and base multiples of 4 floats) and every in-tile offset below
// 2^30 bytes.
template <bool KMAJOR, int R, int BK, int NT>
struct BufVecLoader {
    static constexpr int PER_T = R * BK / 4 / NT;
    static_assert(R * BK % (NT * 4) == 0, "tile must split evenly over threads");
    using Shape = LdsShape<KMAJOR, R, BK>;

    const float* tile;   // element (r0, k = 0) of the operand
    long long ld;
    uint32_t voff[PER_T];
    f32x4 v4[PER_T];

    static __device__ __forceinline__ void coords(int e, int& r, int& k) {
        if constexpr (KMAJOR) { r = e / (BK / 4); k = (e % (BK / 4)) * 4; }
        else { k = e / (R / 4); r = (e % (R / 4)) * 4; }
    }

    __device__ void init(const float* p, long long ld_, int rows, int r0, int tid) {
        ld = ld_;
        tile = KMAJOR ? p + (long long)r0 * ld : p + r0;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int r, k;
            coords(tid + i * NT, r, k);
            voff[i] = (r0 + r < rows) ? (uint32_t)((KMAJOR ? r * ld + k : k * ld + r) * 4) : kOOB;
        }
    }

    // FULL: the slice [k0, k0 + BK) lies inside [0, kEnd).
    template <bool FULL>
    __device__ void load(int k0, int kEnd, int tid) {
        const auto rs = bufferRsrc(tile + (KMAJOR ? (long long)k0 : (long long)k0 * ld), kMaxBufferBytes);
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            uint32_t o = voff[i];
            if constexpr (!FULL) {
                int r, k;
                coords(tid + i * NT, r, k);
                if (k0 + k >= kEnd) o = kOOB;
            }
            v4[i] = bufLoad4(rs, o, 0);
        }
    }

    __device__ void store(float* s, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            int r, k;
            coords(tid + i * NT, r, k);
            float* dst = KMAJOR ? s + r * Shape::LD + k : s + k * Shape::LD + r;
            *reinterpret_cast<f32x4*>(dst) = v4[i];
        }
    }
};

// The generic loader behind the same interface (any alignment, 64-bit
// addressing, per-element bounds tests on every slice).
template <bool KMAJOR, bool VEC, int R, int BK, int NT>
struct DenseLoaderAdapter : DenseLoader<KMAJOR, VEC, R, BK, NT> {
    using Base = DenseLoader<KMAJOR, VEC, R, BK, NT>;
    __device__ void init(const float* p, long long ld, int rows, int r0, int) {
        this->p = p; this->ld = ld; this->rows = rows; this->r0 = r0;
    }
    template <bool FULL>
    __device__ void load(int k0, int kEnd, int tid) {
        this->K = kEnd;
        Base::load(k0, tid);
    }
};

// Operand loader kinds: 0 generic scalar, 1 generic 16-byte vectors,
// 2 buffer-view 16-byte vectors.
template <bool KMAJOR, int LK, int R, int BK, int NT>
using GemmLoader = std::conditional_t<LK == 2, BufVecLoader<KMAJOR, R, BK, NT>,
                                      DenseLoaderAdapter<KMAJOR, LK == 1, R, BK, NT>>;

// Split-K arrival of one piece of a tile. The piece's accumulators go to its
// slot of ws in the tile's own register layout ([split][batch][tile] blocks of
// BM x BN floats, a lane's 16 values of a fragment as four 16-byte words), with
// device-coherent (sc1) stores; once every wave's stores have completed (each
// waits on its own, the block barrier orders them before the add), thread 0
// bumps the tile's counter. The piece that arrives last replaces acc by
// 0 + part 0 + part 1 + ... in split order (device-coherent loads, four splits
// in flight), resets the counter for the next launch and returns true; the
// others return false. The sum order does not depend on which piece arrives
// last, so the result is deterministic.
//
// Ordering. Every access to the exchanged data is an sc1 buffer access, the
// encoding of a monotonic agent-scope atomic load / store in the gfx942 /
// gfx950 memory model: it is performed at the device coherence point, past
// the per-XCD L2s. A piece's stores have completed there (vmcnt 0) before its
// counter add is issued, and the last piece's loads are issued after its add
// has returned, so they read every piece's data. An agent-scope release /
// acquire on the counter would add an L2 write-back (buffer_wbl2 sc1) to every
// arrival and an L2 invalidate (buffer_inv sc1) to the last one; both exist to
// make non-coherent (non-sc1) accesses visible, and none cross between the
// pieces here. Measured on MI355X, they cost 128 x 4096 x 4096 42.5 -> 52.6 us
// (release on the add and acquire in the last piece: 50.5) and 512^3 11.3 ->
// 13.6 us.
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));

template <class Cfg>
__device__ __forceinline__ bool splitArrive(const GemmF32Params& p, f32x16 (&acc)[Cfg::FM][Cfg::FN], float* smem,
                                            int lane, long long batch, int split, int bid) {
    constexpr int TILE = Cfg::BM * Cfg::BN;   // floats per tile and split
    constexpr int LANE_FLOATS = Cfg::FM * Cfg::FN * 16;
    const long long tiles = (long long)p.tilesM * p.tilesN * gridDim.z;
    const long long slot = batch * p.tilesM * p.tilesN + bid;
    // byte offset of this lane's first word in split 0's block of the tile
    const uint32_t laneOff = (uint32_t)((threadIdx.x >> 6) * 64 * LANE_FLOATS + lane * 4) * 4u;
    const auto rw = bufferRsrc(p.ws, (uint32_t)(tiles * p.splits * TILE * 4));
    const uint32_t own = (uint32_t)(((long long)split * tiles + slot) * TILE * 4);
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = {acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1], acc[fm][fn][4 * q + 2], acc[fm][fn][4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4s, v), rw,
                                                       laneOff + (uint32_t)((fm * Cfg::FN + fn) * 4 + q) * 1024u, own,
                                                       kCpolAgent);
            }
    __builtin_amdgcn_s_waitcnt(0);   // this wave's partial stores have completed
    int* flag = reinterpret_cast<int*>(smem);
    __syncthreads();                 // every wave's have (and the LDS stages are free)
    unsigned* ctr = p.ctr + slot;
    if (threadIdx.x == 0)
        *flag = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(p.splits - 1);
    __syncthreads();
    if (!*flag) return false;
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.f;
    const uint32_t stride = (uint32_t)(tiles * TILE * 4);   // bytes from one split's block of the tile to the next
    const uint32_t base = (uint32_t)(slot * TILE * 4);
    for (int s0 = 0; s0 < p.splits; s0 += 4) {
        f32x4 w[4][Cfg::FM * Cfg::FN * 4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < Cfg::FM * Cfg::FN * 4; ++i)   // splits past the last read zero (out of range)
                w[j][i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    rw, s0 + j < p.splits ? laneOff + (uint32_t)i * 1024u : kOOB, base + (uint32_t)(s0 + j) * stride,
                    kCpolAgent));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (s0 + j >= p.splits) break;
#pragma unroll
            for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < Cfg::FN; ++fn)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[fm][fn][4 * q + e] += w[j][(fm * Cfg::FN + fn) * 4 + q][e];
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// One output tile (bid: the tile's linear index, batch, split) of C =
// op(A) * op(B). BSUM (B stored [K, N]): the workgroups of the first row of
// tiles also add B's columns over K, row after row from 0, into p.colSum (the
// bias gradient of a Linear layer whose output gradient is B). GATE: each
// element of C is kept where p.gate (same shape, row stride p.ldg) is > 0 and
// set to 0 elsewhere (a ReLU's backward applied to the product).
template <class Cfg, bool TA, bool TB, int LA, int LB, bool BSUM = false, bool GATE = false>
__device__ __forceinline__ void gemmF32Tile(const GemmF32Params& p, float* smem, int bid, long long batch, int split) {
    static_assert(!BSUM || !TB, "column sums of a B stored [K, N]");
    constexpr bool A_KMAJOR = !TA;
    constexpr bool B_KMAJOR = TB;
    using SA = LdsShape<A_KMAJOR, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<B_KMAJOR, Cfg::BN, Cfg::BK>;
    constexpr int STAGE = SA::SIZE + SB::SIZE;   // floats per LDS buffer (A slice then B slice)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / Cfg::WAVES_N;
    const int wn = wave % Cfg::WAVES_N;

    int tm, tn;
    tile_coords(bid, p.tilesM * p.tilesN, p.tilesM, p.tilesN, 8, tm, tn);
    const int m0 = tm * Cfg::BM;
    const int n0 = tn * Cfg::BN;
    // This split's K range; the loaders treat kEnd as the end of K.
    const int kBeg = split * p.kChunk;
    const int kEnd = min(p.K, kBeg + p.kChunk);
    // BSUM: thread tid < BN owns column n0 + tid; the slice at k0 is in the B
    // region of an LDS stage as [BK][BN + 4].
    const bool doSum = BSUM && p.colSum && tm == 0 && tid < Cfg::BN && n0 + tid < p.N;
    float colAcc = 0.f;
    // The slice's BK values are read first (all inside the LDS stage) and then added in
    // row order; rows past the K range add -0.0f, which leaves every sum unchanged (a
    // guarded read per row made each read wait alone: the first tile row's mainloop ran
    // ~3x longer than the others').
    auto colSum = [&](const float* sB, int k0) {
        if constexpr (BSUM) {
            if (doSum) {
                float v[Cfg::BK];
#pragma unroll
                for (int k = 0; k < Cfg::BK; ++k) v[k] = sB[k * SB::LD + tid];
#pragma unroll
                for (int k = 0; k < Cfg::BK; ++k) colAcc += k0 + k < kEnd ? v[k] : -0.0f;
            }
        }
    };

    GemmLoader<A_KMAJOR, LA, Cfg::BM, Cfg::BK, Cfg::NT> la;
    la.init(p.A + batch * p.sA, p.lda, p.M, m0, tid);
    GemmLoader<B_KMAJOR, LB, Cfg::BN, Cfg::BK, Cfg::NT> lb;
    lb.init(p.B + batch * p.sB, p.ldb, p.N, n0, tid);

    f32x16 acc[Cfg::FM][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Small tiles (short main loops) load the epilogue's bias and gate values before the
    // first slice, so that their latency passes under the main loop instead of in front
    // of the C stores; the large tiles' registers are spoken for, and their main loops
    // are long, so they load the bias in the epilogue.
    constexpr bool PRE = Cfg::BM * Cfg::BN <= 128 * 128;
    float biasv[Cfg::FN];
    if constexpr (PRE) {
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = n0 + wn * Cfg::WN + fn * 32 + (lane & 31);
            biasv[fn] = (p.bias && col < p.N) ? p.bias[col] : 0.f;
        }
    }
    static_assert(!GATE || PRE, "gated tiles prefetch their gate");
    float gatev[GATE ? Cfg::FM : 1][GATE ? Cfg::FN : 1][GATE ? 16 : 1];
    if constexpr (GATE) {
#pragma unroll
        for (int fm = 0; fm < Cfg::FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < Cfg::FN; ++fn) {
                const int col = n0 + wn * Cfg::WN + fn * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    gatev[fm][fn][r] = (row < p.M && col < p.N) ? p.gate[(long long)row * p.ldg + col] : 0.f;
                }
            }
    }

    const int nk = (kEnd - kBeg + Cfg::BK - 1) / Cfg::BK;
    la.template load<false>(kBeg, kEnd, tid);
    lb.template load<false>(kBeg, kEnd, tid);
    la.store(smem, tid);
    lb.store(smem + SA::SIZE, tid);
    const int nFull = (kEnd - kBeg) / Cfg::BK;
    int t = 0;
    if constexpr (PRE) {
        // Two slices in flight: while slice t is multiplied from LDS, slice t+1 (loaded
        // one slice earlier) is stored to the other stage and slice t+2 is loaded into a
        // second register set (la2 / lb2), so a load has two slices of MFMA work to land
        // instead of one. The small tiles run one workgroup per CU with short main loops,
        // where a single slice did not cover the load latency.
        GemmLoader<A_KMAJOR, LA, Cfg::BM, Cfg::BK, Cfg::NT> la2;
        la2.init(p.A + batch * p.sA, p.lda, p.M, m0, tid);
        GemmLoader<B_KMAJOR, LB, Cfg::BN, Cfg::BK, Cfg::NT> lb2;
        lb2.init(p.B + batch * p.sB, p.ldb, p.N, n0, tid);
        if (nk > 1) {
            la.template load<false>(kBeg + Cfg::BK, kEnd, tid);
            lb.template load<false>(kBeg + Cfg::BK, kEnd, tid);
        }
        __syncthreads();
        // Slice t is in stage t & 1; on entry to a trip la / lb hold slice t+1. The
        // unchecked loop runs while the slices it fetches (t+2, t+3) are whole.
        for (; t + 3 < nFull; t += 2) {
            la2.template load<true>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
            lb2.template load<true>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
            __builtin_amdgcn_sched_barrier(0);
            colSum(smem + SA::SIZE, kBeg + t * Cfg::BK);
            mma_slice_split<Cfg, A_KMAJOR, B_KMAJOR>(smem, smem + SA::SIZE, acc, wm, wn, lane, [&] {
                la.store(smem + STAGE, tid);
                lb.store(smem + STAGE + SA::SIZE, tid);
            });
            __syncthreads();
            la.template load<true>(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
            lb.template load<true>(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
            __builtin_amdgcn_sched_barrier(0);
            colSum(smem + STAGE + SA::SIZE, kBeg + (t + 1) * Cfg::BK);
            mma_slice_split<Cfg, A_KMAJOR, B_KMAJOR>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane, [&] {
                la2.store(smem, tid);
                lb2.store(smem + SA::SIZE, tid);
            });
            __syncthreads();
        }
        for (; t < nk; t += 2) {
            if (t + 2 < nk) {
                la2.template load<false>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
                lb2.template load<false>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
            }
            colSum(smem + SA::SIZE, kBeg + t * Cfg::BK);
            mma_slice<Cfg, A_KMAJOR, B_KMAJOR>(smem, smem + SA::SIZE, acc, wm, wn, lane);
            if (t + 1 < nk) {
                la.store(smem + STAGE, tid);
                lb.store(smem + STAGE + SA::SIZE, tid);
            }
            __syncthreads();
            if (t + 1 < nk) {
                if (t + 3 < nk) {
                    la.template load<false>(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
                    lb.template load<false>(kBeg + (t + 3) * Cfg::BK, kEnd, tid);
                }
                colSum(smem + STAGE + SA::SIZE, kBeg + (t + 1) * Cfg::BK);
                mma_slice<Cfg, A_KMAJOR, B_KMAJOR>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane);
                if (t + 2 < nk) {
                    la2.store(smem, tid);
                    lb2.store(smem + SA::SIZE, tid);
                }
                __syncthreads();
            }
        }
    } else {
        __syncthreads();
        // Two slices per trip so both LDS stage addresses are compile-time
        // offsets. The main loop runs while both slices it fetches (t+1, t+2) lie
        // wholly inside the K range, so its loads test nothing; the last slices
        // run in the checked loop below (slice t is always in stage t & 1). The
        // schedule barriers keep each half in the order global loads, MFMAs, LDS
        // stores, block barrier.
        for (; t + 2 < nFull; t += 2) {
            la.template load<true>(kBeg + (t + 1) * Cfg::BK, kEnd, tid);
            lb.template load<true>(kBeg + (t + 1) * Cfg::BK, kEnd, tid);
            __builtin_amdgcn_sched_barrier(0);
            colSum(smem + SA::SIZE, kBeg + t * Cfg::BK);
            mma_slice_split<Cfg, A_KMAJOR, B_KMAJOR>(smem, smem + SA::SIZE, acc, wm, wn, lane, [&] {
                la.store(smem + STAGE, tid);
                lb.store(smem + STAGE + SA::SIZE, tid);
            });
            __syncthreads();
            la.template load<true>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
            lb.template load<true>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
            __builtin_amdgcn_sched_barrier(0);
            colSum(smem + STAGE + SA::SIZE, kBeg + (t + 1) * Cfg::BK);
            mma_slice_split<Cfg, A_KMAJOR, B_KMAJOR>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane, [&] {
                la.store(smem, tid);
                lb.store(smem + SA::SIZE, tid);
            });
            __syncthreads();
        }
        for (; t < nk; t += 2) {
            {
                const bool more = (t + 1) < nk;
                if (more) {
                    la.template load<false>(kBeg + (t + 1) * Cfg::BK, kEnd, tid);
                    lb.template load<false>(kBeg + (t + 1) * Cfg::BK, kEnd, tid);
                }
                colSum(smem + SA::SIZE, kBeg + t * Cfg::BK);
                mma_slice<Cfg, A_KMAJOR, B_KMAJOR>(smem, smem + SA::SIZE, acc, wm, wn, lane);
                if (more) {
                    la.store(smem + STAGE, tid);
                    lb.store(smem + STAGE + SA::SIZE, tid);
                }
                __syncthreads();
            }
            if (t + 1 < nk) {
                const bool more = (t + 2) < nk;
                if (more) {
                    la.template load<false>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
                    lb.template load<false>(kBeg + (t + 2) * Cfg::BK, kEnd, tid);
                }
                colSum(smem + STAGE + SA::SIZE, kBeg + (t + 1) * Cfg::BK);
                mma_slice<Cfg, A_KMAJOR, B_KMAJOR>(smem + STAGE, smem + STAGE + SA::SIZE, acc, wm, wn, lane);
                if (more) {
                    la.store(smem, tid);
                    lb.store(smem + SA::SIZE, tid);
                }
                __syncthreads();
            }
        }
    }

    const int li = lane & 31, h = lane >> 5;
    if constexpr (BSUM) {
        if (doSum) p.colSum[n0 + tid] = colAcc;
    }
    if (p.ws) {
        // Split-K: the last piece of the tile to arrive sums every piece's
        // partial product in split order and writes C.
        if (!splitArrive<Cfg>(p, acc, smem, lane, batch, split, bid)) return;
    }
    float* C = p.C + batch * p.sC;
    const long long ldc = p.ldc;
    const bool bias = p.bias != nullptr;
    const bool relu = p.act == 1;
#pragma unroll
    for (int fm = 0; fm < Cfg::FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < Cfg::FN; ++fn) {
            const int col = n0 + wn * Cfg::WN + fn * 32 + li;
            if (col >= p.N) continue;
            float b = 0.f;
            if constexpr (PRE) b = biasv[fn];
            else b = bias ? p.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * Cfg::WM + fm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                float v = acc[fm][fn][r];
                if (bias) v += b;
                if (relu) v = v > 0.f ? v : 0.f;
                if (row < p.M) {
                    if constexpr (GATE) v = gatev[fm][fn][r] > 0.f ? v : 0.f;
                    C[(long long)row * ldc + col] = v;
                }
            }
        }
    }
}

template <class Cfg, bool TA, bool TB, int LA, int LB>
__global__ __launch_bounds__(Cfg::NT) void gemm_f32_kernel(GemmF32Params p) {
    extern __shared__ float smem[];
    gemmF32Tile<Cfg, TA, TB, LA, LB>(p, smem, blockIdx.x, blockIdx.z, blockIdx.y);
}

template <class Cfg, bool TA, bool TB>
static size_t ldsBytesFor() {
    using SA = LdsShape<!TA, Cfg::BM, Cfg::BK>;
    using SB = LdsShape<TB, Cfg::BN, Cfg::BK>;
    return 2 * (SA::SIZE + SB::SIZE) * sizeof(float);
}

template <class Cfg, bool TA, bool TB, int LA, int LB>
static int launchOne(const GemmF32Params& prm, int batch, int splits) {
    auto kern = gemm_f32_kernel<Cfg, TA, TB, LA, LB>;
    const size_t lds = ldsBytesFor<Cfg, TA, TB>();
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    dim3 grid(prm.tilesM * prm.tilesN, splits, batch);
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), lds, stream(), prm);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

// In-tile byte offsets of the buffer-view loader stay below 2^30.
template <bool KMAJOR, int R, int BK>
static bool bufVecOk(bool vec, long long ld) {
    const long long maxOff = KMAJOR ? ((long long)(R - 1) * ld + BK) * 4 : ((long long)(BK - 1) * ld + R) * 4;
    return vec && maxOff < (long long)kMaxBufferBytes;
}

template <class Cfg, bool TA, bool TB>
static int launchVec(GemmF32Params prm, int batch, int splits, bool va, bool vb) {
    prm.tilesM = (prm.M + Cfg::BM - 1) / Cfg::BM;
    prm.tilesN = (prm.N + Cfg::BN - 1) / Cfg::BN;
    const bool ba = bufVecOk<!TA, Cfg::BM, Cfg::BK>(va, prm.lda);
    const bool bb = bufVecOk<TB, Cfg::BN, Cfg::BK>(vb, prm.ldb);
    if (ba && bb) return launchOne<Cfg, TA, TB, 2, 2>(prm, batch, splits);
    if (va && vb) return launchOne<Cfg, TA, TB, 1, 1>(prm, batch, splits);
    if (va) return launchOne<Cfg, TA, TB, 1, 0>(prm, batch, splits);
    if (vb) return launchOne<Cfg, TA, TB, 0, 1>(prm, batch, splits);
    return launchOne<Cfg, TA, TB, 0, 0>(prm, batch, splits);
}

// Slice depth of the large tile is a build-time constant (LDS: 2 x (256x(BK+4) + BKx260) floats).
// The large tile runs 8 waves of 64 x 128 (two per SIMD, 128 accumulators
// each): while one wave waits on its fragment reads, the block barrier or its
// operand loads, the other keeps the SIMD's matrix core busy. On MI355X it
// beats 4 waves of 128 x 128 (one per SIMD) by 5 % at 4096^3 and 8192^3 and
// by 15 % at 8192 x 256 x 2048.
#ifndef OMHIP_GEMM_BK
#define OMHIP_GEMM_BK 16
#endif
using CfgL = TileCfg<256, 256, OMHIP_GEMM_BK, 64, 128>;
using CfgM = TileCfg<128, 128, 16, 64, 64>;
using CfgS = TileCfg<64, 64, 16, 32, 32>;

// Tile and split-K choice (planGemmFor in gemm_f32.hpp) for this device.
static GemmPlan planGemm(int M, int N, int K, int batch, bool wsOk) {
    return planGemmFor(M, N, K, batch, wsOk, cuCount());
}

template <bool TA, bool TB>
static int launchCfg(const GemmF32Params& prm, int batch, int splits, int cfg, bool va, bool vb) {
    if (cfg == 0) return launchVec<CfgL, TA, TB>(prm, batch, splits, va, vb);
    if (cfg == 1) return launchVec<CfgM, TA, TB>(prm, batch, splits, va, vb);
    return launchVec<CfgS, TA, TB>(prm, batch, splits, va, vb);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launches the GEMM (split-K: partials to ws, summed in the same launch by
// each tile's last piece).
static int gemmF32Run(bool ta, bool tb, int batch, int M, int N, int K, const float* A, long long lda, long long sA,
                      const float* B, long long ldb, long long sB, float* C, long long ldc, long long sC,
                      GemmPlan plan, const float* bias, int act, float* fixedWs = nullptr, size_t fixedBytes = 0) {
    GemmF32Params prm{};
    prm.A = A; prm.B = B; prm.C = C;
    prm.bias = bias; prm.act = act;
    prm.M = M; prm.N = N; prm.K = K;
    prm.lda = lda; prm.ldb = ldb; prm.ldc = ldc;
    prm.sA = sA; prm.sB = sB; prm.sC = sC;
    const int splits = splitPieces(K, plan.splits, &prm.kChunk);
    prm.splits = splits;
    if (splits > 1) {
        const size_t tiles = (size_t)((M + 63) / 64) * ((N + 63) / 64) * batch;   // the split plans' 64 x 64 tiles
        const size_t need = (size_t)splits * tiles * 64 * 64 * sizeof(float);
        if (need >= kMaxBufferBytes) return fail("gemm: %zu bytes of split-K partial products exceed 2^30", need);
        if (fixedWs) {
            if (need > fixedBytes - kNoAllocCounterBytes || tiles * sizeof(unsigned) > kNoAllocCounterBytes)
                return fail("gemm: %d split-K partial products need %zu bytes of scratch; the fixed scratch holds %zu",
                            splits, need, fixedBytes - kNoAllocCounterBytes);
            prm.ws = fixedWs;
            prm.ctr = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(fixedWs) + fixedBytes - kNoAllocCounterBytes);
        } else {
            prm.ws = static_cast<float*>(workspace(need));
            if (!prm.ws) return -1;   // workspace() recorded the cause
            prm.ctr = static_cast<unsigned*>(workspace(tiles * sizeof(unsigned), kWsCounters));
            if (!prm.ctr) return -1;
        }
    }
    // A is K-contiguous unless transposed; the vector axis is K (A) or M (A^T).
    const bool va = aligned16(A) && lda % 4 == 0 && sA % 4 == 0 && (ta ? M % 4 == 0 : K % 4 == 0);
    const bool vb = aligned16(B) && ldb % 4 == 0 && sB % 4 == 0 && (tb ? K % 4 == 0 : N % 4 == 0);
    int rc;
    if (!ta && !tb) rc = launchCfg<false, false>(prm, batch, splits, plan.cfg, va, vb);
    else if (!ta && tb) rc = launchCfg<false, true>(prm, batch, splits, plan.cfg, va, vb);
    else if (ta && !tb) rc = launchCfg<true, false>(prm, batch, splits, plan.cfg, va, vb);
    else rc = launchCfg<true, true>(prm, batch, splits, plan.cfg, va, vb);
    return rc;
}

// Split-K partials are kept to at most this many bytes of workspace.
constexpr size_t kMaxSplitWorkspace = (size_t)256 << 20;

int gemmF32(bool ta, bool tb, int batch, int M, int N, int K,
            const float* A, long long lda, long long sA,
            const float* B, long long ldb, long long sB,
            float* C, long long ldc, long long sC, const float* bias, int act) {
    const bool wsOk = (size_t)64 * batch * M * N * sizeof(float) <= kMaxSplitWorkspace;
    const GemmPlan plan = planGemm(M, N, K, batch, wsOk);
    return gemmF32Run(ta, tb, batch, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC, plan, bias, act);
}

__global__ void zero_rows_kernel(float* C, int rows, int cols, long long ldc, long long sC) {
    const long long b = blockIdx.z;
    const long long n = (long long)rows * cols;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / cols, c = i % cols;
        C[b * sC + r * ldc + c] = 0.f;
    }
}

// Degenerate shapes: C is zeroed when its extent is valid (cpu_backend.ixx:246-251).
int zeroOutput(float* C, int batch, int M, int N, long long ldc, long long sC) {
    if (!C || M <= 0 || N <= 0 || batch <= 0) return 0;
    const long long n = (long long)M * N;
    const int blocks = (int)std::min<long long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_rows_kernel, dim3(blocks, 1, batch), dim3(256), 0, stream(), C, M, N, ldc, sC);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

int gemmF32Checked(const char* name, bool ta, bool tb, int batch, int M, int N, int K,
                   const float* A, long long lda, long long sA,
                   const float* B, long long ldb, long long sB,
                   float* C, long long ldc, long long sC) {
    clearError();
    if (batch <= 0 || M <= 0 || N <= 0) return 0;
    if (!C) return fail("%s: null output", name);
    if (!A || !B || K <= 0) return zeroOutput(C, batch, M, N, ldc, sC);
    if (batch > 65535) return fail("%s: batch %d exceeds 65535", name, batch);
    return gemmF32(ta, tb, batch, M, N, K, A, lda, sA, B, ldb, sB, C, ldc, sC);
}

// ---- Linear backward in one launch -------------------------------------------
// Workgroups [0, tilesW) compute dW = X^T G over 64 x 64 tiles, those of the
// first tile row also adding G's columns into db (BSUM); the rest compute
// dX = G W^T, kept where the gate is > 0 when one is given (GATE). K is not
// split, so every element is the same sum, in the same order, as the separate
// products compute whenever they do not split K either (e.g. every layer of the
// 784-256-128-10 MLP at batch 128).
template <int LK, bool GATE>
__global__ __launch_bounds__(CfgS::NT) void linear_backward_kernel(GemmF32Params pw, GemmF32Params pa, int tilesW) {
    extern __shared__ float smem[];
    if ((int)blockIdx.x < tilesW)
        gemmF32Tile<CfgS, true, false, LK, LK, true, false>(pw, smem, blockIdx.x, 0, 0);
    else
        gemmF32Tile<CfgS, false, true, LK, LK, false, GATE>(pa, smem, blockIdx.x - tilesW, 0, 0);
}

template <int LK, bool GATE>
static int launchLinearBackward(const GemmF32Params& pw, const GemmF32Params& pa, int tilesW, int tilesX) {
    auto kern = linear_backward_kernel<LK, GATE>;
    const size_t lds = std::max(ldsBytesFor<CfgS, true, false>(), ldsBytesFor<CfgS, false, true>());
    OMHIP_CHECK(OMHIP_SET_MAX_DYNAMIC_LDS_ONCE(kern, lds));
    hipLaunchKernelGGL(kern, dim3(tilesW + tilesX), dim3(CfgS::NT), lds, stream(), pw, pa, tilesW);
    OMHIP_CHECK_LAUNCH();
    return 0;
}

static int linearBackward(const float* X, const float* G, const float* W, const float* gate, float* dW, float* db,
                          float* dX, int B, int I, int O) {
    GemmF32Params pw{}, pa{};
    // dW [I, O] = X^T G: A = X stored [K = B, M = I], B = G stored [K = B, N = O]
    pw.A = X; pw.B = G; pw.C = dW; pw.M = I; pw.N = O; pw.K = B;
    pw.lda = I; pw.ldb = O; pw.ldc = O; pw.kChunk = B; pw.colSum = db;
    pw.tilesM = (I + CfgS::BM - 1) / CfgS::BM; pw.tilesN = (O + CfgS::BN - 1) / CfgS::BN;
    // dX [B, I] = G W^T: A = G stored [M = B, K = O], B = W stored [N = I, K = O]
    pa.A = G; pa.B = W; pa.C = dX; pa.M = B; pa.N = I; pa.K = O;
    pa.lda = O; pa.ldb = O; pa.ldc = I; pa.kChunk = O; pa.gate = gate; pa.ldg = I;
    pa.tilesM = (B + CfgS::BM - 1) / CfgS::BM; pa.tilesN = (I + CfgS::BN - 1) / CfgS::BN;
    const long long tilesW = (long long)pw.tilesM * pw.tilesN, tilesX = dX ? (long long)pa.tilesM * pa.tilesN : 0;
    if (tilesW + tilesX > 0x7fffffffLL) return fail("omHipLinearBackward: %lld tiles exceed the grid", tilesW + tilesX);
    // 16-byte operand loads: every operand's contiguous axis (I or O) and base in whole vectors
    bool vec = I % 4 == 0 && O % 4 == 0 && aligned16(X) && aligned16(G) && (!dX || aligned16(W));
    vec = vec && bufVecOk<false, CfgS::BM, CfgS::BK>(true, I) && bufVecOk<false, CfgS::BN, CfgS::BK>(true, O) &&
          bufVecOk<true, CfgS::BM, CfgS::BK>(true, O) && bufVecOk<true, CfgS::BN, CfgS::BK>(true, O);
    if (vec)
        return gate ? launchLinearBackward<2, true>(pw, pa, (int)tilesW, (int)tilesX)
                    : launchLinearBackward<2, false>(pw, pa, (int)tilesW, (int)tilesX);
    return gate ? launchLinearBackward<0, true>(pw, pa, (int)tilesW, (int)tilesX)
                : launchLinearBackward<0, false>(pw, pa, (int)tilesW, (int)tilesX);
}

// ---- fixed scratch of the no-allocation entry ---------------------------------
// Split-K partial sums of omHipGemmStridedBatchedNoAlloc live in this array,
// so that entry never allocates. A plan splits K only over 64 x 64 tiles and
// only while the grid holds fewer than 2 x CUs workgroups, and stops doubling
// the split count once it has reached them, so its partials cover fewer than
// 4 x CUs tiles of 64 x 64 floats: 16 MiB on a 256-CU device (the array holds
// twice that). Each device the library runs on holds its own copy until the
// process ends.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

static std::once_flag g_scratchOnce[kMaxDevices];
static float* g_scratchPtr[kMaxDevices];
static hipError_t g_scratchErr[kMaxDevices];
// Ordering of the calls that use a device's array: the stream of the last such
// call and an event recorded after its kernels. A call on another stream first
// makes its stream wait for that event (no host wait, no device memory).
static std::mutex g_scratchMutex[kMaxDevices];
static hipEvent_t g_scratchEvent[kMaxDevices];
static hipStream_t g_scratchLast[kMaxDevices];
static bool g_scratchRecorded[kMaxDevices];

// Device address of this device's `scratch` (the array's name is a host-side
// stand-in), looked up once per device with that device current.
static float* noAllocScratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)fail("no-allocation GEMM: hipGetDevice: %s", hipGetErrorString(hipGetLastError()));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        (void)fail("no-allocation GEMM: device %d beyond the %d supported", dev, kMaxDevices);
        return nullptr;
    }
    std::call_once(g_scratchOnce[dev], [dev] {
        void* ptr = nullptr;
        g_scratchErr[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratchPtr[dev] = g_scratchErr[dev] == hipSuccess ? static_cast<float*>(ptr) : nullptr;
    });
    if (!g_scratchPtr[dev]) {
        (void)fail("no-allocation GEMM: hipGetSymbolAddress(scratch): %s", hipGetErrorString(g_scratchErr[dev]));
        return nullptr;
    }
    return g_scratchPtr[dev];
}

// Runs `launch` (kernels that use the device's array) ordered after the last
// call that used it, whatever stream that call ran on. A stream that records a
// graph neither waits nor records: ordering a replay against other streams is
// the caller's.
template <class F>
static int withScratchOrder(F&& launch) {
    int dev = 0;
    OMHIP_CHECK(hipGetDevice(&dev));
    const hipStream_t s = stream();
    if (capturing(s)) return launch();
    std::lock_guard<std::mutex> lock(g_scratchMutex[dev]);
    if (!g_scratchEvent[dev]) OMHIP_CHECK(hipEventCreateWithFlags(&g_scratchEvent[dev], hipEventDisableTiming));
    if (g_scratchRecorded[dev] && g_scratchLast[dev] != s) OMHIP_CHECK(hipStreamWaitEvent(s, g_scratchEvent[dev], 0));
    const int rc = launch();
    if (rc) return rc;
    OMHIP_CHECK(hipEventRecord(g_scratchEvent[dev], s));
    g_scratchLast[dev] = s;
    g_scratchRecorded[dev] = true;
    return 0;
}

}  // namespace omhip

using namespace omhip;

extern "C" {

int omHipMatmul(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmul", false, false, 1, nM, nN, nK, pA, nK, 0, pB, nN, 0, pC, nN, 0);
}

int omHipMatmulTransB(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmulTransB", false, true, 1, nM, nN, nK, pA, nK, 0, pB, nK, 0, pC, nN, 0);
}

int omHipMatmulTransA(const float* pA, const float* pB, float* pC, int nM, int nK, int nN) {
    return gemmF32Checked("omHipMatmulTransA", true, false, 1, nM, nN, nK, pA, nM, 0, pB, nN, 0, pC, nN, 0);
}

int omHipLinearBiasAct(const float* pA, const float* pW, const float* pBias, float* pOut, int nM, int nK, int nN,
                       int nAct) {
    clearError();
    if (nAct != 0 && nAct != 1) return fail("omHipLinearBiasAct: unknown activation %d", nAct);
    if (nM <= 0 || nN <= 0) return 0;
    if (!pOut) return fail("omHipLinearBiasAct: null output");
    if (!pA || !pW || nK <= 0) {
        // a product with no terms: act(0 + bias), as the unfused chain computes it
        if (zeroOutput(pOut, 1, nM, nN, nN, 0)) return -1;
        if (pBias && omHipAddBias(pOut, pBias, pOut, nM, nN, 1)) return -1;
        if (nAct == 1) {
            // omHipReLU takes an int count: walk M*N (up to 2^62 elements) in 2^30 pieces
            const long long total = (long long)nM * nN;
            for (long long off = 0; off < total; off += 1LL << 30)
                if (omHipReLU(pOut + off, pOut + off, (int)std::min(total - off, 1LL << 30))) return -1;
        }
        return 0;
    }
    return gemmF32(false, false, 1, nM, nN, nK, pA, nK, 0, pW, nN, 0, pOut, nN, 0, pBias, nAct);
}

int omHipLinearBackward(const float* pInput, const float* pGradOut, const float* pWeight, const float* pGate,
                        float* pGradWeight, float* pGradBias, float* pGradInput, int nBatch, int nIn, int nOut) {
    clearError();
    if (nBatch < 0 || nIn < 0 || nOut < 0) return fail("omHipLinearBackward: negative size");
    if (!pGradWeight && nIn > 0 && nOut > 0) return fail("omHipLinearBackward: null weight gradient");
    if (pGradInput && nBatch > 0 && nIn > 0 && nOut > 0 && !pWeight) return fail("omHipLinearBackward: null weight");
    if (nBatch == 0 || nIn == 0 || nOut == 0 || !pInput || !pGradOut) {
        // some product has no terms or no elements: the separate entries, whose degenerate cases match the chain's
        if (omHipMatmulTransA(pInput, pGradOut, pGradWeight, nIn, nBatch, nOut)) return -1;
        if (pGradBias && omHipAddBiasBackward(pGradOut, pGradBias, nBatch, nOut, 1)) return -1;
        if (pGradInput) {
            if (omHipMatmulTransB(pGradOut, pWeight, pGradInput, nBatch, nOut, nIn)) return -1;
            if (pGate) {
                const long long total = (long long)nBatch * nIn;
                for (long long off = 0; off < total; off += 1LL << 30)
                    if (omHipReLUBackward(pGate + off, pGradInput + off, pGradInput + off,
                                          (int)std::min(total - off, 1LL << 30)))
                        return -1;
            }
        }
        return 0;
    }
    return linearBackward(pInput, pGradOut, pWeight, pGate, pGradWeight, pGradBias, pGradInput, nBatch, nIn, nOut);
}

int omHipBatchedMatmul(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
    return gemmF32Checked("omHipBatchedMatmul", false, false, nBatch, nM, nN, nK,
                          pA, nK, (long long)nM * nK, pB, nN, (long long)nK * nN, pC, nN, (long long)nM * nN);
}

int omHipBatchedMatmulTransB(const float* pA, const float* pB, float* pC, int nBatch, int nM, int nK, int nN) {
    return gemmF32Checked("omHipBatchedMatmulTransB", false, true, nBatch, nM, nN, nK,
                          pA, nK, (long long)nM * nK, pB, nK, (long long)nN * nK, pC, nN, (long long)nM * nN);
}

int omHipGemmStridedBatched(int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                            const float* pA, long long nLda, long long nStrideA,
                            const float* pB, long long nLdb, long long nStrideB,
                            float* pC, long long nLdc, long long nStrideC) {
    clearError();
    if (nBatch > 0 && nM > 0 && nN > 0 && nK > 0) {
        if (nLda < (bTransA ? nM : nK) || nLdb < (bTransB ? nK : nN) || nLdc < nN)
            return fail("omHipGemmStridedBatched: leading dimension smaller than the row length");
        if (nStrideA < 0 || nStrideB < 0 || nStrideC < 0)
            return fail("omHipGemmStridedBatched: negative batch stride");
    }
    return gemmF32Checked("omHipGemmStridedBatched", bTransA != 0, bTransB != 0, nBatch, nM, nN, nK,
                          pA, nLda, nStrideA, pB, nLdb, nStrideB, pC, nLdc, nStrideC);
}

int omHipGemmStridedBatchedNoAlloc(int bTransA, int bTransB, int nBatch, int nM, int nN, int nK,
                                   const float* pA, long long nLda, long long nStrideA,
                                   const float* pB, long long nLdb, long long nStrideB,
                                   float* pC, long long nLdc, long long nStrideC) {
    clearError();
    const char* name = "omHipGemmStridedBatchedNoAlloc";
    if (nBatch <= 0 || nM <= 0 || nN <= 0) return 0;
    if (!pC) return fail("%s: null output", name);
    if (nK > 0 && pA && pB) {
        if (nLda < (bTransA ? nM : nK) || nLdb < (bTransB ? nK : nN) || nLdc < nN)
            return fail("%s: leading dimension smaller than the row length", name);
        if (nStrideA < 0 || nStrideB < 0 || nStrideC < 0) return fail("%s: negative batch stride", name);
    }
    if (!pA || !pB || nK <= 0) return zeroOutput(pC, nBatch, nM, nN, nLdc, nStrideC);
    if (nBatch > 65535) return fail("%s: batch %d exceeds 65535", name, nBatch);
    float* ws = noAllocScratch();
    if (!ws) return -1;
    // the same plan as omHipGemmStridedBatched, so the results are the same bits
    const bool wsOk = (size_t)64 * nBatch * nM * nN * sizeof(float) <= kMaxSplitWorkspace;
    const GemmPlan plan = planGemm(nM, nN, nK, nBatch, wsOk);
    auto run = [&] {
        return gemmF32Run(bTransA != 0, bTransB != 0, nBatch, nM, nN, nK, pA, nLda, nStrideA, pB, nLdb, nStrideB, pC,
                          nLdc, nStrideC, plan, nullptr, 0, ws, kNoAllocScratchBytes);
    };
    if (plan.splits <= 1) return run();   // the array is not touched
    return withScratchOrder(run);
}

}  // extern "C"
