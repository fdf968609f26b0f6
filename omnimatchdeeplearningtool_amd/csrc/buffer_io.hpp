// buffer_io.hpp — raw buffer loads with hardware range checking (gfx950).
//
// A buffer resource covers [base, base + bytes). A load whose per-lane offset
// (voffset) is at or past `bytes` returns 0 without touching memory; the
// kernels here use that as a free zero-fill for padding taps, ragged tile
// edges and rows past the end. Only the voffset operand is used to push a
// lane out of range: the scalar soffset always holds an in-range offset.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace omhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Offsets at or above this byte count are out of range for every buffer used
// with these helpers (buffer views are limited to 2^30 bytes), and two such
// terms plus an in-range offset never wrap 32 bits.
constexpr uint32_t kOOB = 0x40000000u;
constexpr uint32_t kMaxBufferBytes = 0x40000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bufferRsrc(const void* base, uint32_t bytes) {
    // raw buffer, stride 0, range-checked against `bytes` (data format 32-bit)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float bufLoad1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ f32x4 bufLoad4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// Vector-memory store; a lane whose voffset is out of range writes nothing.
__device__ __forceinline__ void bufStore1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, 0);
}

// Cache policy nt: a streaming store (the line is not kept in L2 for reuse),
// for outputs written once that the next kernel reads: they drain to memory
// while the kernel still runs instead of in the L2 write-back at its end.
constexpr int kCpolStream = 2;
__device__ __forceinline__ void bufStore1Stream(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, kCpolStream);
}

// Cache policy sc1: an access coherent at agent scope (the monotonic
// agent-scope atomic load / store of the gfx94x / gfx950 memory model), so
// data exchanged between workgroups on different XCDs (each with its own L2)
// needs no whole-cache writeback or invalidation.
constexpr int kCpolAgent = 16;
__device__ __forceinline__ void bufStore1Agent(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, kCpolAgent);
}
__device__ __forceinline__ float bufLoad1Agent(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kCpolAgent));
}

}  // namespace omhip
