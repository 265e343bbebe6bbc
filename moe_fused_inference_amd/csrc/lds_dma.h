// lds_dma.h -- global -> LDS copies for the tiled MFMA kernels (gfx950).
//
// The copies are buffer loads with an LDS destination, written as inline asm
// on purpose: the compiler's own wait insertion treats any pending LDS copy as
// aliasing every later LDS read and would wait for all of them (vmcnt(0))
// before the first operand read of a step, collapsing a stage ring.  Callers
// wait for them explicitly (s_waitcnt vmcnt(n) before a step's barrier).
// The base and extent of the copied tensor sit in a scalar buffer descriptor
// (reads past its end return zero), a copy's row block and K offset in the
// scalar soffset, and the lane's offset in one VGPR.  The LDS address goes in
// M0, which is saved and restored around the copy: lane i of a dwordx4 copy
// writes LDS bytes [M0 + 16i, M0 + 16i + 16), of a dword copy [M0 + 4i, +4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Descriptor of `bytes` bytes at `base` (clamped to [0, 2^32)), in SGPRs.
__device__ __forceinline__ v4u buf_rsrc(const void* base, int64_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    const uint32_t n = bytes > 0 ? (bytes < 0xFFFFFFFFll ? (uint32_t)bytes : 0xFFFFFFFFu) : 0u;
    v4u r;
    r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xFFFFu);
    r.z = __builtin_amdgcn_readfirstlane(n);
    r.w = 0x00020000u;
    return r;
}

__device__ __forceinline__ void dma16(uint32_t voff, v4u rs, uint32_t soff, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(__builtin_amdgcn_readfirstlane(lds)), "s"(rs),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory");
}

__device__ __forceinline__ void dma4(uint32_t voff, v4u rs, uint32_t soff, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %1, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(__builtin_amdgcn_readfirstlane(lds)), "s"(rs),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory");
}

// XOR swizzle of 128-byte LDS rows (8 chunks of 16 bytes): the slot of logical
// chunk c of row r is c ^ swz_key128(r).  A ds_read_b128 phase covers 16
// consecutive rows (16-aligned) at one logical chunk, 256 bytes over the 64
// banks; rows r and r+1 share a 256-byte bank line, and the 8 rows of either
// parity in the phase get distinct keys.  The key depends on r mod 16 only.
__device__ __forceinline__ int swz_key128(int r) { return (r & 7) ^ ((r >> 3) & 1); }

}  // namespace mx
