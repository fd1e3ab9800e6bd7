// lq_dma.h -- LDS-DMA building blocks shared by the int8 GEMM and the implicit-GEMM conv:
// buffer descriptors, the LDS-DMA form of buffer_load_dwordx4, explicit vmcnt waits, a
// barrier without the memory-model fence, and the stage-row swizzle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lq {

typedef int v4i __attribute__((ext_vector_type(4)));

// LDS slot of logical 16-byte K chunk c in stage row r (tile-local) is c ^ dma_swz(r).  Bits
// 0-2 of the row spread the 16 lanes of a plain fragment (rows r..r+15) over distinct 16-byte
// bank groups; bit 4 of the row separates the rows 16 apart that a permuted fragment reads
// (lane row rho at tile row (rho / 4) * 16 + 4 i + rho % 4, the layout that leaves each lane
// 16 consecutive outputs).
__device__ __forceinline__ int dma_swz(int r) { return (r & 7) ^ ((r >> 2) & 4); }

// s_waitcnt vmcnt(N) only (lgkmcnt and expcnt fields at their no-wait maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without the memory-model fence __syncthreads() adds (that fence waits
// for every outstanding copy).  It first waits for this wave's own LDS reads (lgkmcnt(0)):
// after the barrier another wave may copy into the buffer those reads came from.  The
// copies themselves are covered by wait_vmcnt.  The empty asm keeps the compiler from
// moving memory accesses across the barrier.
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt fields at maximum
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Raw buffer descriptor (base, num_records = bytes, stride 0).
__device__ __forceinline__ v4i buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)b),
               __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)),
               __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// 16 bytes per lane from rsrc + voff + soff into LDS at lds_addr + 16 * lane.  The LDS
// destination travels in M0 as an input operand ("{m0}"): the compiler writes M0 itself and
// knows the instruction reads it, so M0 is never changed behind its back.
__device__ __forceinline__ void lds_dma16(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
                 : "memory");
}

}  // namespace lq
