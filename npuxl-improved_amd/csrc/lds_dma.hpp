// lds_dma.hpp - direct HBM/L2 -> LDS copies and the waits that order them,
// shared by the matrix-core kernels (int8 GEMM, f32 GEMM, attention prefill).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace vnpu {
namespace lds {

// s_waitcnt immediate (gfx9 encoding): vmcnt in bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8.  Issued through the builtin so the compiler's own wait
// insertion knows which counters are already drained.
constexpr int waitcnt_imm(int vm, int exp, int lgkm)
{
    return (vm & 0xF) | ((vm >> 4) << 14) | (exp << 4) | (lgkm << 8);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(N, 7, 15));
}

// Workgroup barrier that does not drain the DMA queue: only this wave's LDS
// reads must be complete (the buffer they read may be refilled right after),
// outstanding global->LDS loads keep flying.  The asm keeps memory accesses
// from being moved across the barrier.
__device__ __forceinline__ void block_barrier()
{
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 7, 0));
    asm volatile("s_barrier" ::: "memory");
}

// 16-byte-per-lane global->LDS copy (lane l writes lds_dst + 16 l).  Written
// as asm on purpose: the compiler books the builtin form as an LDS-counter
// event that may complete out of order, and then waits lgkmcnt(0) before
// every MFMA that uses earlier ds_reads (or vmcnt(0) before the first ds_read
// after a copy), which serialises the copy with the compute.  Every consumer
// of copied data waits for it explicitly (vmcnt + barrier); the compiler's
// own vmcnt waits for its own loads only get more conservative by not seeing
// these.
__device__ __forceinline__ void dma16(const void *src, int8_t *lds_dst)
{
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(lds_dst)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

// The same copy of data read once (nontemporal: no cache line is kept for
// reuse), for streams such as attention's K and V.
__device__ __forceinline__ void dma16_nt(const void *src, int8_t *lds_dst)
{
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(lds_dst)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

// The same copy with a wave-uniform 64-bit base (SGPRs) and a 32-bit
// per-lane byte offset: lane l reads base + voff and writes lds_dst + 16 l.
__device__ __forceinline__ void dma16_s(const int8_t *base, uint32_t voff, int8_t *lds_dst)
{
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int8_t *)(lds_dst)));
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

}  // namespace lds
}  // namespace vnpu
