// Tile streaming helpers shared by the MFMA scan kernels: HBM -> LDS copies that bypass the
// registers (global_load_lds_dwordx4) and the explicit vmcnt waits that order them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace zcgvs_hip {

// LDS byte address of a __shared__ location.
__device__ __forceinline__ std::uint32_t ldsAddress(const void* p) {
    return static_cast<std::uint32_t>(
        reinterpret_cast<std::uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// One global_load_lds_dwordx4: every active lane copies 16 bytes from `src` to LDS at
// lds_base + 16 * lane. Issued as inline assembly so that the compiler, which cannot tell the
// ring slots apart, does not make every later LDS read wait for all copies in flight; the
// kernel orders the copies itself (vmcnt waits + barriers). M0 carries the LDS base (bound as
// an operand, so the compiler writes it); the s_nop is the wait state an M0 write needs before
// an LDS DMA instruction. The corpus is streamed once, so the copies carry the non-temporal hint
// (measured: the same or up to 4% faster scans).
__device__ __forceinline__ void copyToLds(const void* src, std::uint32_t lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(src), "{m0}"(lds_base)
                 : "memory");
}

// The same copy from a wave-uniform base address (SGPR pair) plus a per-lane 32-bit byte
// offset, so no 64-bit address arithmetic runs per lane.
__device__ __forceinline__ void copyToLds(const void* uniform_base, std::uint32_t lane_offset,
                                          std::uint32_t lds_base) {
    // readfirstlane returns int: each half goes through uint32_t so the low word is not
    // sign-extended into the high one.
    const auto address = reinterpret_cast<std::uintptr_t>(uniform_base);
    const auto hi = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(address >> 32)));
    const auto lo = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<std::uint32_t>(address)));
    const std::uint64_t sbase = (static_cast<std::uint64_t>(hi) << 32) | lo;
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(lane_offset), "s"(sbase), "{m0}"(lds_base)
                 : "memory");
}

// One global_load_lds_dword: every active lane copies 4 bytes from `src` to LDS at
// lds_base + 4 * lane (same ordering rules as copyToLds).
__device__ __forceinline__ void copyDwordToLds(const void* src, std::uint32_t lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(src), "{m0}"(lds_base)
                 : "memory");
}

// s_waitcnt that waits until at most n vector-memory operations of this wavefront are pending
// (expcnt and lgkmcnt fields at their "no wait" maxima).
__device__ constexpr int vmcntOnly(int n) {
    return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14);
}

// Waits until at most `later * kPerTile` copies are pending (later <= kMaxLater, wave-uniform;
// kMaxLater * kPerTile fits the 6-bit vmcnt).
template <int kPerTile, int kMaxLater>
__device__ __forceinline__ void waitTiles(int later) {
    static_assert(kMaxLater * kPerTile <= 63, "vmcnt counts at most 63 operations");
    if constexpr (kMaxLater >= 1) {
        if (later >= kMaxLater) {
            __builtin_amdgcn_s_waitcnt(vmcntOnly(kMaxLater * kPerTile));
            return;
        }
        waitTiles<kPerTile, kMaxLater - 1>(later);
    } else {
        __builtin_amdgcn_s_waitcnt(vmcntOnly(0));
    }
}

// SIMD of the calling wavefront (HW_ID register, SIMD_ID field: bits 5:4).
__device__ __forceinline__ int simdId() {
    constexpr int kHwId = 4;
    return __builtin_amdgcn_s_getreg(((2 - 1) << 11) | (4 << 6) | kHwId) & 3;
}

}  // namespace zcgvs_hip
