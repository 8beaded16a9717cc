// lds_dma.h — LDS DMA, exact memory-counter waits and the weight-row layout
// in LDS shared by the matrix-core expert kernels (expert_mfma.hip,
// expert_stream.hip).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_internal.h"

namespace moe {
namespace lds {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Bytes of one 32-value block, and dwords per weight row per K step of 64
// values (two blocks; a row's step always starts 4-byte aligned since
// K % 64 == 0).
template <int DT>
struct Fmt;
template <>
struct Fmt<MOE_DT_Q4_0> {
    static constexpr int bytes = 18, rd = 9;
};
template <>
struct Fmt<MOE_DT_Q5_0> {
    static constexpr int bytes = 22, rd = 11;
};
template <>
struct Fmt<MOE_DT_Q8_0> {
    static constexpr int bytes = 34, rd = 17;
};

// Weight DMA.  A row's step (rd dwords) is split into nx4 16-byte lanes
// (dwords 0 .. 4 nx4 - 1) and nd dword lanes (the rest).  One 32-row region
// is laid out as
//   X part  lane q = 32 x + r  (x < nx4) at 16 q: dwords 4x .. 4x+3 of row r
//   D part  lane q = 32 e + r  (e < nd)  at X + 4 q: dword 4 nx4 + e of row r
// and filled by nx4 / 2 dwordx4 DMAs plus ceil(nd / 2) dword DMAs (lanes
// past nd load row 0 into the padding at the region's end).  Dword d of row
// r of the region therefore sits at loc(d, r) below.
template <int DT>
struct BLay {
    static constexpr int rd = Fmt<DT>::rd;
    static constexpr int nx4 = rd / 4;             // 2, 2, 4 (even)
    static constexpr int nd = rd - 4 * nx4;        // 1, 3, 1
    static constexpr int ix = nx4 / 2;             // dwordx4 DMAs per region
    static constexpr int id = (nd + 1) / 2;        // dword DMAs per region
    static constexpr int inst = ix + id;
    static constexpr int xbytes = 512 * nx4;
    static constexpr int region = xbytes + 256 * id;  // bytes
    static constexpr int stage = 8 * region;
    static_assert(nx4 % 2 == 0, "whole dwordx4 DMAs per region");
    __host__ __device__ static constexpr uint32_t loc(int d, int r) {
        return d < 4 * nx4 ? (uint32_t)(512 * (d >> 2) + 16 * r + 4 * (d & 3))
                           : (uint32_t)(xbytes + 128 * (d - 4 * nx4) + 4 * r);
    }
};

// ---- LDS DMA and exact waits ------------------------------------------------
// global_load_lds writes lane l's 16 (or 4) bytes to LDS address m0 + 16 l
// (4 l); lanes with EXEC clear write nothing.  Addresses are an SGPR base
// plus a 32-bit VGPR offset; the base and the LDS address are wave-uniform
// (readfirstlane states that to the compiler, which may not prove it).
//
// The compiler cannot see that the assembly below is a vector memory load
// that reads an SGPR base and M0, so it would not insert the wait states the
// hardware needs between a VALU write of an SGPR (v_readfirstlane) and a
// vector memory instruction reading it (5), or between an M0 write and an
// LDS DMA (1).  The assembly therefore copies the base with s_mov_b64 (a
// scalar read, which the hardware interlocks) into SGPRs that nothing but
// scalar instructions ever wrote, and pads one wait state after the copy.
__device__ inline const void *uniform_ptr(const void *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const void *>(lo | (hi << 32));
}
__device__ inline void dma16(const void *base, uint32_t off, uint32_t lds) {
    uint64_t sb;
    asm volatile(
        "s_mov_b64 %0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %0"
        : "=&s"(sb)
        : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane((int)lds))
        : "memory");
}
__device__ inline void dma4(const void *base, uint32_t off, uint32_t lds) {
    uint64_t sb;
    asm volatile(
        "s_mov_b64 %0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, %0"
        : "=&s"(sb)
        : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane((int)lds))
        : "memory");
}
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait for all but the newest N of this wave's loads and for its LDS reads,
// then meet the other waves.
template <int N>
__device__ inline void wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
typedef const __attribute__((address_space(3))) uint8_t *lds_p;
typedef uint32_t u32x4l __attribute__((ext_vector_type(4)));
__device__ inline uint32_t lds_u32(lds_p p) { return *(const __attribute__((address_space(3))) uint32_t *)p; }
__device__ inline half8 lds_h8(lds_p p) { return *(const __attribute__((address_space(3))) half8 *)p; }

__device__ inline uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t s) { return __builtin_amdgcn_alignbyte(hi, lo, s); }
__device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }
__device__ inline uint32_t spread4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

}  // namespace lds
}  // namespace moe
