// gmem.h — explicit global / LDS memory access for the gfx950 kernels.
//
// A pointer the compiler cannot place in an address space (one read from a
// table in memory, or passed through a struct) is accessed with FLAT
// instructions.  On gfx950 a flat access counts against both the vector
// memory counter and the LDS counter, so a wave that waits for an LDS read
// also waits for every flat load it has in flight — which turns a pipeline of
// weight loads into a serial one.  The kernels therefore load weights and
// activations through these helpers, which cast to the global address space
// (address space 1) and emit global_load / global_store.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

template <typename T>
using gptr = const __attribute__((address_space(1))) T *;
template <typename T>
using gptr_mut = __attribute__((address_space(1))) T *;
template <typename T>
using lptr = __attribute__((address_space(3))) T *;

template <typename T>
__device__ inline T gload(const T *p) {
    return *(gptr<T>)p;
}
template <typename T>
__device__ inline void gstore(T *p, T v) {
    *(gptr_mut<T>)p = v;
}
// 16 bytes from a global address that is only 4-byte aligned.
typedef uint32_t u32x4_dw __attribute__((ext_vector_type(4), aligned(4)));
__device__ inline u32x4_dw gload_x4(const uint32_t *p) { return *(const __attribute__((address_space(1))) u32x4_dw *)p; }

// LDS pointer from a generic one that points into LDS.
template <typename T>
__device__ inline lptr<T> to_lds(T *p) {
    return (lptr<T>)p;
}

}  // namespace moe
