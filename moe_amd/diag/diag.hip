// diag.hip — measurement probes for the bench (libmoe_diag.so), kept out of
// the layer library: the HBM read ceiling of a plain streaming kernel, the
// cost of a grid-wide barrier, and the issue rate of the MFMA kernels'
// instruction mix.  bench.py loads this library for --hbm-ceiling,
// --grid-barrier and --mfma-valu; nothing in libmoe_hip.so calls it.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/moe_hip.h"  // status codes only
#include "moe_diag.h"

namespace {

thread_local char g_err[512];
int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
int launch_rc(const char *what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_OK : fail(MOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}
template <typename T>
__device__ inline T gload(const T *p) {
    return *(const __attribute__((address_space(1))) T *)p;
}

// The HBM read ceiling.  Grid-stride 16-byte loads, eight in
// flight per thread, folded into one word per block so nothing is elided;
// NT = true marks the loads nontemporal (streamed past the caches).
typedef uint32_t sr_u32x4 __attribute__((ext_vector_type(4)));
template <bool NT>
__global__ __launch_bounds__(256) void stream_read_kernel(const sr_u32x4 *__restrict__ src, size_t n16,
                                                          uint32_t *__restrict__ out) {
    constexpr int U = 8;
    const size_t stride = (size_t)gridDim.x * 256;
    uint32_t acc = 0;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        sr_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const sr_u32x4 *p = src + i + u * stride;
            if constexpr (NT)
                v[u] = __builtin_nontemporal_load((const __attribute__((address_space(1))) sr_u32x4 *)p);
            else
                v[u] = gload(p);
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const sr_u32x4 v = gload(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// The cost of a grid-wide barrier.  `barriers` barriers of
// every block of a cooperative launch: a release fence, one device atomic
// per block on a shared counter, the last arrival resets it and advances a
// generation word that the others poll.  The poll is bounded (2^20 reads;
// state[2] = 1 records that a bound was hit), so no wave can spin forever.
struct GridBarrier {
    unsigned count, gen, err, pad;
};

__global__ __launch_bounds__(512) void grid_barrier_kernel(GridBarrier *b, int barriers) {
    __shared__ unsigned s_gen;
    if (threadIdx.x == 0) s_gen = __hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    unsigned g = s_gen;
    for (int i = 0; i < barriers; i++) {
        __syncthreads();
        if (threadIdx.x == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            const unsigned old = __hip_atomic_fetch_add(&b->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == gridDim.x - 1) {
                __hip_atomic_store(&b->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&b->gen, g + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                for (unsigned n = 0; __hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g; n++)
                    if (n > (1u << 20)) {
                        __hip_atomic_store(&b->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        g++;
        __syncthreads();
    }
}

// Issue-rate probe for the two-pass MFMA kernels' mix: each wave runs
// `iters` iterations of MF V_MFMA_F32_32X32X16_F16 (two independent
// accumulator chains) and VA f32 fmas on 32 registers of their own;
// MIX = 0: the fmas after the iteration's MFMAs (a scheduling barrier
// between), 1: VA / MF fmas after each MFMA.  One result per thread keeps
// the work live.
typedef _Float16 probe_half8 __attribute__((ext_vector_type(8)));
typedef float probe_floatx16 __attribute__((ext_vector_type(16)));
template <int MF, int VA, bool MIX>
__global__ __launch_bounds__(512) void mfma_valu_probe_kernel(float *out, int iters, float s) {
    const int lane = threadIdx.x & 63;
    probe_half8 a, b;
    for (int i = 0; i < 8; i++) a[i] = (_Float16)(lane * 0.001f + i), b[i] = (_Float16)(i * 0.5f);
    probe_floatx16 c0 = {}, c1 = {};
    float v[32];
    for (int i = 0; i < 32; i++) v[i] = (float)(lane + i);
    constexpr int per = MF > 0 ? VA / MF : 0;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int m = 0; m < MF; m++) {
            if (m & 1)
                c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
            else
                c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            if constexpr (MIX) {
#pragma unroll
                for (int k = 0; k < per; k++) v[(m * per + k) & 31] = fmaf(v[(m * per + k) & 31], s, 1.0f);
            }
        }
        if constexpr (!MIX || MF == 0) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < VA; k++) v[k & 31] = fmaf(v[k & 31], s, 1.0f);
        }
    }
    float r = 0.0f;
    for (int i = 0; i < 16; i++) r += c0[i] + c1[i];
    for (int i = 0; i < 32; i++) r += v[i];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = r;
}

}  // namespace

extern "C" {

const char *moe_diag_last_error(void) { return g_err; }

int moe_debug_stream_read(const void *src, uint64_t bytes, uint32_t *out, int32_t blocks, int32_t nontemporal,
                          void *stream) {
    if (!src || !out || blocks <= 0 || bytes % 16 || ((uintptr_t)src & 15))
        return fail(MOE_EINVAL, "moe_debug_stream_read: bad argument");
    if (bytes == 0) return MOE_OK;
    const sr_u32x4 *s4 = static_cast<const sr_u32x4 *>(src);
    if (nontemporal)
        hipLaunchKernelGGL(stream_read_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, s4,
                           (size_t)(bytes / 16), out);
    else
        hipLaunchKernelGGL(stream_read_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, s4,
                           (size_t)(bytes / 16), out);
    return launch_rc("stream-read kernel");
}

int moe_debug_mfma_valu(int32_t mfmas, int32_t valus, int32_t interleave, int32_t waves_per_simd, int32_t blocks,
                        int32_t iters, float *out, void *stream) {
    if (!out || blocks <= 0 || iters < 0 || (waves_per_simd != 1 && waves_per_simd != 2))
        return fail(MOE_EINVAL, "moe_debug_mfma_valu: bad argument");
    const dim3 grid(blocks), block(256 * waves_per_simd);
    hipStream_t s = (hipStream_t)stream;
    const int key = mfmas * 10000 + valus * 10 + (interleave ? 1 : 0);
    switch (key) {
    case 80000: hipLaunchKernelGGL((mfma_valu_probe_kernel<8, 0, false>), grid, block, 0, s, out, iters, 0.999f); break;
    case 560: hipLaunchKernelGGL((mfma_valu_probe_kernel<0, 56, false>), grid, block, 0, s, out, iters, 0.999f); break;
    case 80560: hipLaunchKernelGGL((mfma_valu_probe_kernel<8, 56, false>), grid, block, 0, s, out, iters, 0.999f); break;
    case 80561: hipLaunchKernelGGL((mfma_valu_probe_kernel<8, 56, true>), grid, block, 0, s, out, iters, 0.999f); break;
    case 80321: hipLaunchKernelGGL((mfma_valu_probe_kernel<8, 32, true>), grid, block, 0, s, out, iters, 0.999f); break;
    default:
        return fail(MOE_EINVAL,
                    "moe_debug_mfma_valu: (mfmas, valus, interleave) must be (8,0,0), (0,56,0), (8,56,0), (8,56,1) "
                    "or (8,32,1)");
    }
    return launch_rc("MFMA/VALU probe kernel");
}

int moe_debug_grid_barrier(int32_t blocks, int32_t barriers, uint32_t *state, void *stream) {
    if (blocks <= 0 || barriers < 0 || !state) return fail(MOE_EINVAL, "moe_debug_grid_barrier: bad argument");
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)grid_barrier_kernel, 512, 0) !=
            hipSuccess)
        return fail(MOE_EHIP, "moe_debug_grid_barrier: device query failed");
    if (blocks > cus * per_cu)
        return fail(MOE_EINVAL, "moe_debug_grid_barrier: %d blocks cannot all be resident (%d per CU, %d CUs)", blocks,
                    per_cu, cus);
    GridBarrier *b = reinterpret_cast<GridBarrier *>(state);
    void *args[] = {&b, &barriers};
    const hipError_t e = hipLaunchCooperativeKernel((const void *)grid_barrier_kernel, dim3(blocks), dim3(512), args, 0,
                                                    (hipStream_t)stream);
    return e == hipSuccess ? MOE_OK : fail(MOE_EHIP, "grid-barrier kernel: %s", hipGetErrorString(e));
}

}  // extern "C"
