// model_ops.hip — the decoder around the routed layer, on gfx950.
//
// The reference's forward (src/model.rs:646-834) wraps every routed layer in
// the same few operations; these kernels run them on the device so that a
// whole model stays in HBM between layers:
//   embed_rows_kernel   trunk's embedding lookup (dequant_row of the token's
//                       row, src/model.rs:669-671)
//   rmsnorm_kernel      rmsnorm (src/model.rs:211-216), row by row
//   rope_kernel         rope (src/model.rs:324-333) on chosen heads of rows
//   add_bias_kernel     the q/k/v biases (src/model.rs:707-713)
//   scatter_rows_kernel the KV-cache write of GQA (src/model.rs:732-733)
//   mla_kv_kernel       MLA's expanded key/value rows (src/model.rs:773-787)
//   attention_kernel    causal attention with windows and grouped heads
//                       (src/model.rs:790-831)
//   argmax_kernel       greedy sampling (src/sample.rs:87-95)
// Projections (quant::matmul) run on the expert kernels through moe_linear
// (moe_abi.hip).  Everything computes in f32; sums are reduced in a
// different order than the reference's sequential loops, so results agree
// to f32 rounding, not bit for bit (the argmax ties go to the lower index,
// as the reference's strict `>` scan gives them).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "exact_math.h"
#include "gmem.h"
#include "moe_internal.h"

namespace moe {
int fail(int code, const char *fmt, ...);

namespace {

__device__ inline float half_at(const uint8_t *p) {
    return __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
}

// Value c of a stored row (src/quant.rs:177-227).
__device__ inline float row_value(const uint8_t *row, int dt, int c) {
    const int b = c >> 5, i = c & 31;
    switch (dt) {
    case MOE_DT_F32: {
        float v;
        __builtin_memcpy(&v, row + 4 * (size_t)c, 4);
        return v;
    }
    case MOE_DT_F16: return half_at(row + 2 * (size_t)c);
    case MOE_DT_BF16: {
        const uint32_t u = (uint32_t)(row[2 * (size_t)c] | (row[2 * (size_t)c + 1] << 8)) << 16;
        return __uint_as_float(u);
    }
    case MOE_DT_Q8_0: {
        const uint8_t *blk = row + 34 * (size_t)b;
        return half_at(blk) * (float)(int8_t)blk[2 + i];
    }
    case MOE_DT_Q4_0: {
        const uint8_t *blk = row + 18 * (size_t)b;
        const uint32_t v = blk[2 + (i & 15)];
        const int nib = i < 16 ? (int)(v & 15) : (int)(v >> 4);
        return half_at(blk) * (float)(nib - 8);
    }
    default: {  // Q5_0
        const uint8_t *blk = row + 22 * (size_t)b;
        const uint32_t v = blk[6 + (i & 15)];
        const int nib = i < 16 ? (int)(v & 15) : (int)(v >> 4);
        const int hb = (blk[2 + i / 8] >> (i % 8)) & 1;
        return half_at(blk) * (float)((nib | (hb << 4)) - 16);
    }
    }
}

__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t *__restrict__ table, int dt, uint32_t rows,
                                                         int cols, size_t row_bytes,
                                                         const int32_t *__restrict__ tokens, float *__restrict__ x) {
    const uint32_t tok = (uint32_t)tokens[blockIdx.x] % rows;
    const uint8_t *row = table + (size_t)tok * row_bytes;
    float *o = x + (size_t)blockIdx.x * cols;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) o[c] = row_value(row, dt, c);
}

// Block sum of v (256 threads); every thread receives it.
__device__ inline float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int64_t xs,
                                                      const float *__restrict__ w, int n, float eps,
                                                      float *__restrict__ out, int64_t os) {
    __shared__ float red[4];
    const float *v = x + (size_t)blockIdx.x * xs;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(v[i], v[i], ss);
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    float *o = out + (size_t)blockIdx.x * os;
    for (int i = threadIdx.x; i < n; i += 256) o[i] = (v[i] * scale) * w[i];
}

__global__ __launch_bounds__(256) void rope_kernel(float *__restrict__ x, int64_t rs, int heads, int hs, int off,
                                                   int dim, const int32_t *__restrict__ pos,
                                                   const float *__restrict__ inv, int n_inv) {
    const int half = dim / 2, n = min(half, n_inv);
    const float p = (float)pos[blockIdx.x];
    float *row = x + (size_t)blockIdx.x * rs + off;
    for (int q = threadIdx.x; q < heads * n; q += blockDim.x) {
        const int h = q / n, i = q % n;
        float *hx = row + (size_t)h * hs;
        const float ang = p * inv[i];
        const float s = sinf(ang), c = cosf(ang);
        const float a = hx[i], b = hx[i + half];
        hx[i] = a * c - b * s;
        hx[i + half] = a * s + b * c;
    }
}

__global__ void add_bias_kernel(float *__restrict__ x, size_t total, const float *__restrict__ b, int blen) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x)
        x[i] += b[i % blen];
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(const float *__restrict__ src, int n, int64_t ss,
                                                           float *__restrict__ dst, int64_t ds,
                                                           const int64_t *__restrict__ dst_rows) {
    const float *s = src + (size_t)blockIdx.x * ss;
    float *d = dst + (size_t)dst_rows[blockIdx.x] * ds;
    for (int c = threadIdx.x; c < n; c += blockDim.x) d[c] = s[c];
}

// MLA: head h of cache row dst_rows[r] gets key [kv nope part, shared k_pe]
// and value kv's value part (src/model.rs:773-787).
__global__ __launch_bounds__(256) void mla_kv_kernel(const float *__restrict__ kv, const float *__restrict__ c,
                                                     int64_t cs, int kv_lora, int heads, int nope, int rope, int vd,
                                                     float *__restrict__ kc, float *__restrict__ vc,
                                                     const int64_t *__restrict__ dst_rows) {
    const int r = blockIdx.x, qd = nope + rope, kvw = nope + vd;
    const float *src = kv + (size_t)r * heads * kvw;
    const float *kpe = c + (size_t)r * cs + kv_lora;
    float *kd = kc + (size_t)dst_rows[r] * heads * qd;
    float *vv = vc + (size_t)dst_rows[r] * heads * vd;
    for (int q = threadIdx.x; q < heads * qd; q += blockDim.x) {
        const int h = q / qd, i = q % qd;
        kd[q] = i < nope ? src[h * kvw + i] : kpe[i - nope];
    }
    for (int q = threadIdx.x; q < heads * vd; q += blockDim.x) {
        const int h = q / vd, i = q % vd;
        vv[q] = src[h * kvw + nope + i];
    }
}

// One wavefront per (row, head): scores of positions [lo, p] (one lane per
// position, the key read as a contiguous row), softmax with glibc's expf,
// then the weighted sum of values (one lane per output column, positions
// in order).
constexpr int kAttnMaxDim = 256;
__global__ __launch_bounds__(64) void attention_kernel(const float *__restrict__ q, int64_t q_stride, int heads,
                                                       int n_kv, int qd, int vd, float scale,
                                                       const float *__restrict__ kc, const float *__restrict__ vc,
                                                       int64_t ctx, const int32_t *__restrict__ seq,
                                                       const int32_t *__restrict__ pos, int window,
                                                       float *__restrict__ out, int64_t out_stride) {
    extern __shared__ float sc[];
    __shared__ float qs[kAttnMaxDim];
    const int r = blockIdx.x / heads, h = blockIdx.x % heads, lane = threadIdx.x;
    const int p = pos[r];
    const int lo = window > 0 ? max(0, p + 1 - window) : 0;
    const int n = p + 1 - lo;
    const int rep = heads / max(n_kv, 1);
    const int kvh = rep > 1 ? h / rep : min(h, n_kv - 1);
    const size_t kd = (size_t)n_kv * qd, vdim = (size_t)n_kv * vd;
    const float *qv = q + (size_t)r * q_stride + (size_t)h * qd;
    for (int i = lane; i < qd; i += 64) qs[i] = qv[i];
    __syncthreads();
    const float *kbase = kc + ((size_t)seq[r] * ctx) * kd + (size_t)kvh * qd;
    const float *vbase = vc + ((size_t)seq[r] * ctx) * vdim + (size_t)kvh * vd;
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64) {
        const float *k = kbase + (size_t)(lo + j) * kd;
        float d = 0.0f;
        for (int i = 0; i < qd; i++) d = fmaf(qs[i], k[i], d);
        const float s = d * scale;
        sc[j] = s;
        m = fmaxf(m, s);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float sum = 0.0f;
    for (int j = lane; j < n; j += 64) {
        const float e = expf_exact(sc[j] - m);
        sc[j] = e;
        sum += e;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    __syncthreads();
    float *o = out + (size_t)r * out_stride + (size_t)h * vd;
    for (int c = lane; c < vd; c += 64) {
        float acc = 0.0f;
        for (int j = 0; j < n; j++) {
            const float w = sc[j] / sum;
            acc += w * vbase[(size_t)(lo + j) * vdim + c];
        }
        o[c] = acc;
    }
}

// First index of the row's maximum.
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ x, int n, int32_t *__restrict__ out) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const float *row = x + (size_t)blockIdx.x * n;
    float best = -INFINITY;
    int idx = n;
    for (int i = threadIdx.x; i < n; i += 256)
        if (row[i] > best || idx == n) best = row[i], idx = i;
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int s = 128; s >= 1; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = bv[threadIdx.x + s];
            const int oi = bi[threadIdx.x + s];
            if (oi < n && (bi[threadIdx.x] == n || ov > bv[threadIdx.x] || (ov == bv[threadIdx.x] && oi < bi[threadIdx.x])))
                bv[threadIdx.x] = ov, bi[threadIdx.x] = oi;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = bi[0];
}

__global__ void add_kernel(float *__restrict__ dst, const float *__restrict__ src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] += src[i];
}

// Diagnostics: the HBM read ceiling.  Grid-stride 16-byte loads, eight in
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

// Diagnostics: the cost of a grid-wide barrier.  `barriers` barriers of
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

// y = sum over the k parts (p ascending) of parts[p n + i]; residual[i] +=
// y[i] when given.  The K parts of a split projection.
__global__ __launch_bounds__(256) void sum_parts_kernel(const float *__restrict__ parts, int k, size_t n,
                                                        float *__restrict__ y, float *__restrict__ residual) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = parts[i];
        for (int p = 1; p < k; p++) v = v + parts[(size_t)p * n + i];
        y[i] = v;
        if (residual) residual[i] = residual[i] + v;
    }
}

int launch_rc(const char *what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_OK : fail(MOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

hipError_t launch_sum_parts(const float *parts, int k, size_t n, float *y, float *residual, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (k <= 0) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(sum_parts_kernel, dim3(blocks), dim3(256), 0, s, parts, k, n, y, residual);
    return hipGetLastError();
}

hipError_t launch_add(float *dst, const float *src, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(add_kernel, dim3(blocks), dim3(256), 0, s, dst, src, n);
    return hipGetLastError();
}

}  // namespace moe

using namespace moe;

extern "C" {

int moe_embed_rows(const void *table, int32_t dt, int32_t rows, int32_t cols, const int32_t *tokens, int32_t t,
                   float *x, void *stream) {
    const uint64_t rb = moe_row_bytes(dt, (uint64_t)cols);
    if (!table || !tokens || !x || rows <= 0 || cols <= 0 || t < 0 || rb == 0 ||
        (dt != MOE_DT_F32 && dt != MOE_DT_F16 && dt != MOE_DT_BF16 && cols % 32))
        return fail(MOE_EINVAL, "moe_embed_rows: bad argument");
    if (t == 0) return MOE_OK;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(t), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const uint8_t *>(table), dt, (uint32_t)rows, cols, (size_t)rb, tokens, x);
    return launch_rc("embedding kernel");
}

int moe_rmsnorm(const float *x, int64_t x_stride, const float *w, int32_t rows, int32_t n, float eps, float *out,
                int64_t out_stride, void *stream) {
    if (!x || !w || !out || rows < 0 || n <= 0) return fail(MOE_EINVAL, "moe_rmsnorm: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, x_stride, w, n, eps, out,
                       out_stride);
    return launch_rc("rmsnorm kernel");
}

int moe_rope(float *x, int32_t rows, int64_t row_stride, int32_t heads, int32_t head_stride, int32_t offset,
             int32_t dim, const int32_t *pos, const float *inv_freq, int32_t n_inv, void *stream) {
    if (!x || !pos || !inv_freq || rows < 0 || heads <= 0 || dim <= 0 || n_inv < 0)
        return fail(MOE_EINVAL, "moe_rope: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(rope_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, row_stride, heads, head_stride,
                       offset, dim, pos, inv_freq, n_inv);
    return launch_rc("rope kernel");
}

int moe_add_bias(float *x, uint64_t total, const float *bias, int32_t bias_len, void *stream) {
    if (!x || !bias || bias_len <= 0) return fail(MOE_EINVAL, "moe_add_bias: bad argument");
    if (total == 0) return MOE_OK;
    const unsigned blocks = (unsigned)std::min<uint64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(add_bias_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, (size_t)total, bias,
                       bias_len);
    return launch_rc("bias kernel");
}

int moe_scatter_rows(const float *src, int32_t rows, int32_t n, int64_t src_stride, float *dst, int64_t dst_stride,
                     const int64_t *dst_rows, void *stream) {
    if (!src || !dst || !dst_rows || rows < 0 || n <= 0) return fail(MOE_EINVAL, "moe_scatter_rows: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(scatter_rows_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, src, n, src_stride, dst,
                       dst_stride, dst_rows);
    return launch_rc("cache write kernel");
}

int moe_mla_kv_store(const float *kv, const float *c, int64_t c_stride, int32_t kv_lora, int32_t rows,
                     int32_t heads, int32_t qk_nope, int32_t qk_rope, int32_t v_head, float *kcache, float *vcache,
                     const int64_t *dst_rows, void *stream) {
    if (!kv || !c || !kcache || !vcache || !dst_rows || rows < 0 || heads <= 0)
        return fail(MOE_EINVAL, "moe_mla_kv_store: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(mla_kv_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, kv, c, c_stride, kv_lora, heads,
                       qk_nope, qk_rope, v_head, kcache, vcache, dst_rows);
    return launch_rc("MLA cache write kernel");
}

int moe_attention(const float *q, int64_t q_stride, int32_t rows, int32_t heads, int32_t n_kv, int32_t qd,
                  int32_t vd, float scale, const float *kcache, const float *vcache, int64_t ctx, const int32_t *seq,
                  const int32_t *pos, int32_t max_pos, int32_t window, float *out, int64_t out_stride,
                  void *stream) {
    if (!q || !kcache || !vcache || !seq || !pos || !out || rows < 0 || heads <= 0 || n_kv <= 0 || qd <= 0 ||
        vd <= 0 || qd > kAttnMaxDim || max_pos < 0 || max_pos >= ctx)
        return fail(MOE_EINVAL, "moe_attention: bad argument (qd %d, vd %d, max position %d, context %lld)", qd, vd,
                    max_pos, (long long)ctx);
    if (rows == 0) return MOE_OK;
    const int span = window > 0 ? std::min(window, max_pos + 1) : max_pos + 1;
    const size_t lds = (size_t)span * 4;
    if (lds > 64 * 1024) return fail(MOE_EUNSUP, "moe_attention: %d positions exceed the score buffer", span);
    // Past 32 KiB of scores the launch asks for the larger dynamic LDS limit
    // (on the current device, every time: the setting is per device).
    if (lds > 32 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *)attention_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
        if (e != hipSuccess) return fail(MOE_EHIP, "moe_attention: LDS limit: %s", hipGetErrorString(e));
    }
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)rows * heads), dim3(64), lds, (hipStream_t)stream, q,
                       q_stride, heads, n_kv, qd, vd, scale, kcache, vcache, ctx, seq, pos, window, out, out_stride);
    return launch_rc("attention kernel");
}

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

int moe_argmax(const float *x, int32_t rows, int32_t n, int32_t *out, void *stream) {
    if (!x || !out || rows < 0 || n <= 0) return fail(MOE_EINVAL, "moe_argmax: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, n, out);
    return launch_rc("argmax kernel");
}

}  // extern "C"
