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

int moe_argmax(const float *x, int32_t rows, int32_t n, int32_t *out, void *stream) {
    if (!x || !out || rows < 0 || n <= 0) return fail(MOE_EINVAL, "moe_argmax: bad argument");
    if (rows == 0) return MOE_OK;
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, n, out);
    return launch_rc("argmax kernel");
}

}  // extern "C"
