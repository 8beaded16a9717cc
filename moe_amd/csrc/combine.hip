// combine.hip — weighted combine, shared expert and residual add.
//
// out[t] = sum over t's experts in ascending expert order of w * y, starting
// from +0 with separate multiply and add (src/model.rs:842, 936-942); then
// the shared expert's output, times its sigmoid gate if the layer has one
// (src/model.rs:956-970); then, if asked, residual[t] += out[t]
// (src/model.rs:680-683).  Compiled with -ffp-contract=off, so the order and
// rounding match the reference exactly given the same y.
//
// One block per (token, column range); a thread owns four consecutive
// columns (one 16-byte load per partial row) when H is a multiple of 4.
#include <hip/hip_runtime.h>

#include "moe_internal.h"

namespace moe {
namespace {

constexpr int kThreads = 256;

__device__ inline float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ inline float4 mul4(float s, float4 a) { return make_float4(s * a.x, s * a.y, s * a.z, s * a.w); }

template <bool VEC>
__global__ __launch_bounds__(kThreads) void combine_kernel(CombineArgs a) {
    const int t = blockIdx.x;
    const int k = a.k;
    // The token's slots sorted by permuted row.  Rows are grouped by
    // ascending expert and a token meets an expert at most once, so the rows
    // are distinct and a slot's rank is the number of rows below it.
    __shared__ int ps[kMaxTopK];
    __shared__ float ws[kMaxTopK];
    if ((int)threadIdx.x < k) {
        const int p = a.pos[(size_t)t * k + threadIdx.x];
        int rank = 0;
        for (int s = 0; s < k; s++) rank += a.pos[(size_t)t * k + s] < p;
        ps[rank] = p;
        ws[rank] = a.wsel[(size_t)t * k + threadIdx.x];
    }
    __syncthreads();
    const float g = a.shgate ? a.shgate[t] : 1.0f;
    const size_t orow = (size_t)t * a.H;
    if constexpr (VEC) {
        const int H4 = a.H >> 2;
        for (int c = blockIdx.y * kThreads + threadIdx.x; c < H4; c += gridDim.y * kThreads) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int s = 0; s < k; s++) {
                const float4 *yp = reinterpret_cast<const float4 *>(a.y + (size_t)ps[s] * a.H) + c;
                float4 yv = *yp;
                for (int q = 1; q < a.parts; q++) yv = add4(yv, *reinterpret_cast<const float4 *>(
                                                                   reinterpret_cast<const float *>(yp) + q * a.ypart));
                acc = add4(acc, mul4(ws[s], yv));
            }
            if (a.has_shared) {
                const float4 *sp = reinterpret_cast<const float4 *>(a.ys + orow) + c;
                float4 v = *sp;
                for (int q = 1; q < a.parts; q++)
                    v = add4(v, *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(sp) + q * a.yspart));
                if (a.shgate) v = mul4(g, v);
                acc = add4(acc, v);
            }
            reinterpret_cast<float4 *>(a.out + orow)[c] = acc;
            if (a.residual) {
                float4 *rp = reinterpret_cast<float4 *>(a.residual + orow) + c;
                *rp = add4(*rp, acc);
            }
        }
    } else {
        for (int c = blockIdx.y * kThreads + threadIdx.x; c < a.H; c += gridDim.y * kThreads) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) {
                float yv = a.y[(size_t)ps[s] * a.H + c];
                for (int q = 1; q < a.parts; q++) yv = yv + a.y[q * a.ypart + (size_t)ps[s] * a.H + c];
                const float prod = ws[s] * yv;
                acc = acc + prod;
            }
            if (a.has_shared) {
                float v = a.ys[orow + c];
                for (int q = 1; q < a.parts; q++) v = v + a.ys[q * a.yspart + orow + c];
                if (a.shgate) v = v * g;
                acc = acc + v;
            }
            a.out[orow + c] = acc;
            if (a.residual) a.residual[orow + c] = a.residual[orow + c] + acc;
        }
    }
}

}  // namespace

hipError_t launch_combine(const CombineArgs &a, hipStream_t s) {
    if (a.k > kMaxTopK) return hipErrorInvalidValue;
    const bool vec = (a.H & 3) == 0 && ((uintptr_t)a.y & 15) == 0 && ((uintptr_t)a.out & 15) == 0 &&
                     (!a.has_shared || ((uintptr_t)a.ys & 15) == 0) && (!a.residual || ((uintptr_t)a.residual & 15) == 0) &&
                     (a.ypart & 3) == 0 && (a.yspart & 3) == 0;
    const int per = vec ? 4 * kThreads : kThreads;
    int gy = (a.H + per - 1) / per;
    if (gy > 8) gy = 8;
    if (vec)
        hipLaunchKernelGGL(combine_kernel<true>, dim3(a.T, gy), dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL(combine_kernel<false>, dim3(a.T, gy), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
