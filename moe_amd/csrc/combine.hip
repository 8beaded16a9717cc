// combine.hip — weighted combine, shared expert and residual add.
//
// out[t] = sum over t's experts in ascending expert order of w * y, starting
// from +0 with separate multiply and add (src/model.rs:842, 936-942); then
// the shared expert's output, times its sigmoid gate if the layer has one
// (src/model.rs:956-970); then, if asked, residual[t] += out[t]
// (src/model.rs:680-683).  Compiled with -ffp-contract=off, so the order and
// rounding match the reference exactly given the same y.
#include <hip/hip_runtime.h>

#include "moe_internal.h"

namespace moe {
namespace {

__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int t = blockIdx.x;
    const int k = a.k;
    // Permuted rows are grouped by ascending expert, so sorting a token's
    // slots by row sorts them by expert.
    int ps[kMaxTopK];
    float ws[kMaxTopK];
    for (int s = 0; s < k; s++) {
        const int p = a.pos[(size_t)t * k + s];
        const float w = a.wsel[(size_t)t * k + s];
        int j = s;
        while (j > 0 && ps[j - 1] > p) {
            ps[j] = ps[j - 1];
            ws[j] = ws[j - 1];
            j--;
        }
        ps[j] = p;
        ws[j] = w;
    }
    const float g = a.shgate ? a.shgate[t] : 1.0f;
    for (int c = blockIdx.y * 256 + threadIdx.x; c < a.H; c += gridDim.y * 256) {
        float acc = 0.0f;
        for (int s = 0; s < k; s++) {
            float yv = a.y[(size_t)ps[s] * a.H + c];
            for (int q = 1; q < a.parts; q++) yv = yv + a.y[q * a.ypart + (size_t)ps[s] * a.H + c];
            const float prod = ws[s] * yv;
            acc = acc + prod;
        }
        if (a.has_shared) {
            float v = a.ys[(size_t)t * a.H + c];
            for (int q = 1; q < a.parts; q++) v = v + a.ys[q * a.yspart + (size_t)t * a.H + c];
            if (a.shgate) v = v * g;
            acc = acc + v;
        }
        a.out[(size_t)t * a.H + c] = acc;
        if (a.residual) a.residual[(size_t)t * a.H + c] = a.residual[(size_t)t * a.H + c] + acc;
    }
}

}  // namespace

hipError_t launch_combine(const CombineArgs &a, hipStream_t s) {
    int gy = (a.H + 255) / 256;
    if (gy > 8) gy = 8;
    hipLaunchKernelGGL(combine_kernel, dim3(a.T, gy), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
