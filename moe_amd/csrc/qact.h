// qact.h — three-level int8 activations for the integer-dot expert kernels.
//
// A row of activations is stored as 64-value units of 224 bytes:
//   [0, 64)     a0   int8, one per value
//   [64, 128)   a1   int8, one per value
//   [128, 192)  a2   int8, one per value
//   [192, 200)  s3   float per 32-value block
//   [200, 208)  q01  int32 per block: sum of (254 a0 + a1) over the block
//   [208, 216)  q2   int32 per block: sum of a2 over the block
//   [216, 224)  padding (units stay 16-byte aligned)
// and value i stands for s3[b] * (254^2 a0[i] + 254 a1[i] + a2[i]),
// b = i / 32.  With s = amax / 127 for the block's largest magnitude amax,
// t = x / s, a0 = rint(t), a1 = rint(254 (t - a0)) and
// a2 = rint(254 (254 (t - a0) - a1)), so the representation error is at most
// amax / (127 * 2 * 254^2) per value — 2^-24 of the block's range, the
// rounding step of f32 at the block's largest value.  A quantised weight
// block dotted with it is three exact integer sums (v_dot4_i32_i8) finished
// by one float scale, so the product path computes in f32 precision.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kQUnitBytes = 224;  // one 64-value unit
constexpr int kQUnitDw = 56;
constexpr int kQA1 = 16, kQA2 = 32;  // first dword of a1 and a2
constexpr int kQS = 48, kQ01 = 50, kQ2 = 52;  // s3, q01 and q2 dwords (block 0, then block 1)

__device__ inline float qact_s3(float amax) { return amax > 0.0f ? ((amax / 127.0f) / 254.0f) / 254.0f : 0.0f; }
__device__ inline float qact_inv(float amax) { return amax > 0.0f ? 127.0f / amax : 0.0f; }

// The three levels of value v in a block whose largest magnitude is amax;
// `inv` is 127 / amax, or 0 for an all-zero block (every value then encodes
// as 0).  t - a0 and r - a1 are exact in f32 (|t| <= 127 after rounding).
__device__ inline void qact_encode(float v, float inv, int &a0, int &a1, int &a2) {
    const float t = v * inv;
    const float f0 = fminf(fmaxf(rintf(t), -127.0f), 127.0f);
    const float r = (t - f0) * 254.0f;
    const float f1 = fminf(fmaxf(rintf(r), -127.0f), 127.0f);
    const float f2 = fminf(fmaxf(rintf((r - f1) * 254.0f), -127.0f), 127.0f);
    a0 = (int)f0, a1 = (int)f1, a2 = (int)f2;
}

// One thread encodes 32 values as block `half` (0 or 1) of a unit.
struct QBlock {
    uint32_t w0[8], w1[8], w2[8];
    float s3;
    int32_t q01, q2;
};
__device__ inline QBlock qact_block(const float (&v)[32]) {
    QBlock q;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float inv = qact_inv(amax);
    int q01 = 0, q2 = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int a0, a1, a2;
            qact_encode(v[4 * d + j], inv, a0, a1, a2);
            w0 |= ((uint32_t)a0 & 0xffu) << (8 * j);
            w1 |= ((uint32_t)a1 & 0xffu) << (8 * j);
            w2 |= ((uint32_t)a2 & 0xffu) << (8 * j);
            q01 += 254 * a0 + a1;
            q2 += a2;
        }
        q.w0[d] = w0, q.w1[d] = w1, q.w2[d] = w2;
    }
    q.s3 = qact_s3(amax);
    q.q01 = q01;
    q.q2 = q2;
    return q;
}

// A whole unit in registers, laid out as in memory: the same bits
// qact_block_put stores.  Loading (64 values, 16-byte aligned, global
// memory) and encoding are separate so a caller can issue other loads in
// between.
typedef float qa_f32x4 __attribute__((ext_vector_type(4)));
__device__ inline void qact_unit_load(const float *v, float (&f)[64]) {
    // Global loads (not flat ones, which LDS waits would also wait for).
    typedef const __attribute__((address_space(1))) qa_f32x4 *g4p;
    const g4p s4 = (g4p)v;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const qa_f32x4 t = s4[i];
        f[4 * i] = t.x, f[4 * i + 1] = t.y, f[4 * i + 2] = t.z, f[4 * i + 3] = t.w;
    }
}
__device__ inline void qact_unit_encode(const float (&f)[64], uint32_t (&x)[kQUnitDw]) {
#pragma unroll
    for (int b = 0; b < 2; b++) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = f[32 * b + i];
        const QBlock q = qact_block(v);
#pragma unroll
        for (int d = 0; d < 8; d++) x[8 * b + d] = q.w0[d], x[kQA1 + 8 * b + d] = q.w1[d], x[kQA2 + 8 * b + d] = q.w2[d];
        x[kQS + b] = __float_as_uint(q.s3);
        x[kQ01 + b] = (uint32_t)q.q01;
        x[kQ2 + b] = (uint32_t)q.q2;
    }
    x[54] = 0u, x[55] = 0u;
}
__device__ inline void qact_unit_from_f32(const float *v, uint32_t (&x)[kQUnitDw]) {
    float f[64];
    qact_unit_load(v, f);
    qact_unit_encode(f, x);
}

// Store an encoded block into a unit (16-byte aligned) through pointers of
// address space AS (1: global, 3: LDS).
typedef uint32_t qa_u32x4 __attribute__((ext_vector_type(4)));
template <int AS>
__device__ inline void qact_block_put(const QBlock &q, uint8_t *unit, int half) {
    typedef __attribute__((address_space(AS))) qa_u32x4 *v4p;
    typedef __attribute__((address_space(AS))) float *fp;
    typedef __attribute__((address_space(AS))) int32_t *ip;
#pragma unroll
    for (int l = 0; l < 3; l++) {
        const uint32_t *w = l == 0 ? q.w0 : l == 1 ? q.w1 : q.w2;
        v4p p = (v4p)(unit + 64 * l + 32 * half);
        p[0] = qa_u32x4{w[0], w[1], w[2], w[3]};
        p[1] = qa_u32x4{w[4], w[5], w[6], w[7]};
    }
    ((fp)(unit + 4 * kQS))[half] = q.s3;
    ((ip)(unit + 4 * kQ01))[half] = q.q01;
    ((ip)(unit + 4 * kQ2))[half] = q.q2;
}

}  // namespace moe
