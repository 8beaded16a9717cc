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

typedef uint32_t qa_u32x4 __attribute__((ext_vector_type(4)));

// A unit from global memory (16-byte aligned) into registers.
__device__ inline void qact_unit_gload(const uint8_t *unit, uint32_t (&x)[kQUnitDw]) {
    typedef const __attribute__((address_space(1))) qa_u32x4 *g4p;
    const g4p p = (g4p)unit;
#pragma unroll
    for (int i = 0; i < kQUnitDw / 4; i++) {
        const qa_u32x4 t = p[i];
        x[4 * i] = t.x, x[4 * i + 1] = t.y, x[4 * i + 2] = t.z, x[4 * i + 3] = t.w;
    }
}

// Store an encoded block into a unit (16-byte aligned) through pointers of
// address space AS (1: global, 3: LDS).
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

// One wavefront encodes one unit, one value per lane: lanes 0..31 form
// block 0, 32..63 block 1.  The block's largest magnitude and the sums of
// its codes come from shuffles inside each half; every lane writes its own
// three level bytes (the unit's bytes i, 64 + i and 128 + i), and lanes 0
// and 32 their block's s3, q01 and q2.  Same bits as qact_block: the
// maximum and the integer sums do not depend on the order they are taken
// in.
__device__ inline void qact_wave_encode(float v, uint8_t *unit, int lane) {
    float amax = fmaxf(0.0f, fabsf(v));  // as the sequential fold from 0
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    int a0, a1, a2;
    qact_encode(v, qact_inv(amax), a0, a1, a2);
    int q01 = 254 * a0 + a1, q2 = a2;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) q01 += __shfl_xor(q01, m, 64), q2 += __shfl_xor(q2, m, 64);
    typedef __attribute__((address_space(1))) uint8_t *g8;
    typedef __attribute__((address_space(1))) float *gf;
    typedef __attribute__((address_space(1))) int32_t *gi;
    ((g8)unit)[lane] = (uint8_t)(a0 & 0xff);
    ((g8)unit)[64 + lane] = (uint8_t)(a1 & 0xff);
    ((g8)unit)[128 + lane] = (uint8_t)(a2 & 0xff);
    if ((lane & 31) == 0) {
        ((gf)(unit + 4 * kQS))[lane >> 5] = qact_s3(amax);
        ((gi)(unit + 4 * kQ01))[lane >> 5] = q01;
        ((gi)(unit + 4 * kQ2))[lane >> 5] = q2;
    }
}

}  // namespace moe
