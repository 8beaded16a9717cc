// qact.h — two-level int8 activations for the decode kernels.
//
// A row of activations is stored as 64-value units of 144 bytes:
//   [0, 64)     hi  int8, one per value
//   [64, 128)   lo  int8, one per value
//   [128, 136)  s2  float per 32-value block
//   [136, 144)  sq  int32 per block: sum of (254 * hi + lo) over the block
// and value i stands for s2[b] * (254 * hi[i] + lo[i]), b = i / 32.  With
// s = amax / 127 for the block's largest magnitude amax, hi = rint(x / s) and
// lo = rint(254 * (x / s - hi)), so the representation error is at most
// amax / (127 * 508) per value (2^-16 of the block's range), about 12 times
// finer than rounding to f16.  A quantised weight block dotted with it is an
// exact integer sum (v_dot4_i32_i8) times one float scale.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kQUnitBytes = 144;  // one 64-value unit
constexpr int kQUnitDw = 36;

__device__ inline float qact_s2(float amax) { return amax > 0.0f ? (amax / 127.0f) / 254.0f : 0.0f; }

// hi and lo of value v in a block whose largest magnitude is amax; `inv` is
// 127 / amax, or 0 for an all-zero block (every value then encodes as 0).
__device__ inline void qact_encode(float v, float inv, int &hi, int &lo) {
    const float t = v * inv;
    const float fh = fminf(fmaxf(rintf(t), -127.0f), 127.0f);
    const float fl = fminf(fmaxf(rintf((t - fh) * 254.0f), -127.0f), 127.0f);
    hi = (int)fh, lo = (int)fl;
}
__device__ inline float qact_inv(float amax) { return amax > 0.0f ? 127.0f / amax : 0.0f; }

// One thread encodes 32 values as block `half` (0 or 1) of a unit: the
// unit's hi dwords, lo dwords, s2 and sq for that block.
struct QBlock {
    uint32_t hw[8], lw[8];
    float s2;
    int32_t sq;
};
__device__ inline QBlock qact_block(const float (&v)[32]) {
    QBlock q;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float inv = qact_inv(amax);
    int sq = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        uint32_t hw = 0, lw = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int hi, lo;
            qact_encode(v[4 * d + j], inv, hi, lo);
            hw |= ((uint32_t)hi & 0xffu) << (8 * j);
            lw |= ((uint32_t)lo & 0xffu) << (8 * j);
            sq += 254 * hi + lo;
        }
        q.hw[d] = hw, q.lw[d] = lw;
    }
    q.s2 = qact_s2(amax);
    q.sq = sq;
    return q;
}

// A whole unit in registers, laid out as in memory (hi dwords 0..15, lo
// dwords 16..31, s2 at 32..33, sq at 34..35): the same bits qact_block_put
// stores.  Loading (64 values, 16-byte aligned, global memory) and encoding
// are separate so a caller can issue other loads in between.
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
        for (int d = 0; d < 8; d++) x[8 * b + d] = q.hw[d], x[16 + 8 * b + d] = q.lw[d];
        x[32 + b] = __float_as_uint(q.s2);
        x[34 + b] = (uint32_t)q.sq;
    }
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
    v4p h4 = (v4p)(unit + 32 * half);
    v4p l4 = (v4p)(unit + 64 + 32 * half);
    h4[0] = qa_u32x4{q.hw[0], q.hw[1], q.hw[2], q.hw[3]};
    h4[1] = qa_u32x4{q.hw[4], q.hw[5], q.hw[6], q.hw[7]};
    l4[0] = qa_u32x4{q.lw[0], q.lw[1], q.lw[2], q.lw[3]};
    l4[1] = qa_u32x4{q.lw[4], q.lw[5], q.lw[6], q.lw[7]};
    ((fp)(unit + 128))[half] = q.s2;
    ((ip)(unit + 136))[half] = q.sq;
}

}  // namespace moe
