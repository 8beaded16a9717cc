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

// The 32 lanes of a half wave hold the values of block g of one row (lane i
// value i): quantise them and store the block into the row's units.
__device__ inline void qact_store_block(float v, int lane32, uint8_t *row, int g) {
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    int hi, lo;
    qact_encode(v, qact_inv(amax), hi, lo);
    int q = 254 * hi + lo;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) q += __shfl_xor(q, m, 32);
    uint8_t *u = row + (size_t)(g >> 1) * kQUnitBytes;
    const int half = (g & 1) * 32;
    u[half + lane32] = (uint8_t)(int8_t)hi;
    u[64 + half + lane32] = (uint8_t)(int8_t)lo;
    if (lane32 == 0) {
        reinterpret_cast<float *>(u + 128)[g & 1] = qact_s2(amax);
        reinterpret_cast<int32_t *>(u + 136)[g & 1] = q;
    }
}

// One thread encodes the 32 floats at src (16-byte aligned) as block
// `half` (0 or 1) of the unit at `unit` (16-byte aligned, any address space).
__device__ inline void qact_block_store(const float *src, uint8_t *unit, int half) {
    float v[32];
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 f = s4[i];
        v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float inv = qact_inv(amax);
    uint32_t hw[8], lw[8];
    int sq = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        hw[d] = 0, lw[d] = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int hi, lo;
            qact_encode(v[4 * d + j], inv, hi, lo);
            hw[d] |= ((uint32_t)hi & 0xffu) << (8 * j);
            lw[d] |= ((uint32_t)lo & 0xffu) << (8 * j);
            sq += 254 * hi + lo;
        }
    }
    uint4 *h4 = reinterpret_cast<uint4 *>(unit + 32 * half);
    uint4 *l4 = reinterpret_cast<uint4 *>(unit + 64 + 32 * half);
    h4[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    h4[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
    l4[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    l4[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
    reinterpret_cast<float *>(unit + 128)[half] = qact_s2(amax);
    reinterpret_cast<int32_t *>(unit + 136)[half] = sq;
}

// Encode the 64 floats at src (16-byte aligned) as one unit in registers,
// laid out as the 36 dwords of the stored form.
__device__ inline void qact_unit_from_f32(const float *src, uint32_t (&xa)[kQUnitDw]) {
#pragma unroll
    for (int b = 0; b < 2; b++) {
        float v[32];
        const float4 *s4 = reinterpret_cast<const float4 *>(src + 32 * b);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = s4[i];
            v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
        }
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
            xa[8 * b + d] = hw;
            xa[16 + 8 * b + d] = lw;
        }
        xa[32 + b] = __float_as_uint(qact_s2(amax));
        xa[34 + b] = (uint32_t)sq;
        // Keep the two blocks' loads apart: one block of floats live at a time.
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace moe
