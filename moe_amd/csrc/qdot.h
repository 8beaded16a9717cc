// qdot.h — quantised weight units dotted with three-level int8 activations.
//
// Shared by the one-token kernels and the few-tokens-per-expert kernels: a
// 64-value unit of a Q4_0 / Q5_0 / Q8_0 weight row (two 32-value blocks) is
// loaded into registers and dotted with an activation unit (qact.h) by
// v_dot4_i32_i8; the integer sums are exact, one float scale per block
// finishes them.  Lane-slice sums use DPP.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "gmem.h"
#include "moe_internal.h"
#include "qact.h"

namespace moe {
namespace qd {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)(bits & 0xffff))); }
__device__ inline uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t s) { return __builtin_amdgcn_alignbyte(hi, lo, s); }
__device__ inline int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
// Bits 0..3 of h moved to bit 4 of bytes 0..3.
__device__ inline uint32_t spread4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

// A 64-value unit of a weight row: two quantisation blocks, 4-byte aligned.
template <int DT>
struct WUnit;
template <>
struct WUnit<MOE_DT_Q4_0> {
    static constexpr int dw = 9, bytes = 36;
};
template <>
struct WUnit<MOE_DT_Q5_0> {
    static constexpr int dw = 11, bytes = 44;
};
template <>
struct WUnit<MOE_DT_Q8_0> {
    static constexpr int dw = 17, bytes = 68;
};

// Loads the first WUnit<DT>::dw entries of d (a buffer sized for the widest
// format in use).
template <int DT, int DN>
__device__ inline void load_wunit(const uint8_t *p, uint32_t (&d)[DN]) {
    static_assert(DN >= WUnit<DT>::dw, "unit buffer too small");
    const uint32_t *q = reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p, 4));
    constexpr int N = WUnit<DT>::dw;
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const u32x4_dw v = gload_x4(q + i);
        d[i] = v.x, d[i + 1] = v.y, d[i + 2] = v.z, d[i + 3] = v.w;
    }
#pragma unroll
    for (int i = N & ~3; i < N; i++) d[i] = gload(q + i);
}

// The activation unit (144 bytes, 16-byte aligned) into 36 registers, from
// address space AS (1: global, 3: LDS).
template <int AS>
__device__ inline void load_qunit(const uint8_t *p, uint32_t (&x)[kQUnitDw]) {
    typedef const __attribute__((address_space(AS))) u32x4 *v4p;
    const v4p q = (v4p)p;
#pragma unroll
    for (int i = 0; i < kQUnitDw / 4; i++) {
        const u32x4 v = q[i];
        x[4 * i] = v.x, x[4 * i + 1] = v.y, x[4 * i + 2] = v.z, x[4 * i + 3] = v.w;
    }
}

// Dot of a weight unit with an activation unit: qdot_multi for one token.
template <int DT, int DN, int NT>
__device__ inline void qdot_multi(const uint32_t (&d)[DN], const uint32_t (&x)[NT][kQUnitDw], float (&out)[NT]);
template <int DT, int DN>
__device__ inline float qdot(const uint32_t (&d)[DN], const uint32_t (&x)[kQUnitDw]) {
    const uint32_t(&xs)[1][kQUnitDw] = reinterpret_cast<const uint32_t(&)[1][kQUnitDw]>(x);
    float r[1];
    qdot_multi<DT, DN, 1>(d, xs, r);
    return r[0];
}

// Sum over groups of CG consecutive lanes (CG = 16, 32, 64); every lane of
// a group receives the same sum.  The first four steps are DPP moves inside
// a row of 16 lanes.
__device__ inline float dpp_add(float v, int ctrl) {
    int r;
    switch (ctrl) {
    case 0: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false); break;   // quad [1,0,3,2]
    case 1: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false); break;   // quad [2,3,0,1]
    case 2: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false); break;  // half-row mirror
    default: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false); break; // row mirror
    }
    return v + __int_as_float(r);
}
// Sums over slices of CG consecutive lanes (CG = 16, 32, 64): afterwards
// the last lane of each slice holds its slice's sum (every lane of it for
// CG = 16).  Rows of 16 lanes reduce through quad permutes and mirrors; rows
// join through row broadcasts, which leave the total in the last lane.
__device__ inline float slice_sum(float v, int cg) {
    v = dpp_add(v, 0);
    v = dpp_add(v, 1);
    v = dpp_add(v, 2);
    v = dpp_add(v, 3);
    if (cg >= 32) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
    if (cg >= 64) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));
    return v;
}

__device__ inline float silu_mul(float g, float u) { return (g / (1.0f + __expf(-g))) * u; }

// Lanes of a row slice: CG lanes (16, 32, 64) own UPL units each (1, or 2
// for rows of 65..128 units: units c and c + 64 of lane c).
__device__ inline int lanes_for(int units) { return units <= 16 ? 16 : units <= 32 ? 32 : 64; }

// A weight unit dotted with the activation units of NT tokens: out[t] for
// every t (the weights are unpacked once for all of them; callers pad with
// all-zero units, whose dots are zero).
//   Q4_0 [dA qA0..15][dB qB0..15]: byte j holds value j (low nibble) and
//        value j + 16 (high nibble), stored unsigned with offset 8.
//   Q5_0 [dA hA(4) qA][dB hB qB]: bit j of h is bit 4 of value j, offset 16.
//   Q8_0 [dA qA0..31][dB qB0..31]: signed bytes.
// For a block with codes c_i = q_i + o: sum_i d q_i x_i =
// d s3 (254 (254 A + B) + C) with A = sum c a0, B = sum c a1 - o q01 and
// C = sum c a2 - o q2 (the offset folded into the finer levels' starting
// values).  Every sum is an exact int32 (|254 A + B| < 2^31); the two
// conversions and the fma round as f32 arithmetic does.
template <int DT, int DN, int NT>
__device__ inline void qdot_multi(const uint32_t (&d)[DN], const uint32_t (&x)[NT][kQUnitDw], float (&out)[NT]) {
    static_assert(DN >= WUnit<DT>::dw, "unit buffer too small");
    int A[NT][2], B[NT][2], Cs[NT][2];
    float sa, sb;
    constexpr int off = DT == MOE_DT_Q4_0 ? 8 : DT == MOE_DT_Q5_0 ? 16 : 0;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            A[t][b] = 0;
            B[t][b] = -off * (int)x[t][kQ01 + b];
            Cs[t][b] = -off * (int)x[t][kQ2 + b];
        }
    // Codes dword c of block b (four consecutive values starting at value
    // 4 (c % 4) + 16 (c / 4) for nibble formats, 4 c for Q8_0) against the
    // matching dword of every level.
    auto dot3 = [&](uint32_t c, int b, int dw) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            A[t][b] = sdot4(c, x[t][8 * b + dw], A[t][b]);
            B[t][b] = sdot4(c, x[t][kQA1 + 8 * b + dw], B[t][b]);
            Cs[t][b] = sdot4(c, x[t][kQA2 + 8 * b + dw], Cs[t][b]);
        }
    };
    if constexpr (DT == MOE_DT_Q4_0 || DT == MOE_DT_Q5_0) {
        constexpr bool q5 = DT == MOE_DT_Q5_0;
        sa = h2f(d[0]), sb = h2f(d[q5 ? 5 : 4] >> 16);
        const uint32_t hA = q5 ? alignb(d[1], d[0], 2) : 0u, hB = q5 ? d[6] : 0u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t qa = q5 ? alignb(d[i + 2], d[i + 1], 2) : alignb(d[i + 1], d[i], 2);
            const uint32_t qb = q5 ? d[7 + i] : d[5 + i];
            uint32_t la = qa & 0x0f0f0f0fu, ha = (qa >> 4) & 0x0f0f0f0fu;
            uint32_t lb = qb & 0x0f0f0f0fu, hb = (qb >> 4) & 0x0f0f0f0fu;
            if constexpr (q5) {
                la |= spread4((hA >> (4 * i)) & 0xfu), ha |= spread4((hA >> (16 + 4 * i)) & 0xfu);
                lb |= spread4((hB >> (4 * i)) & 0xfu), hb |= spread4((hB >> (16 + 4 * i)) & 0xfu);
            }
            dot3(la, 0, i), dot3(ha, 0, 4 + i);
            dot3(lb, 1, i), dot3(hb, 1, 4 + i);
        }
    } else {
        sa = h2f(d[0]), sb = h2f(d[8] >> 16);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            dot3(alignb(d[i + 1], d[i], 2), 0, i);
            dot3(d[9 + i], 1, i);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float fa = fmaf((float)(254 * A[t][0] + B[t][0]), 254.0f, (float)Cs[t][0]);
        const float fb = fmaf((float)(254 * A[t][1] + B[t][1]), 254.0f, (float)Cs[t][1]);
        const float s3a = __uint_as_float(x[t][kQS]), s3b = __uint_as_float(x[t][kQS + 1]);
        out[t] = fmaf(sb * s3b, fb, (sa * s3a) * fa);
    }
}

}  // namespace qd
}  // namespace moe
