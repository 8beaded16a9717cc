// exact_math.h — host/device restatement of glibc's expf (glibc 2.35,
// sysdeps/ieee754/flt-32/e_expf.c, the ARM optimized-routines algorithm),
// bit-identical to the x86-64 FMA build that Rust's f32::exp calls on
// linux-gnu (the reference computes its gates with it, src/model.rs:224 and
// :858).  Algorithm: x*N/ln2 = k + r with N = 32, 2^(k/N) from a 32-entry
// table of 2^(i/32) (stored minus i<<47 so the exponent add is one integer
// add), 2^(r/N) from a cubic, all in double, one rounding to float at the
// end.  The x86-64 FMA build fuses the range-reduction multiply into both the
// shift-add and the remainder; that fusion is written out explicitly here and
// is what makes the result match glibc on all 2^32 inputs (the unfused form
// differs on two).  The table entries are 2^(i/32) rounded to nearest double,
// computed from exact decimal arithmetic.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define MOE_HD __host__ __device__
#else
#define MOE_HD
#endif

namespace moe {

#define MOE_EXP2_TAB                                                                           \
    {                                                                                          \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull \
    }
#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t kExp2TabDev[32] = MOE_EXP2_TAB;
#endif
static const uint64_t kExp2TabHost[32] = MOE_EXP2_TAB;


MOE_HD inline uint32_t f2u(float f) {
    union { float f; uint32_t u; } c;
    c.f = f;
    return c.u;
}
MOE_HD inline float u2f(uint32_t u) {
    union { float f; uint32_t u; } c;
    c.u = u;
    return c.f;
}
MOE_HD inline uint64_t d2u(double f) {
    union { double f; uint64_t u; } c;
    c.f = f;
    return c.u;
}
MOE_HD inline double u2d(uint64_t u) {
    union { double f; uint64_t u; } c;
    c.u = u;
    return c.f;
}

// Double-precision fused multiply-add, spelled so that neither the host nor
// the device compiler is free to split it.
MOE_HD inline double fma_d(double a, double b, double c) { return __builtin_fma(a, b, c); }

MOE_HD inline float expf_exact(float x) {
    const double kShift = 0x1.8p+52;
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux = f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;                 // -inf
        if (abstop >= 0x7f8) return x + x;                  // nan or +inf
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);     // overflow -> +inf
        if (x < -0x1.9fe368p6f) return 0.0f;                // underflow -> +0
    }
    double xd = (double)x;
    double kd = fma_d(kInvLn2N, xd, kShift);
    uint64_t ki = d2u(kd);
    kd -= kShift;
    double r = fma_d(kInvLn2N, xd, -kd);
#if defined(__HIP_DEVICE_COMPILE__)
    uint64_t t = kExp2TabDev[ki % 32];
#else
    uint64_t t = kExp2TabHost[ki % 32];
#endif
    t += ki << 47;
    double s = u2d(t);
    double z = fma_d(kC0, r, kC1);
    double r2 = r * r;
    double y = fma_d(kC2, r, 1.0);
    y = fma_d(z, r2, y);
    y = y * s;
    return (float)y;
}

#if defined(__HIPCC__)
// expf_exact with its table spread over a wavefront: lane l holds entry
// l % 32 (exp2_lane_entry, loaded once), and each lane fetches the entry it
// needs from that lane instead of from memory.  Every lane of the wavefront
// must call it together.
__device__ inline uint64_t exp2_lane_entry() { return kExp2TabDev[threadIdx.x & 31]; }

__device__ inline float expf_exact_w(float x, uint64_t lane_entry) {
    const double kShift = 0x1.8p+52;
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = (double)x;
    double kd = fma_d(kInvLn2N, xd, kShift);
    uint64_t ki = d2u(kd);
    const int src = (int)(ki % 32);
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)lane_entry, src, 64);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(lane_entry >> 32), src, 64);
    uint32_t ux = f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;                 // -inf
        if (abstop >= 0x7f8) return x + x;                  // nan or +inf
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);     // overflow -> +inf
        if (x < -0x1.9fe368p6f) return 0.0f;                // underflow -> +0
    }
    kd -= kShift;
    double r = fma_d(kInvLn2N, xd, -kd);
    uint64_t t = ((uint64_t)hi << 32) | lo;
    t += ki << 47;
    double s = u2d(t);
    double z = fma_d(kC0, r, kC1);
    double r2 = r * r;
    double y = fma_d(kC2, r, 1.0);
    y = fma_d(z, r2, y);
    y = y * s;
    return (float)y;
}
#endif

}  // namespace moe
