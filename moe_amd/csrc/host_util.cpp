// host_util.cpp — host-side formats and seeded synthetic data.
//
// Block formats and the quantiser restate src/quant.rs:68-83, 131-227 and
// 304-365 (the reference's own quantiser, which differs from ggml's: Q4 uses
// d = amax/7, Q5 amax/15, Q8 amax/127, and the reciprocal of the f16-rounded
// scale).  The generator has no reference counterpart: splitmix64 uniforms,
// Box-Muller in double, one rounding to float.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/moe_hip.h"

namespace moe {
int fail(int code, const char *fmt, ...);
}
using moe::fail;

namespace {

inline uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float float_of(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// IEEE half -> float, subnormals renormalised (src/quant.rs:131-147).
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return float_of(sign | 0x7f800000u | (m << 13));
    if (e != 0) return float_of(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return float_of(sign);
    int shift = 0;
    uint32_t mm = m;
    while (!(mm & 0x400u)) mm <<= 1, shift++;
    return float_of(sign | ((uint32_t)(113 - shift) << 23) | ((mm & 0x3ffu) << 13));
}

// float -> half as the reference rounds it (src/quant.rs:149-174): nearest
// even for normals, round-half-up for subnormals, everything too large
// (NaN included) to infinity.
uint16_t float_to_half(float f) {
    const uint32_t x = bits_of(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int e = (int)((x >> 23) & 0xffu) - 112;
    const uint32_t m = x & 0x7fffffu;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t full = (m | 0x800000u) >> (1 - e);
        return sign | (uint16_t)((full + 0x1000u) >> 13);
    }
    const uint32_t r = m + 0x0fffu + ((m >> 13) & 1u);
    if (r & 0x800000u) {
        if (++e >= 31) return sign | 0x7c00u;
    }
    return sign | (uint16_t)(e << 10) | (uint16_t)((r & 0x7fffffu) >> 13);
}

// Rust `f32 as i32` after round(): saturating, NaN -> 0.
inline int32_t to_i32(float v) {
    if (std::isnan(v)) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v < -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
inline float max_num(float a, float b) { return std::isnan(a) ? b : (std::isnan(b) ? a : (a > b ? a : b)); }

struct BlockScale {
    uint16_t half;
    float inv;
};
inline BlockScale scale_for(const float *v, float levels) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = max_num(amax, std::fabs(v[i]));
    const float d = amax / levels;
    BlockScale s;
    s.half = float_to_half(d);
    s.inv = d > 0.0f ? 1.0f / half_to_float(s.half) : 0.0f;
    return s;
}
inline void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
inline uint8_t level(float v, float inv, int32_t off, int32_t top) {
    int32_t q = to_i32(std::round(v * inv)) + off;
    return (uint8_t)(q < 0 ? 0 : (q > top ? top : q));
}

void quantize_row(int dt, const float *s, uint64_t cols, uint8_t *dst) {
    switch (dt) {
    case MOE_DT_F32: std::memcpy(dst, s, cols * 4); return;
    case MOE_DT_F16:
        for (uint64_t i = 0; i < cols; i++) put16(dst + 2 * i, float_to_half(s[i]));
        return;
    case MOE_DT_Q8_0:
        for (uint64_t b = 0; b < cols / 32; b++, s += 32, dst += 34) {
            BlockScale sc = scale_for(s, 127.0f);
            put16(dst, sc.half);
            for (int i = 0; i < 32; i++) {
                float q = std::round(s[i] * sc.inv);
                q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
                dst[2 + i] = (uint8_t)(int8_t)to_i32(q);
            }
        }
        return;
    case MOE_DT_Q4_0:
        for (uint64_t b = 0; b < cols / 32; b++, s += 32, dst += 18) {
            BlockScale sc = scale_for(s, 7.0f);
            put16(dst, sc.half);
            for (int i = 0; i < 16; i++)
                dst[2 + i] = (uint8_t)(level(s[i], sc.inv, 8, 15) | (level(s[16 + i], sc.inv, 8, 15) << 4));
        }
        return;
    case MOE_DT_Q5_0:
        for (uint64_t b = 0; b < cols / 32; b++, s += 32, dst += 22) {
            BlockScale sc = scale_for(s, 15.0f);
            put16(dst, sc.half);
            uint32_t high = 0;
            for (int i = 0; i < 16; i++) {
                const uint8_t lo = level(s[i], sc.inv, 16, 31), hi = level(s[16 + i], sc.inv, 16, 31);
                dst[6 + i] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
                high |= (uint32_t)(lo >> 4) << i;
                high |= (uint32_t)(hi >> 4) << (16 + i);
            }
            std::memcpy(dst + 2, &high, 4);  // little-endian bit plane
        }
        return;
    }
}

void dequant_row(int dt, const uint8_t *src, uint64_t cols, float *out) {
    auto rd16 = [](const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); };
    switch (dt) {
    case MOE_DT_F32: std::memcpy(out, src, cols * 4); return;
    case MOE_DT_F16:
        for (uint64_t i = 0; i < cols; i++) out[i] = half_to_float(rd16(src + 2 * i));
        return;
    case MOE_DT_BF16:
        for (uint64_t i = 0; i < cols; i++) out[i] = float_of((uint32_t)rd16(src + 2 * i) << 16);
        return;
    case MOE_DT_Q8_0:
        for (uint64_t b = 0; b < cols / 32; b++, src += 34, out += 32) {
            const float d = half_to_float(rd16(src));
            for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)src[2 + i];
        }
        return;
    case MOE_DT_Q4_0:
        for (uint64_t b = 0; b < cols / 32; b++, src += 18, out += 32) {
            const float d = half_to_float(rd16(src));
            for (int i = 0; i < 16; i++) {
                out[i] = d * (float)((int)(src[2 + i] & 15) - 8);
                out[16 + i] = d * (float)((int)(src[2 + i] >> 4) - 8);
            }
        }
        return;
    case MOE_DT_Q5_0:
        for (uint64_t b = 0; b < cols / 32; b++, src += 22, out += 32) {
            const float d = half_to_float(rd16(src));
            uint32_t high;
            std::memcpy(&high, src + 2, 4);
            for (int i = 0; i < 16; i++) {
                out[i] = d * (float)((int)((src[6 + i] & 15) | (((high >> i) & 1) << 4)) - 16);
                out[16 + i] = d * (float)((int)((src[6 + i] >> 4) | (((high >> (16 + i)) & 1) << 4)) - 16);
            }
        }
        return;
    }
}

bool fits(int dt, uint64_t cols) {
    switch (dt) {
    case MOE_DT_F32:
    case MOE_DT_F16:
    case MOE_DT_BF16: return true;
    case MOE_DT_Q8_0:
    case MOE_DT_Q4_0:
    case MOE_DT_Q5_0: return cols % 32 == 0;
    default: return false;
    }
}

// ------------------------------------------------------------- generator

constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
// splitmix64 state for (seed, stream); output i is mix64(key + (i+1) * gamma).
inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(seed) ^ mix64(stream * kGamma + 1); }
inline double uniform(uint64_t key, uint64_t i) { return (double)(mix64(key + (i + 1) * kGamma) >> 11) * 0x1.0p-53; }

// Elements [i0, i0 + n) of the stream: element 2j and 2j+1 are the cosine
// and sine halves of Box-Muller pair j over uniforms 2j (as 1 - u, in (0,1])
// and 2j+1.
void normals(uint64_t key, uint64_t i0, uint64_t n, double mean, double std, float *out) {
    uint64_t i = i0;
    const uint64_t end = i0 + n;
    while (i < end) {
        const uint64_t j = i >> 1;
        const double u1 = 1.0 - uniform(key, 2 * j), u2 = uniform(key, 2 * j + 1);
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 6.283185307179586 * u2;
        if ((i & 1) == 0) {
            out[i - i0] = (float)(mean + std * (r * std::cos(a)));
            if (i + 1 < end) out[i + 1 - i0] = (float)(mean + std * (r * std::sin(a)));
            i += 2;
        } else {
            out[i - i0] = (float)(mean + std * (r * std::sin(a)));
            i += 1;
        }
    }
}

template <class F>
void parallel_for(uint64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 64) nt = 64;
    if (n < 2 * nt) nt = 1;
    if (nt == 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> th;
    const uint64_t chunk = (n + nt - 1) / nt;
    for (unsigned w = 0; w < nt; w++) {
        const uint64_t a = w * chunk, b = std::min<uint64_t>(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([=, &f] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

}  // namespace

extern "C" {

uint64_t moe_row_bytes(int32_t dt, uint64_t cols) {
    // Saturating, like the container reader: a row too wide for 64 bits of
    // bytes reports UINT64_MAX rather than a wrapped small size.
    uint64_t r;
    switch (dt) {
    case MOE_DT_F32: return __builtin_mul_overflow(cols, (uint64_t)4, &r) ? UINT64_MAX : r;
    case MOE_DT_F16:
    case MOE_DT_BF16: return __builtin_mul_overflow(cols, (uint64_t)2, &r) ? UINT64_MAX : r;
    case MOE_DT_Q8_0: return cols / 32 * 34;
    case MOE_DT_Q4_0: return cols / 32 * 18;
    case MOE_DT_Q5_0: return cols / 32 * 22;
    default: return 0;
    }
}

int moe_rope_inv_freqs(int32_t kind, float theta, float factor, uint64_t original_ctx, float low_freq_factor,
                       float high_freq_factor, float beta_fast, float beta_slow, int32_t head_dim, float *out) {
    if (!out || head_dim < 2 || kind < 0 || kind > 4) return fail(MOE_EINVAL, "moe_rope_inv_freqs: bad argument");
    // Rope::inv_freqs (src/spec.rs:89-145) in f32 with libm's powf, logf:
    // the same operations in the same order, so the table is the engine's.
    const int half = head_dim / 2;
    const float dim = (float)head_dim;
    const float s = factor > 1e-6f ? factor : 1e-6f;
    float th = theta;
    if (kind == 2) th = theta * std::pow(s, dim / std::max(dim - 2.0f, 1.0f));
    for (int i = 0; i < half; i++) out[i] = std::pow(th, -2.0f * (float)i / dim);
    const float pi = 3.14159265358979323846f;
    if (kind == 1) {
        for (int i = 0; i < half; i++) out[i] = out[i] / s;
    } else if (kind == 4) {
        const float l = (float)original_ctx;
        const float lo_wave = l / low_freq_factor, hi_wave = l / high_freq_factor;
        const float span = std::max(high_freq_factor - low_freq_factor, 1e-6f);
        for (int i = 0; i < half; i++) {
            const float f = out[i], wave = 2.0f * pi / f;
            if (wave > lo_wave) {
                out[i] = f / s;
            } else if (wave >= hi_wave) {
                const float t = ((l / wave) - low_freq_factor) / span;
                out[i] = (1.0f - t) * f / s + t * f;
            }
        }
    } else if (kind == 3) {
        const float l = (float)original_ctx;
        const float ln_base = std::max(std::log(theta), 1e-6f);
        auto bound = [&](float beta) { return dim * std::log(l / (beta * 2.0f * pi)) / (2.0f * ln_base); };
        const float low = std::floor(bound(beta_fast)), high = std::ceil(bound(beta_slow));
        const float span = std::max(high - low, 1e-3f);
        for (int i = 0; i < half; i++) {
            const float f = out[i];
            const float ramp = std::min(std::max(((float)i - low) / span, 0.0f), 1.0f);
            out[i] = (1.0f - ramp) * (f / s) + ramp * f;
        }
    }
    return MOE_OK;
}

int moe_quantize_rows(int32_t dt, const float *src, uint64_t rows, uint64_t cols, uint8_t *dst) {
    if (!src || !dst || dt == MOE_DT_BF16 || !fits(dt, cols) || moe_row_bytes(dt, cols) == 0) return MOE_EINVAL;
    const uint64_t rb = moe_row_bytes(dt, cols);
    parallel_for(rows, [&](uint64_t a, uint64_t b) {
        for (uint64_t r = a; r < b; r++) quantize_row(dt, src + r * cols, cols, dst + r * rb);
    });
    return MOE_OK;
}

int moe_dequant_rows(int32_t dt, const uint8_t *src, uint64_t rows, uint64_t cols, float *dst) {
    if (!src || !dst || !fits(dt, cols) || moe_row_bytes(dt, cols) == 0) return MOE_EINVAL;
    const uint64_t rb = moe_row_bytes(dt, cols);
    parallel_for(rows, [&](uint64_t a, uint64_t b) {
        for (uint64_t r = a; r < b; r++) dequant_row(dt, src + r * rb, cols, dst + r * cols);
    });
    return MOE_OK;
}

int moe_synth_normal(uint64_t seed, uint64_t stream, uint64_t n, double mean, double std, float *out) {
    if (!out && n) return MOE_EINVAL;
    const uint64_t key = stream_key(seed, stream);
    const uint64_t blocks = (n + 4095) / 4096;
    parallel_for(blocks, [&](uint64_t a, uint64_t b) {
        for (uint64_t q = a; q < b; q++) {
            const uint64_t i0 = q * 4096, m = std::min<uint64_t>(4096, n - i0);
            normals(key, i0, m, mean, std, out + i0);
        }
    });
    return MOE_OK;
}

int moe_synth_quantized(uint64_t seed, uint64_t stream, int32_t dt, uint64_t rows, uint64_t cols, double mean,
                        double std, uint8_t *dst) {
    if (!dst || dt == MOE_DT_BF16 || !fits(dt, cols) || moe_row_bytes(dt, cols) == 0) return MOE_EINVAL;
    const uint64_t key = stream_key(seed, stream), rb = moe_row_bytes(dt, cols);
    parallel_for(rows, [&](uint64_t a, uint64_t b) {
        std::vector<float> buf(cols);
        for (uint64_t r = a; r < b; r++) {
            normals(key, r * cols, cols, mean, std, buf.data());
            quantize_row(dt, buf.data(), cols, dst + r * rb);
        }
    });
    return MOE_OK;
}

}  // extern "C"
