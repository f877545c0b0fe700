// Test infrastructure (see hip_runtime.h in this directory): fp16 storage type and round-to-
// nearest-even conversions for the host emulation of the persistent step kernel.
#pragma once
#include <cstdint>
#include <cstring>
#include <cmath>
#include <hip/hip_runtime.h>
struct __half { uint16_t x; };
struct __half2 { __half a, b; };
inline float __emu_h2f(uint16_t h) {
    const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 1024), (int)e - 25);
    return s ? -v : v;
}
inline uint16_t __emu_f2h(float f) {  // round to nearest even
    uint32_t x; std::memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
    if (x >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);  // rounds to >= 65520 -> inf
    float a; std::memcpy(&a, &x, 4);
    if (a < 6.103515625e-05f) {  // subnormal: multiples of 2^-24
        const float q = std::nearbyint(a * 16777216.0f);
        return (uint16_t)(s | (uint16_t)q);
    }
    int e; const float fr = std::frexp(a, &e);  // a = fr * 2^e, fr in [0.5, 1)
    float mant = std::nearbyint(fr * 2048.0f);   // 11 bits
    if (mant == 2048.0f) { mant = 1024.0f; e += 1; }
    const int he = e - 1 + 15;
    return (uint16_t)(s | (uint16_t)(he << 10) | ((uint16_t)mant & 1023));
}
inline float __half2float(__half h) { return __emu_h2f(h.x); }
inline __half __ushort_as_half(uint16_t b) { return __half{b}; }
inline uint16_t __half_as_ushort(__half h) { return h.x; }
inline __half __float2half_rn(float f) { return __half{__emu_f2h(f)}; }
inline __half __float2half(float f) { return __float2half_rn(f); }
inline float2 __half22float2(__half2 h) { return {__half2float(h.a), __half2float(h.b)}; }
