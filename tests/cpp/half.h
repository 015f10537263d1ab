// IEEE binary16 <-> binary32 on the host for the C++ tests, round to nearest
// even (gcc 11 has no _Float16 on x86).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

inline std::uint16_t to_half(float f)
{
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    const std::uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (std::uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (std::uint16_t)(sign | 0x7c00u);  // rounds past 65504
    if (ax < 0x38800000u) {                                          // half subnormal range
        float af;
        std::memcpy(&af, &ax, 4);
        return (std::uint16_t)(sign | (std::uint32_t)std::nearbyint(af * 16777216.0f));
    }
    std::uint32_t h = ((((ax >> 23) - 127 + 15) << 10) | ((ax & 0x7fffffu) >> 13));
    const std::uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (std::uint16_t)(sign | h);
}

inline float from_half(std::uint16_t h)
{
    const std::uint32_t sign = (std::uint32_t)(h & 0x8000u) << 16;
    const std::uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        const float v = std::ldexp((float)m, -24);
        return sign ? -v : v;
    }
    const std::uint32_t bits = sign | (e == 31 ? (0x7f800000u | (m << 13)) : (((e - 15 + 127) << 23) | (m << 13)));
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
