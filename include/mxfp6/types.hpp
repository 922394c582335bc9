#pragma once
// MXFP6 element formats, host side (header-only).
//
// Same functions and semantics as the reference's include/mxfp6/types.hpp (eeezio/mxfp6-gemm):
//   * FP6 E2M3: 1 sign, 2 exponent (bias 1), 3 mantissa bits; no Inf/NaN; |x| <= 7.5;
//     subnormals 0.125 * m. Encoding rounds to the nearest representable value, ties to an
//     even mantissa, saturating at 7.5 (types.hpp:26-72).
//   * E8M0: value 2^(u - 127), code 255 is NaN (types.hpp:74-95).
//   * Dense packing: four 6-bit codes in three bytes, code i in bits [6i, 6i+6) of the
//     little-endian 24-bit group (types.hpp:97-123).
#include <cassert>
#include <cmath>
#include <cstdint>

namespace mxfp6 {

// ---- FP6 E2M3 ----------------------------------------------------------------------------

inline float fp6_e2m3_to_float(uint8_t bits6) {
    const int mant = bits6 & 7;
    const int expo = (bits6 >> 3) & 3;
    // subnormal binade (expo 0): m/8; normal: (8+m)/8 * 2^(expo-1) == (8+m) * 2^(expo-4)
    const float mag = expo == 0 ? (float)mant * 0.125f : std::ldexp((float)(8 + mant), expo - 4);
    return (bits6 & 0x20) ? -mag : mag;
}

// Nearest E2M3 code of v. Magnitudes above 7.5 saturate. The sign bit is set for any v < 0
// (so small negatives give the negative-zero code 0x20); -0.0f encodes as 0x00.
inline uint8_t float_to_fp6_e2m3(float v) {
    const uint8_t sign = v < 0.0f ? 0x20 : 0x00;
    float a = std::fabs(v);
    if (!(a > 0.0f)) return sign;  // zero (NaN is outside the contract: encodes as +-0)
    if (a > 7.5f) a = 7.5f;
    // Binade index b: [0,1) -> 0 (subnormal, step 1/8), [1,2) -> 1, [2,4) -> 2, [4,7.5] -> 3.
    const int b = a < 1.0f ? 0 : a < 2.0f ? 1 : a < 4.0f ? 2 : 3;
    // Offset into the binade in units of the binade's step; exact (power-of-two scaling).
    const float steps = b == 0 ? a * 8.0f : (std::ldexp(a, 1 - b) - 1.0f) * 8.0f;
    const int m = (int)std::nearbyint(steps);  // default rounding mode: ties to even
    // m == 8 carries into the next binade: code (b<<3) + 8 == ((b+1)<<3) + 0.
    int code = (b << 3) + m;
    if (code > 31) code = 31;
    return (uint8_t)(sign | code);
}

// ---- E8M0 ---------------------------------------------------------------------------------

inline float e8m0_to_float(uint8_t code) {
    if (code == 0xFF) return NAN;
    return std::ldexp(1.0f, (int)code - 127);
}

// Power of two nearest to v in the log domain (threshold sqrt(2) on the normalised
// significand), clamped to codes [0, 254]. NaN -> 255, v <= 0 -> 0.
inline uint8_t float_to_e8m0(float v) {
    if (std::isnan(v)) return 0xFF;
    if (v <= 0.0f) return 0;
    int e2;
    const float sig = std::frexp(v, &e2) * 2.0f;  // v = sig * 2^(e2-1), sig in [1, 2)
    int e = e2 - 1 + (sig >= 1.41421356f ? 1 : 0);
    int code = e + 127;
    code = code < 0 ? 0 : code > 254 ? 254 : code;
    return (uint8_t)code;
}

// ---- dense FP6 packing ----------------------------------------------------------------------

inline void pack_fp6x4(const uint8_t* in, uint8_t* out) {
    const uint32_t w = (uint32_t)(in[0] & 0x3F) | ((uint32_t)(in[1] & 0x3F) << 6) |
                       ((uint32_t)(in[2] & 0x3F) << 12) | ((uint32_t)(in[3] & 0x3F) << 18);
    out[0] = (uint8_t)w;
    out[1] = (uint8_t)(w >> 8);
    out[2] = (uint8_t)(w >> 16);
}

inline void unpack_fp6x4(const uint8_t* in, uint8_t* out) {
    const uint32_t w = (uint32_t)in[0] | ((uint32_t)in[1] << 8) | ((uint32_t)in[2] << 16);
    for (int i = 0; i < 4; i++) out[i] = (uint8_t)((w >> (6 * i)) & 0x3F);
}

inline void pack_fp6(const uint8_t* vals, int n, uint8_t* packed) {
    assert(n % 4 == 0);
    for (int g = 0; g < n / 4; g++) pack_fp6x4(vals + 4 * g, packed + 3 * g);
}

inline void unpack_fp6(const uint8_t* packed, int n, uint8_t* vals) {
    assert(n % 4 == 0);
    for (int g = 0; g < n / 4; g++) unpack_fp6x4(packed + 3 * g, vals + 4 * g);
}

inline int fp6_packed_bytes(int n) {
    assert(n % 4 == 0);
    return n / 4 * 3;
}

}  // namespace mxfp6
