// Shared helpers of the CDA HIP kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <string>

#include "../../include/cda_hip.h"

namespace cda {

constexpr int kD = 128;

// Per-thread last error message (returned by cda_hip_last_error()).
void set_error(const std::string &msg);

inline int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

#define CDA_REQUIRE(cond, msg)                                               \
    do {                                                                     \
        if (!(cond)) return ::cda::fail(CDA_E_INVALID, std::string(msg));    \
    } while (0)

#define CDA_LAUNCH_CHECK(what)                                               \
    do {                                                                     \
        hipError_t e__ = hipGetLastError();                                  \
        if (e__ != hipSuccess)                                               \
            return ::cda::fail(CDA_E_HIP, std::string(what) + ": " +         \
                                              hipGetErrorString(e__));       \
    } while (0)

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// ---------------------------------------------------------------- device --

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// Correctly rounded (nearest-even) float64 -> float16 bits.  The same integer
// procedure as cda_oracle_f64_to_f16 in the CPU checker, so both sides agree
// on every input.
__device__ __forceinline__ uint16_t f64_to_f16_rn(double v) {
    uint64_t b = (uint64_t)__double_as_longlong(v);
    uint32_t sign = (uint32_t)((b >> 48) & 0x8000u);
    int e = (int)((b >> 52) & 0x7FF);
    uint64_t m = b & 0xFFFFFFFFFFFFFull;
    if (e == 0x7FF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    if (e == 0) return (uint16_t)sign;
    int ue = e - 1023;
    if (ue > 15) return (uint16_t)(sign | 0x7C00u);
    uint64_t sig = m | (1ull << 52);
    int shift;
    uint32_t hexp;
    if (ue >= -14) {
        shift = 42;
        hexp = (uint32_t)(ue + 15);
    } else {
        shift = 42 + (-14 - ue);
        hexp = 0;
        if (shift > 63) return (uint16_t)sign;
    }
    uint64_t kept = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (kept & 1))) kept++;
    uint32_t out;
    if (hexp) {
        if (kept == (1ull << 11)) {
            kept >>= 1;
            hexp++;
        }
        if (hexp >= 31) return (uint16_t)(sign | 0x7C00u);
        out = (hexp << 10) | (uint32_t)(kept & 0x3FFu);
    } else {
        out = (uint32_t)kept;
    }
    return (uint16_t)(sign | out);
}

// Correctly rounded fp32 square root of a float64 value, independent of the
// hardware sqrt accuracy: start from an approximation and move it until the
// exact fp32 rounding midpoints (25-bit values, whose squares are exact in
// float64) bracket x.  Same procedure as the CPU checker.
__device__ __forceinline__ float sqrt_f64_to_f32_rn(double x) {
    if (!(x > 0.0)) return (x == 0.0) ? 0.0f : __int_as_float(0x7FC00000);
    if (x == __longlong_as_double(0x7FF0000000000000ll)) return __int_as_float(0x7F800000);
    float f = (float)sqrt(x);
    for (int it = 0; it < 4; ++it) {
        float up = __int_as_float(__float_as_int(f) + 1);
        double mid = ((double)f + (double)up) * 0.5;
        double mm = mid * mid;
        if (mm < x || (mm == x && (__float_as_int(f) & 1))) {
            f = up;
            continue;
        }
        float dn = __int_as_float(__float_as_int(f) - 1);
        double midl = ((double)f + (double)dn) * 0.5;
        double ml = midl * midl;
        if (ml > x || (ml == x && (__float_as_int(f) & 1))) {
            f = dn;
            continue;
        }
        break;
    }
    return f;
}

}  // namespace cda
