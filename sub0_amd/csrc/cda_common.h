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

// Forces a lambda (or function) inline: kernels here keep MFMA operands and
// accumulators in registers, which an out-of-line call would spill.
#define CDA_INLINE __attribute__((always_inline))

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// float64 -> fp16, round to nearest even, in a few instructions: round to
// fp32 *to odd* (truncate toward zero, then set the last bit when inexact),
// then fp32 -> fp16 to nearest even.  fp32 keeps 13 bits more than fp16, so
// the odd intermediate never creates or hides a tie and the result equals
// the correctly rounded fp16 of the float64 value (also for fp16 subnormals,
// overflow to infinity and NaN).
__device__ __forceinline__ uint16_t f64_to_f16_rn(double v) {
    float f = (float)v;                          // nearest even
    const double back = (double)f;
    if (back != v && v == v) {
        uint32_t fb = __float_as_uint(f);
        if (fabs(back) > fabs(v)) fb -= 1;       // one ulp toward zero
        f = __uint_as_float(fb | 1u);
    }
    return __half_as_ushort(__float2half_rn(f));
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
