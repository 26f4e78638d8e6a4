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
// fp16(RN32(v)): the fp32 value is materialised first (an empty asm makes it
// opaque), so the compiler cannot fuse the operation that produced it with
// the conversion into one rounding (v_fma_mixlo_f16).  The reference rounds
// twice: its fp32 arithmetic, then .to(torch.float16).
__device__ __forceinline__ uint16_t f2h_after_f32(float v) {
    asm volatile("" : "+v"(v));
    return __half_as_ushort(__float2half_rn(v));
}

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
    const float f = (float)v;                    // nearest even
    const double back = (double)f;
    // Branch-free: an exact conversion changes nothing; an inexact one steps
    // one ulp toward zero if it went past v and sets the sticky last bit.
    uint32_t fb = __float_as_uint(f) - (fabs(back) > fabs(v) ? 1u : 0u);
    fb |= (back != v && v == v) ? 1u : 0u;
    return __half_as_ushort(__float2half_rn(__uint_as_float(fb)));
}

// Correctly rounded fp32 square root of a float64 value, independent of the
// hardware sqrt accuracy beyond a few float64 ulps: f = fp32(sqrt(x)) is then
// within one fp32 ulp of the answer, and one branch-free step against the
// exact fp32 rounding midpoints (25-bit values, whose squares are exact in
// float64) moves it there (ties to even).  Same result as the CPU checker's
// iteration.
__device__ __forceinline__ float sqrt_f64_to_f32_rn(double x) {
    const float f = (float)sqrt(x);
    const int fi = __float_as_int(f);
    const float up = __int_as_float(fi + 1), dn = __int_as_float(fi - 1);
    const double mu = ((double)f + (double)up) * 0.5, md = ((double)f + (double)dn) * 0.5;
    const double mmu = mu * mu, mmd = md * md;
    const bool odd = (fi & 1) != 0;
    const bool go_up = mmu < x || (mmu == x && odd);
    const bool go_dn = mmd > x || (mmd == x && odd);
    const float r = go_up ? up : (go_dn ? dn : f);
    if (!(x > 0.0)) return (x == 0.0) ? 0.0f : __int_as_float(0x7FC00000);
    return (x == __longlong_as_double(0x7FF0000000000000ll)) ? __int_as_float(0x7F800000) : r;
}

}  // namespace cda
